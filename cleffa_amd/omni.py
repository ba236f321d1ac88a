"""Omni decoder attention (hd 128, FP32 operands, FP64-accumulated output) through the C ABI:
the host side of clef_omni_encode_attention (clef_metal_omni.m:200-245) between the QKV GEMM
and o_proj. torch provides device memory and the stream; the compute is libclef_hip_attn.so."""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import OmniAttnArgs, OmniPrepArgs
from .attention import _device, _err, _i32p, _ptr, _stream_handle

HD = 128
BLOCK_Q = 16
SLACK = 32


def omni_rope_table(theta=1e6):
    """[192] f32: the f32 inverse frequencies, then the FP64 frequencies as hi / lo pairs."""
    t = np.zeros(192, np.float32)
    _lib.load().clef_hip_omni_rope_table(float(theta), t.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return t


class OmniPlan:
    """16-row query blocks of packed records (cu_seqlens), longest key range first."""

    def __init__(self, cu_seqlens, device="cuda"):
        lib = _lib.load()
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        self.n_seq, self.T = len(cu) - 1, int(cu[-1])
        max_blk = lib.clef_hip_omni_plan_max_blocks(self.n_seq, self.T)
        blocks = np.zeros((max(max_blk, 1), 8), np.int32)
        n = ctypes.c_int(0)
        err = _err()
        _lib.check(lib.clef_hip_omni_plan(_i32p(cu), self.n_seq, _i32p(blocks), max_blk, ctypes.byref(n), err, len(err)), err)
        self.n_blk = n.value
        self.blocks_host = blocks[: self.n_blk].copy()
        self.device = _device(device)
        self.blocks = torch.from_numpy(blocks[: max(self.n_blk, 1)].copy()).to(self.device)

    def pairs(self):
        """(query, key) pairs the causal mask keeps."""
        b = self.blocks_host
        nq, q0 = b[:, 1].astype(np.int64), b[:, 2].astype(np.int64)
        return int((nq * q0 + nq * (nq + 1) // 2).sum())


class OmniAttention:
    def __init__(self, nh, nkv, theta=1e6, eps=1e-6, rope_exact=True, device="cuda"):
        self.nh, self.nkv, self.eps, self.rope_exact = nh, nkv, eps, rope_exact
        self.device = _device(device)
        self.scale = 1.0 / float(np.sqrt(HD))
        self.freq = torch.from_numpy(omni_rope_table(theta)).to(self.device)

    def planes(self, T):
        """Q [nh][T][128], K and V [nkv][T + 32][128] f32 scratch."""
        f = dict(dtype=torch.float32, device=self.device)
        return (torch.empty(self.nh, max(T, 1), HD, **f), torch.empty(self.nkv, T + SLACK, HD, **f),
                torch.empty(self.nkv, T + SLACK, HD, **f))

    def prep(self, qkv, q_norm, k_norm, pos3, planes=None, status=None, stream=None):
        T = qkv.shape[0]
        row = (self.nh + 2 * self.nkv) * HD
        if qkv.shape != (T, row) or qkv.dtype != torch.float32 or not qkv.is_contiguous():
            raise ValueError(f"qkv must be contiguous f32 [T][{row}]")
        if pos3.shape != (T, 3) or pos3.dtype != torch.int32:
            raise ValueError("pos3 must be int32 [T][3]")
        for w in (q_norm, k_norm):
            if w.shape != (HD,) or w.dtype != torch.float32:
                raise ValueError("norm weights must be f32 [128]")
        Q, K, V = self.planes(T) if planes is None else planes
        if status is None:
            status = torch.zeros(1, dtype=torch.int32, device=self.device)
        a = OmniPrepArgs()
        a.nh, a.nkv, a.T, a.kvT, a.eps, a.rope_exact = self.nh, self.nkv, T, K.shape[1], self.eps, int(self.rope_exact)
        a.qkv, a.q_norm, a.k_norm, a.pos3, a.freq = _ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(pos3), _ptr(self.freq)
        a.q_plane, a.k_plane, a.v_plane, a.status = _ptr(Q), _ptr(K), _ptr(V), _ptr(status)
        err = _err()
        _lib.check(_lib.load().clef_hip_omni_prep(ctypes.byref(a), _stream_handle(stream), err, len(err)), err)
        return Q, K, V, status

    def attention(self, Q, K, V, plan, out=None, stream=None):
        T = plan.T
        if out is None:
            out = torch.empty(T, self.nh * HD, dtype=torch.float32, device=self.device)
        if out.shape != (T, self.nh * HD) or out.dtype != torch.float32:
            raise ValueError("out must be f32 [T][nh*128]")
        if Q.shape[1] < T or K.shape[1] < T + SLACK or V.shape != K.shape:
            raise ValueError("planes do not fit the pass")
        a = OmniAttnArgs()
        a.nh, a.nkv, a.T, a.kvT, a.scale = self.nh, self.nkv, T, K.shape[1], self.scale
        a.q_plane, a.k_plane, a.v_plane, a.blocks, a.n_blk = _ptr(Q), _ptr(K), _ptr(V), _ptr(plan.blocks), plan.n_blk
        a.out = _ptr(out)
        err = _err()
        _lib.check(_lib.load().clef_hip_omni_attention(ctypes.byref(a), _stream_handle(stream), err, len(err)), err)
        return out

    def forward(self, qkv, q_norm, k_norm, pos3, plan, out=None, stream=None):
        """Returns (out [T][nh*128] f32, status [1] int32: 2 when a value was not finite)."""
        Q, K, V, status = self.prep(qkv, q_norm, k_norm, pos3, stream=stream)
        return self.attention(Q, K, V, plan, out=out, stream=stream), status
