"""Host-side layer above the C ABI: plans, plane allocation and the attention calls.

This mirrors what cleffa's Metal backend does around its attention kernels:

* ``AttnPlan`` is the per-pass block list and kv-row map (clef_metal.m:1243-1257, built once per
  forward from seq_bounds; clef.c:470-497 packs the records);
* ``TextAttention.forward`` is one full-attention layer, the call that replaces
  ``encode_attention_tu`` (clef_metal.m:829-882) and the FP32 branch (clef_metal.m:1330-1413);
* ``VisionAttention.forward`` replaces the vision loop's vis_qkv_rope + vis_attention_mma/_mpp
  dispatches (clef_metal.m:1022-1049), here with all images packed in one launch via cu_seqlens.

torch provides device memory and the stream; every computation runs in libclef_hip_attn.so.
Shapes and dtypes are checked here, on the host, before any launch.
"""
import ctypes
import math

import numpy as np
import torch

from . import _lib
from ._lib import AttnArgs, VisArgs, OUT_BF16, OUT_F16, OUT_F32, BLOCK_INTS

_OUT_TYPES = {"bf16": (OUT_BF16, torch.bfloat16), "f16": (OUT_F16, torch.float16),
              "f32": (OUT_F32, torch.float32)}


def _i32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def _err():
    return ctypes.create_string_buffer(512)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_CUS = {}


def _device_cus(dev):
    """Compute units of a device (the persistent grid's workgroup count)."""
    if dev.index not in _CUS:
        _CUS[dev.index] = torch.cuda.get_device_properties(dev).multi_processor_count
    return _CUS[dev.index]


def _device(device):
    """torch.device with an explicit index for cuda ("cuda" -> "cuda:<current>")."""
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    return d


def _stream_handle(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


_initialised = set()


def init_device(device=None):
    """clef_hip_attn_init on the given (or current) device, once per device."""
    lib = _lib.load()
    dev = _device("cuda" if device is None else device)
    if dev.index in _initialised:
        return
    with torch.cuda.device(dev):
        err = _err()
        _lib.check(lib.clef_hip_attn_init(err, len(err)), err)
    _initialised.add(dev.index)


def rope_inv_freq(theta, n_rot):
    """f32 table 1/theta^(2j/n_rot), j < n_rot/2, computed by the library (clef_metal.m:176-192)."""
    lib = _lib.load()
    out = np.zeros(max(n_rot // 2, 1), dtype=np.float32)
    lib.clef_hip_rope_inv_freq(ctypes.c_float(theta), n_rot,
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out[: n_rot // 2]


def vision_positions(cu_seqlens, grid_w, merge=2):
    """[P][2] (grid row, grid column) of every patch, merge-window order (metal/clef.metal:1639-1641)."""
    lib = _lib.load()
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    gw = np.ascontiguousarray(grid_w, dtype=np.int32)
    n = len(cu) - 1
    if len(gw) != n:
        raise ValueError("grid_w needs one entry per image")
    pos2 = np.zeros((max(int(cu[-1]), 1), 2), dtype=np.int32)
    err = _err()
    _lib.check(lib.clef_hip_vis_positions(_i32p(cu), n, _i32p(gw), merge, _i32p(pos2), err, len(err)), err)
    return pos2[: int(cu[-1])]


class AttnPlan:
    """Query blocks and kv rows of one pass (host arrays plus their device copies).

    cu_q: record bounds over the pass rows (int32, cu_q[0] = 0).
    cu_k: None for a fresh pass; for a prefix-cache pass the records' kv-row bounds, each
          record's cached keys first and its new tokens last (cu_k[r] multiples of 8).
    """

    def __init__(self, cu_q, cu_k=None, causal=True, device="cuda"):
        lib = _lib.load()
        cu_q = np.ascontiguousarray(cu_q, dtype=np.int32)
        self.n_seq = len(cu_q) - 1
        self.T = int(cu_q[-1])
        self.cu_q = cu_q
        self.cu_k = None if cu_k is None else np.ascontiguousarray(cu_k, dtype=np.int32)
        if self.cu_k is not None and len(self.cu_k) != len(cu_q):
            raise ValueError("cu_seqlens_k must have as many entries as cu_seqlens_q")
        self.causal = bool(causal)
        max_blk = lib.clef_hip_attn_plan_max_blocks(self.n_seq, self.T)
        blocks = np.zeros((max(max_blk, 1), BLOCK_INTS), dtype=np.int32)
        tok_kv = np.zeros(max(self.T, 1), dtype=np.int32)
        # plane rows: a fresh pass starts each record at a multiple of 8 rows and reads whole 64-key
        # tiles from it; a prefix pass ends at cu_k[-1] + 64 (a bound: the plan reports kv_rows)
        max_kv = (self.T + 64 * self.n_seq if self.cu_k is None else int(self.cu_k[-1]) + 64) + 64
        kv_tok = np.zeros(max_kv, dtype=np.int32)
        n_blk, kv_rows = ctypes.c_int(0), ctypes.c_int(0)
        err = _err()
        ok = lib.clef_hip_attn_plan(_i32p(cu_q), None if self.cu_k is None else _i32p(self.cu_k),
                                    self.n_seq, int(self.causal), _i32p(blocks), max_blk,
                                    _i32p(tok_kv), self.T, _i32p(kv_tok), max_kv,
                                    ctypes.byref(n_blk), ctypes.byref(kv_rows), err, len(err))
        _lib.check(ok, err)
        self.n_blk = n_blk.value
        self.kv_rows = kv_rows.value
        self.blocks_host = blocks[: self.n_blk].copy()
        self.tok_kv_host = tok_kv[: self.T].copy()
        self.kv_tok_host = kv_tok[: self.kv_rows].copy()
        self.device = _device(device)
        self.blocks = torch.from_numpy(np.ascontiguousarray(blocks[: max(self.n_blk, 1)])).to(self.device)
        self.tok_kv = torch.from_numpy(np.ascontiguousarray(tok_kv)).to(self.device)
        self.kv_tok = torch.from_numpy(np.ascontiguousarray(kv_tok[: max(self.kv_rows, 1)])).to(self.device)
        # kv rows the planes must hold, rounded to the 16-byte V^T chunk
        self.kvT = max(8, (self.kv_rows + 7) // 8 * 8)
        # each pass row's record start (the reference's seq_start): where the K/V prologue flags
        # a key that leaves f16's range
        seq_start = np.repeat(cu_q[:-1], np.diff(cu_q)).astype(np.int32)
        self.seq_start = torch.from_numpy(np.ascontiguousarray(seq_start if self.T else np.zeros(1, np.int32))).to(self.device)

    def schedule(self, nh, nkv, n_wg):
        """Per-workgroup item lists of the attention core over n_wg workgroups (device int32,
        clef_hip_attn_schedule), built once per (nh, nkv, n_wg) and kept with the plan."""
        key = (nh, nkv, n_wg)
        cache = self.__dict__.setdefault("_sched", {})
        if key not in cache:
            lib = _lib.load()
            n = lib.clef_hip_attn_sched_size(self.n_blk, nh, n_wg)
            sched = np.zeros(max(n, 1), dtype=np.int32)
            blocks = np.ascontiguousarray(self.blocks_host, dtype=np.int32)
            err = _err()
            _lib.check(lib.clef_hip_attn_schedule(_i32p(blocks), self.n_blk, nh, nkv, n_wg,
                                                  _i32p(sched), len(sched), err, len(err)), err)
            cache[key] = torch.from_numpy(sched).to(self.device)
        return cache[key]

    def pairs(self):
        """(query, key) pairs the plan visits under its mask: the algorithmic work unit."""
        total = 0
        for r in range(self.n_seq):
            nq = int(self.cu_q[r + 1] - self.cu_q[r])
            nk = nq if self.cu_k is None else int(self.cu_k[r + 1] - self.cu_k[r])
            L = nk - nq
            total += nq * L + nq * (nq + 1) // 2 if self.causal else nq * nk
        return total


def _check(t, name, shape, dtype, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


class TextAttention:
    """One gated full-attention layer of the dense Clef models (hd 256, GQA)."""

    def __init__(self, nh, nkv, hd=256, n_rot=64, eps=1e-6, rope_theta=1e7, device="cuda"):
        self.nh, self.nkv, self.hd, self.n_rot, self.eps = nh, nkv, hd, n_rot, eps
        self.scale = 1.0 / math.sqrt(hd)
        self.row = 2 * nh * hd + 2 * nkv * hd
        self.device = _device(device)
        init_device(self.device)
        self.inv_freq = torch.from_numpy(rope_inv_freq(rope_theta, n_rot).copy()).to(self.device) \
            if n_rot else torch.zeros(1, dtype=torch.float32, device=self.device)

    def planes(self, kvT, fp32=False):
        """K plane [nkv][kvT][hd] (f16) and V^T plane [nkv][hd][kvT] (bf16); with fp32 (the
        FP32 mode, f32 qkv rows) K and V planes [nkv][kvT][hd], both f32."""
        if fp32:
            return (torch.empty((self.nkv, kvT, self.hd), dtype=torch.float32, device=self.device),
                    torch.empty((self.nkv, kvT, self.hd), dtype=torch.float32, device=self.device))
        k = torch.empty((self.nkv, kvT, self.hd), dtype=torch.float16, device=self.device)
        vt = torch.empty((self.nkv, self.hd, kvT), dtype=torch.bfloat16, device=self.device)
        return k, vt

    def rope_table(self, T):
        """[T][n_rot/2][2] f32 scratch for the rotary cos/sin of each pass row."""
        return torch.empty((max(T, 1), max(self.n_rot // 2, 1), 2), dtype=torch.float32, device=self.device)

    def args(self, qkv, q_norm, k_norm, pos3, plan, out, k_plane, vt_plane, kvT,
             out_type=OUT_BF16, gate=True, ovf=None, f16_lim=65504.0, rope_cs=None, trace=None,
             schedule=True):
        """The C argument block. qkv rows in bf16 select the tensor-unit path, f32 rows the FP32
        path (qkv_type CLEF_HIP_QKV_F32, with f32 K and V planes). schedule: hand the bf16 core a
        per-workgroup item split (clef_hip_attn_schedule) over the device's CUs (True) or over
        that many workgroups (an int), else (False) it falls back to its static order; the FP32
        core takes none."""
        T = plan.T
        dev = self.device
        fp32 = qkv.dtype == torch.float32
        _check(qkv, "qkv", (T, qkv.shape[1] if qkv.dim() == 2 else -1), torch.float32 if fp32 else torch.bfloat16, dev)
        if qkv.shape[1] < self.row or qkv.shape[1] % 8:
            raise ValueError(f"qkv row {qkv.shape[1]} must be >= {self.row} and a multiple of 8")
        if (q_norm is None) != (k_norm is None):
            raise ValueError("q_norm and k_norm must both be given or both be None")
        if q_norm is not None:
            _check(q_norm, "q_norm", (self.hd,), torch.float32, dev)
            _check(k_norm, "k_norm", (self.hd,), torch.float32, dev)
        if self.n_rot:
            _check(pos3, "pos3", (T, 3), torch.int32, dev)
        if fp32:
            _check(k_plane, "k_plane", (self.nkv, kvT, self.hd), torch.float32, dev)
            _check(vt_plane, "v_plane", (self.nkv, kvT, self.hd), torch.float32, dev)
        else:
            _check(k_plane, "k_plane", (self.nkv, kvT, self.hd), torch.float16, dev)
            _check(vt_plane, "vt_plane", (self.nkv, self.hd, kvT), torch.bfloat16, dev)
        if kvT < plan.kv_rows or kvT % 8:
            raise ValueError(f"kvT {kvT} must be >= {plan.kv_rows} and a multiple of 8")
        if out is not None:   # None: a call that writes no output (the prologue, the QKV GEMM)
            _check(out, "out", (T, self.nh * self.hd), {OUT_BF16: torch.bfloat16, OUT_F16: torch.float16,
                                                        OUT_F32: torch.float32}[out_type], dev)
        if ovf is not None:
            _check(ovf, "ovf", (T,), torch.int32, dev)
        if rope_cs is not None:
            _check(rope_cs, "rope_cs", (max(T, 1), max(self.n_rot // 2, 1), 2), torch.float32, dev)
        if plan.device != dev:
            raise ValueError("plan lives on another device")
        if plan.n_blk:
            b = plan.blocks_host
            if int((b[:, 0] + b[:, 1]).max()) > T or int((b[:, 3] + b[:, 4]).max()) > kvT:
                raise ValueError("plan does not fit the pass rows / planes")
        a = AttnArgs()
        a.nh, a.nkv, a.hd, a.n_rot = self.nh, self.nkv, self.hd, self.n_rot
        a.eps, a.scale = self.eps, self.scale
        a.T, a.row = T, qkv.shape[1]
        a.qkv, a.q_norm, a.k_norm = _ptr(qkv), _ptr(q_norm), _ptr(k_norm)
        a.pos3, a.inv_freq, a.rope_cs = _ptr(pos3), _ptr(self.inv_freq), _ptr(rope_cs)
        a.k_plane, a.vt_plane, a.kvT = _ptr(k_plane), _ptr(vt_plane), kvT
        a.blocks, a.n_blk = _ptr(plan.blocks), plan.n_blk
        a.kv_tok, a.kv_rows = _ptr(plan.kv_tok), plan.kv_rows
        a.causal, a.gate = int(plan.causal), int(gate)
        a.out, a.out_type, a.f16_lim, a.ovf = _ptr(out), out_type, f16_lim, _ptr(ovf)
        a.trace = _ptr(trace)
        a.seq_start, a.qkv_type = _ptr(plan.seq_start), _lib.QKV_F32 if fp32 else _lib.QKV_BF16
        a.tok_kv = _ptr(plan.tok_kv)
        if schedule and plan.n_blk and not fp32:
            # True: one workgroup per CU; an int: that many workgroups
            n_wg = _device_cus(dev) if schedule is True else int(schedule)
            if n_wg <= 0:
                raise ValueError(f"schedule: {n_wg} workgroups")
            a.sched, a.n_wg = _ptr(plan.schedule(self.nh, self.nkv, n_wg)), n_wg
        return a

    def forward(self, qkv, q_norm, k_norm, pos3, plan, out=None, out_dtype="bf16", gate=True,
                k_plane=None, vt_plane=None, kvT=None, ovf=None, f16_lim=65504.0, stream=None,
                stage="prefill", rope_cs=None, trace=None, schedule=True):
        """Runs one layer's attention. stage: "prefill" (prep_kv + core), "prep", or "core".
        rope_cs: the rotary cos/sin scratch (see rope_table); allocated here for "prefill" when
        not given. A "core" call with a table reads what the last "prep" call wrote."""
        lib = _lib.load()
        out_type, odt = _OUT_TYPES[out_dtype]
        if out is None:
            out = torch.empty((plan.T, self.nh * self.hd), dtype=odt, device=self.device)
        if k_plane is None:
            kvT = plan.kvT
            k_plane, vt_plane = self.planes(kvT, fp32=qkv.dtype == torch.float32)
        elif kvT is None:
            kvT = k_plane.shape[1]
        if rope_cs is None and stage == "prefill" and self.n_rot:
            rope_cs = self.rope_table(plan.T)
        a = self.args(qkv, q_norm, k_norm, pos3, plan, out, k_plane, vt_plane, kvT,
                      out_type=out_type, gate=gate, ovf=ovf, f16_lim=f16_lim, rope_cs=rope_cs,
                      trace=trace, schedule=schedule)
        fn = {"prefill": lib.clef_hip_attn_prefill, "prep": lib.clef_hip_attn_prep_kv,
              "core": lib.clef_hip_attn_core}[stage]
        err = _err()
        _lib.check(fn(ctypes.byref(a), _stream_handle(stream), err, len(err)), err)
        return out


    def project(self, X, W, plan, q_norm=None, k_norm=None, pos3=None, qkv=None, k_plane=None, vt_plane=None,
                kvT=None, ovf=None, f16_lim=65504.0, rope_cs=None, prologue=True, stream=None):
        """The QKV projection qkv = X . W^T (X [T][H] bf16, W [row][H] bf16, the attn_qkv weight as
        stored) through clef_hip_qkv_gemm. With prologue, its epilogue also writes the K / V^T
        planes (and rope_cs) as the "prep" stage would, so forward(stage="core") may follow on
        the same planes and table. Returns qkv."""
        dev = self.device
        T, H = plan.T, X.shape[1] if X.dim() == 2 else -1
        _check(X, "X", (T, H), torch.bfloat16, dev)
        _check(W, "W", (self.row, H), torch.bfloat16, dev)
        if qkv is None:
            qkv = torch.empty((T, self.row), dtype=torch.bfloat16, device=dev)
        _check(qkv, "qkv", (T, self.row), torch.bfloat16, dev)
        if prologue:
            if k_plane is None:
                kvT = plan.kvT
                k_plane, vt_plane = self.planes(kvT)
            elif kvT is None:
                kvT = k_plane.shape[1]
            a = self.args(qkv, q_norm, k_norm, pos3, plan, None, k_plane, vt_plane, kvT, ovf=ovf, f16_lim=f16_lim,
                          rope_cs=rope_cs, schedule=False)
        else:   # the product alone: only the geometry and the output rows
            a = AttnArgs()
            a.nh, a.nkv, a.hd, a.n_rot, a.T, a.row = self.nh, self.nkv, self.hd, self.n_rot, T, self.row
            a.qkv, a.qkv_type = _ptr(qkv), _lib.QKV_BF16
        err = _err()
        _lib.check(_lib.load().clef_hip_qkv_gemm(H, X.data_ptr(), W.data_ptr(), ctypes.byref(a),
                                                 _ptr(plan.tok_kv) if prologue else None,
                                                 _stream_handle(stream), err, len(err)), err)
        return qkv


class VisionAttention:
    """Vision tower attention: hd 72, MHA, bidirectional within each image, 2-D rotary."""


    def __init__(self, heads=16, hd=72, theta=10000.0, device="cuda"):
        self.heads, self.hd = heads, hd
        self.E = heads * hd
        self.scale = 1.0 / math.sqrt(hd)
        self.device = _device(device)
        init_device(self.device)
        self.inv_freq = torch.from_numpy(rope_inv_freq(theta, hd // 2).copy()).to(self.device)

    def forward(self, qkv, bias, pos2, plan, out=None, out_dtype="bf16", ovf=None,
                f16_lim=65504.0, stream=None, scratch=None, noalloc=False, rows_prologue=True):
        """noalloc: run clef_hip_vis_attention_noalloc, whose planes are the library's own
        device scratch (no plane tensors are made; `out` is still allocated here if None).
        rows_prologue: hand the library the plan's tok_kv, so the prologue runs over patches
        (else it runs over plane rows through kv_tok)."""
        lib = _lib.load()
        if plan.causal or plan.cu_k is not None:
            raise ValueError("vision attention takes a bidirectional fresh plan")
        P, dev = plan.T, self.device
        _check(qkv, "qkv", (P, 3 * self.E), torch.bfloat16, dev)
        if bias is not None:
            _check(bias, "bias", (3 * self.E,), torch.float32, dev)
        _check(pos2, "pos2", (P, 2), torch.int32, dev)
        out_type, odt = _OUT_TYPES[out_dtype]
        if out is None:
            out = torch.empty((P, self.E), dtype=odt, device=dev)
        _check(out, "out", (P, self.E), odt, dev)
        if ovf is not None:
            _check(ovf, "ovf", (P,), torch.int32, dev)
        kvT = plan.kvT
        if noalloc:
            q_plane = k_plane = vt_plane = None
        else:
            if scratch is None:
                scratch = self.scratch(P, kvT)
            q_plane, k_plane, vt_plane = scratch
            _check(q_plane, "q_plane", (self.heads, P, self.hd), torch.bfloat16, dev)
            _check(k_plane, "k_plane", (self.heads, kvT, self.hd), torch.bfloat16, dev)
            _check(vt_plane, "vt_plane", (self.heads, self.hd, kvT), torch.bfloat16, dev)
        a = VisArgs()
        a.P, a.heads, a.hd, a.scale = P, self.heads, self.hd, self.scale
        a.qkv, a.bias, a.pos2, a.inv_freq = _ptr(qkv), _ptr(bias), _ptr(pos2), _ptr(self.inv_freq)
        a.q_plane, a.k_plane, a.vt_plane, a.kvT = _ptr(q_plane), _ptr(k_plane), _ptr(vt_plane), kvT
        a.blocks, a.n_blk, a.kv_tok, a.kv_rows = _ptr(plan.blocks), plan.n_blk, _ptr(plan.kv_tok), plan.kv_rows
        a.out, a.out_type, a.f16_lim, a.ovf = _ptr(out), out_type, f16_lim, _ptr(ovf)
        a.tok_kv = _ptr(plan.tok_kv) if rows_prologue else None
        err = _err()
        fn = lib.clef_hip_vis_attention_noalloc if noalloc else lib.clef_hip_vis_attention
        _lib.check(fn(ctypes.byref(a), _stream_handle(stream), err, len(err)), err)
        return out

    def scratch(self, P, kvT):
        dev = self.device
        return (torch.empty((self.heads, max(P, 1), self.hd), dtype=torch.bfloat16, device=dev),
                torch.empty((self.heads, kvT, self.hd), dtype=torch.bfloat16, device=dev),
                torch.empty((self.heads, self.hd, kvT), dtype=torch.bfloat16, device=dev))
