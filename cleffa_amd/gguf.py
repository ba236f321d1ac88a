"""The projections' weights from a clef GGUF (clef_gguf.c reader, clef.c:27-59 geometry,
clef.c:180-256 per-layer binding), through the C ABI: a read-only mmap'd view, the attention
geometry, and one layer's attention tensors copied into device tensors."""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import AttnConfig, GgufTensorInfo
from .attention import _err, _stream_handle

_NP = {_lib.GGML_F32: np.float32, _lib.GGML_F16: np.float16, _lib.GGML_BF16: np.uint16}


class GgufFile:
    def __init__(self, path):
        lib = _lib.load()
        self._h = ctypes.c_void_p()
        err = _err()
        _lib.check(lib.clef_hip_gguf_open(str(path).encode(), ctypes.byref(self._h), err, len(err)), err)

    def close(self):
        if self._h:
            _lib.load().clef_hip_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, info)] in file order."""
        lib = _lib.load()
        out = []
        name = ctypes.create_string_buffer(512)
        for i in range(lib.clef_hip_gguf_tensor_count(self._h)):
            info = GgufTensorInfo()
            assert lib.clef_hip_gguf_tensor_at(self._h, i, ctypes.byref(info), name, len(name))
            out.append((name.value.decode("utf-8", "surrogateescape"), info))
        return out

    def tensor(self, name):
        """The tensor as a numpy array over the mapping (bf16 as uint16), shape reversed from ne."""
        info = GgufTensorInfo()
        if not _lib.load().clef_hip_gguf_find_tensor(self._h, name.encode(), ctypes.byref(info)):
            raise KeyError(name)
        dt = _NP[info.type]
        shape = tuple(int(info.ne[d]) for d in range(info.n_dims))[::-1]
        buf = (ctypes.c_uint8 * info.nbytes).from_address(info.data)
        return np.frombuffer(buf, dtype=dt).reshape(shape)

    def u32(self, key):
        v = ctypes.c_uint32()
        return v.value if _lib.load().clef_hip_gguf_get_u32(self._h, key.encode(), ctypes.byref(v)) else None

    def f32(self, key):
        v = ctypes.c_float()
        return v.value if _lib.load().clef_hip_gguf_get_f32(self._h, key.encode(), ctypes.byref(v)) else None

    def attn_config(self):
        c = AttnConfig()
        err = _err()
        _lib.check(_lib.load().clef_hip_gguf_attn_config(self._h, ctypes.byref(c), err, len(err)), err)
        return c

    def attn_layer(self, layer, device="cuda", stream=None):
        """Layer `layer`'s w_qkv [n_attn][H] bf16, w_o [H][nh*hd] bf16, q_norm, k_norm [hd] f32 on the
        device (the QKV GEMM's and o_proj's W, the path's norm weights)."""
        c = self.attn_config()
        n_attn = 2 * c.nh * c.hd + 2 * c.nkv * c.hd
        w_qkv = torch.empty(n_attn, c.H, dtype=torch.bfloat16, device=device)
        w_o = torch.empty(c.H, c.nh * c.hd, dtype=torch.bfloat16, device=device)
        qn = torch.empty(c.hd, dtype=torch.float32, device=device)
        kn = torch.empty(c.hd, dtype=torch.float32, device=device)
        err = _err()
        ok = _lib.load().clef_hip_gguf_attn_layer(self._h, ctypes.byref(c), layer, w_qkv.data_ptr(), w_o.data_ptr(),
                                                  qn.data_ptr(), kn.data_ptr(), _stream_handle(stream), err, len(err))
        _lib.check(ok, err)
        return w_qkv, w_o, qn, kn

    def vis_layer(self, layer, heads=16, device="cuda", stream=None):
        E = 72 * heads
        w_qkv = torch.empty(3 * E, E, dtype=torch.bfloat16, device=device)
        b_qkv = torch.empty(3 * E, dtype=torch.float32, device=device)
        w_o = torch.empty(E, E, dtype=torch.bfloat16, device=device)
        b_o = torch.empty(E, dtype=torch.float32, device=device)
        err = _err()
        ok = _lib.load().clef_hip_gguf_vis_layer(self._h, layer, heads, w_qkv.data_ptr(), b_qkv.data_ptr(), w_o.data_ptr(),
                                                 b_o.data_ptr(), _stream_handle(stream), err, len(err))
        _lib.check(ok, err)
        return w_qkv, b_qkv, w_o, b_o
