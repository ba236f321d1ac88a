"""A prefix-cache entry's attention planes (clef_metal.m:15-29 struct clef_gpu_prefix,
762-805 prefix_reserve), on torch device memory, grown and copied through the C ABI.

Per attention layer the entry holds K [nkv][cap][hd] (f16) and V^T [nkv][hd][cap] (bf16), indexed by the
record's own token rows. A prefix pass over tokens L..T-1 of the record passes them to
TextAttention.forward as k_plane / vt_plane with kvT = cap and cu_seqlens_k = [0, T]."""
import ctypes

import torch

from . import _lib
from .attention import _stream_handle


class PrefixEntry:
    def __init__(self, n_layers, nkv, hd=256, device="cuda"):
        self.n_layers, self.nkv, self.hd, self.device = n_layers, nkv, hd, device
        self.cap = 0
        self.K = [None] * n_layers
        self.Vt = [None] * n_layers

    def nbytes(self):
        return 2 * self.n_layers * int(_lib.load().clef_hip_prefix_plane_bytes(self.nkv, self.hd, self.cap))

    def reserve(self, rows, keep, stream=None):
        """Capacity for `rows` tokens keeping rows [0, keep). Every new plane is allocated before
        any is replaced, so a failed allocation leaves the entry as it was."""
        lib = _lib.load()
        cap = lib.clef_hip_prefix_capacity(int(rows), self.cap, self.hd)
        if cap < 0:
            raise RuntimeError(f"hip: prefix cache entry of {rows} rows exceeds the plane limit")
        if cap == self.cap:
            return False
        if keep > self.cap:
            raise ValueError(f"keep {keep} exceeds the entry's {self.cap} rows")
        K = [torch.empty(self.nkv, cap, self.hd, dtype=torch.float16, device=self.device) for _ in range(self.n_layers)]
        Vt = [torch.empty(self.nkv, self.hd, cap, dtype=torch.bfloat16, device=self.device) for _ in range(self.n_layers)]
        err = ctypes.create_string_buffer(256)
        s = _stream_handle(stream)
        for l in range(self.n_layers):
            ks = self.K[l].data_ptr() if self.K[l] is not None else None
            vs = self.Vt[l].data_ptr() if self.Vt[l] is not None else None
            ok = lib.clef_hip_prefix_copy(ks, vs, self.cap, K[l].data_ptr(), Vt[l].data_ptr(), cap,
                                          self.nkv, self.hd, int(keep) if ks else 0, s, err, len(err))
            _lib.check(ok, err)
        self.K, self.Vt, self.cap = K, Vt, cap
        return True
