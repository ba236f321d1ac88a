"""ctypes wrapper of the CPU oracle (libattn_oracle.so, built from attn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. Never part of the product path.
"""
import ctypes
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libattn_oracle.so"

_lib = None


REF_GGUF = HERE / "_ref" / "libclef_gguf_ref.so"
REF_SRC = Path("/root/reference/clef_gguf.c")


def build():
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True, capture_output=True)
    # the reference's own GGUF reader, compiled from its sources where they lie, when present
    if REF_SRC.exists():
        subprocess.run(["make", "-B", "-C", str(HERE), "ref"], check=True, capture_output=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        for sfx, real in (("f64", c_double), ("f32", c_float)):
            fn = getattr(lib, f"orc_text_prep_{sfx}")
            fn.argtypes = [c_int, c_int, c_int, c_int, c_int, c_int, c_double] + [c_void_p] * 9
            fn.restype = None
            fn = getattr(lib, f"orc_attention_{sfx}")
            fn.argtypes = [c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                           c_void_p, c_int, c_int, c_double, c_void_p, c_void_p, c_void_p, c_int]
            fn.restype = None
            fn = getattr(lib, f"orc_vis_prep_{sfx}")
            fn.argtypes = [c_int, c_int, c_int] + [c_void_p] * 7
            fn.restype = None
            fn = getattr(lib, f"orc_omni_prep_{sfx}")
            fn.argtypes = [c_int, c_int, c_int, c_double, c_int, c_double] + [c_void_p] * 8
            fn.restype = None
        lib.orc_num_threads.restype = c_int
        _lib = lib
    return _lib


def _dt(precision):
    return {"f64": np.float64, "f32": np.float32}[precision]


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def num_threads():
    return load().orc_num_threads()


def text_prep(qkv, nh, nkv, hd, n_rot, q_norm, k_norm, pos3, inv_freq, eps=1e-6, precision="f64"):
    """Q [nh][T][hd], K, V [nkv][T][hd], G [T][nh*hd] from fused qkv rows (metal/clef.metal:245-300).
    q_norm/k_norm None: no RMSNorm (the plain-SDPA operands of C0)."""
    lib = load()
    dt = _dt(precision)
    qkv = _f32(qkv)
    T, row = qkv.shape
    Q = np.empty((nh, T, hd), dt); K = np.empty((nkv, T, hd), dt)
    V = np.empty((nkv, T, hd), dt); G = np.empty((T, nh * hd), dt)
    qn, kn = _f32(q_norm), _f32(k_norm)
    inv = _f32(inv_freq) if n_rot else np.zeros(1, np.float32)
    pos = _i32(pos3) if pos3 is not None else np.zeros((T, 3), np.int32)
    getattr(lib, f"orc_text_prep_{precision}")(T, nh, nkv, hd, n_rot, row, eps, _p(qkv), _p(qn), _p(kn),
                                               _p(pos), _p(inv), _p(Q), _p(K), _p(V), _p(G))
    return Q, K, V, G


def attention(Q, K, V, cu_q, cu_k=None, causal=True, scale=None, G=None, rows=None, precision="f64"):
    """Packed varlen GQA SDPA (ref/safe_attn.py semantics). Returns O [Tq or len(rows)][nh*hd]."""
    lib = load()
    dt = _dt(precision)
    Q, K, V = (np.ascontiguousarray(x, dtype=dt) for x in (Q, K, V))
    nh, Tq, hd = Q.shape
    nkv, Tk, _ = K.shape
    cu_q = _i32(cu_q)
    cu_k = _i32(cu_k)
    G = None if G is None else np.ascontiguousarray(G, dtype=dt)
    rows = _i32(rows)
    n_out = Tq if rows is None else len(rows)
    O = np.empty((n_out, nh * hd), dt)
    scale = hd ** -0.5 if scale is None else scale
    getattr(lib, f"orc_attention_{precision}")(nh, nkv, hd, Tq, Tk, _p(Q), _p(K), _p(V), _p(cu_q), _p(cu_k),
                                               len(cu_q) - 1, int(causal), scale, _p(G), _p(O), _p(rows),
                                               0 if rows is None else len(rows))
    return O


def vis_prep(qkv, heads, hd, bias, pos2, inv_freq, precision="f64"):
    """Q, K, V [heads][P][hd] (metal/clef.metal:1616-1656)."""
    lib = load()
    dt = _dt(precision)
    qkv = _f32(qkv)
    P = qkv.shape[0]
    Q = np.empty((heads, P, hd), dt); K = np.empty_like(Q); V = np.empty_like(Q)
    getattr(lib, f"orc_vis_prep_{precision}")(P, heads, hd, _p(qkv), _p(_f32(bias)), _p(_i32(pos2)),
                                              _p(_f32(inv_freq)), _p(Q), _p(K), _p(V))
    return Q, K, V


def omni_prep(qkv, nh, nkv, q_norm, k_norm, pos3, theta=1e6, exact=True, inv_freq=None, eps=1e-6,
              precision="f64"):
    """Q [nh][T][128], K, V [nkv][T][128] of Omni's attention prep (metal/clef.metal:2074-2131).
    exact=False needs inv_freq [64] (the f32 table): angle = (float)pos * inv_freq[i]."""
    lib = load()
    dt = _dt(precision)
    qkv = _f32(qkv)
    T = qkv.shape[0]
    Q = np.empty((nh, T, 128), dt); K = np.empty((nkv, T, 128), dt); V = np.empty_like(K)
    inv = _f32(inv_freq) if inv_freq is not None else np.zeros(64, np.float32)
    getattr(lib, f"orc_omni_prep_{precision}")(T, nh, nkv, eps, int(bool(exact)), float(theta), _p(qkv),
                                               _p(_f32(q_norm)), _p(_f32(k_norm)), _p(_i32(pos3)), _p(inv),
                                               _p(Q), _p(K), _p(V))
    return Q, K, V
