"""The C ABI library loads, exports every function include/clef_hip_attn.h declares, and rejects
bad arguments with a "hip: " message before touching the device (clef_metal.m:83-86 error
convention). No GPU needed."""
import ctypes
import re
from pathlib import Path

import pytest

from cleffa_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "clef_hip_attn.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(clef_hip_\w+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert names, "no declarations found"
    for name in names:
        assert hasattr(lib, name), f"{name} is declared but not exported"
    assert set(names) == set(_lib.EXPORTS)


def test_version_and_wave():
    lib = _lib.load()
    assert lib.clef_hip_attn_version() >= 1
    assert lib.clef_hip_attn_wave_size() == 64


def _args(**over):
    a = _lib.AttnArgs()
    a.nh, a.nkv, a.hd, a.n_rot, a.eps, a.scale = 24, 4, 256, 64, 1e-6, 1 / 16
    a.T, a.row, a.kvT, a.n_blk, a.kv_rows = 8, 14336, 64, 1, 64
    fake = ctypes.c_void_p(1 << 20)   # aligned, never dereferenced: every case fails validation first
    for f in ("qkv", "q_norm", "k_norm", "pos3", "inv_freq", "k_plane", "vt_plane", "blocks", "kv_tok", "out"):
        setattr(a, f, fake)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,msg", [
    (dict(hd=128), "hd 256"),
    (dict(nh=24, nkv=5), "head counts"),
    (dict(n_rot=48), "n_rot"),
    (dict(row=1000), "qkv row"),
    (dict(kvT=60), "kvT"),
    (dict(qkv=ctypes.c_void_p((1 << 20) + 2)), "qkv must be"),
    (dict(out_type=7), "out_type"),
    (dict(q_norm=None), "both"),
    (dict(qkv_type=2), "qkv_type"),
])
def test_core_rejects_bad_arguments(over, msg):
    lib = _lib.load()
    err = ctypes.create_string_buffer(256)
    a = _args(**over)
    assert not lib.clef_hip_attn_core(ctypes.byref(a), None, err, len(err))
    text = err.value.decode()
    assert text.startswith("hip: ") and msg in text, text


def test_vision_rejects_bad_head_dim():
    lib = _lib.load()
    a = _lib.VisArgs()
    a.hd, a.heads, a.P = 64, 16, 16
    err = ctypes.create_string_buffer(256)
    assert not lib.clef_hip_vis_attention(ctypes.byref(a), None, err, len(err))
    assert "hd 72" in err.value.decode()


def test_null_args_and_small_error_buffer():
    lib = _lib.load()
    assert not lib.clef_hip_attn_prefill(None, None, None, 0)
    err = ctypes.create_string_buffer(8)
    assert not lib.clef_hip_attn_core(None, None, err, len(err))
    assert err.value.decode() == "hip: nu"
