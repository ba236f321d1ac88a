"""The C ABI as a C compiler sees it: tests/c_abi/abi_layout.c prints every argument struct's
field offsets and sizes from include/clef_hip_attn.h, which must match the ctypes mirror the
Python layer passes (cleffa_amd/_lib.py); tests/c_abi/abi_run.c is a C caller that plans and runs
a small prefill through libclef_hip_attn.so (GPU), checked here against the float64 oracle."""
import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from cleffa_amd import _lib, workloads
from tests.helpers import assert_close, oracle_text

ROOT = Path(__file__).resolve().parents[1]
C_DIR = ROOT / "tests" / "c_abi"
STRUCTS = {"clef_hip_attn_args": _lib.AttnArgs, "clef_hip_vis_args": _lib.VisArgs,
           "clef_hip_omni_prep_args": _lib.OmniPrepArgs, "clef_hip_omni_attn_args": _lib.OmniAttnArgs}


def _c_layout(tmp_path):
    exe = tmp_path / "abi_layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-I", str(ROOT / "include"), str(C_DIR / "abi_layout.c"),
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    fields, sizes = {}, {}
    for line in out.splitlines():
        p = line.split()
        if p[1] == "sizeof":
            sizes[p[0]] = int(p[2])
        else:
            fields.setdefault(p[0], []).append((p[1], int(p[2]), int(p[3])))
    return fields, sizes


def test_struct_layout_matches_ctypes(tmp_path):
    fields, sizes = _c_layout(tmp_path)
    assert set(fields) == set(STRUCTS)
    for name, cls in STRUCTS.items():
        c_fields = fields[name]
        py_fields = [f[0] for f in cls._fields_]
        assert [f[0] for f in c_fields] == py_fields, f"{name}: field order differs"
        for fname, off, size in c_fields:
            desc = getattr(cls, fname)
            assert (desc.offset, desc.size) == (off, size), f"{name}.{fname}: C {off}/{size}, ctypes {desc.offset}/{desc.size}"
        assert ctypes.sizeof(cls) == sizes[name], f"{name}: sizeof differs"


@pytest.mark.gpu
def test_c_caller_prefill(tmp_path):
    """plan -> prefill from C (with and without a host schedule), then the f32-row refusal."""
    print("[c-abi] abi_run", flush=True)
    exe = C_DIR / "abi_run"
    assert exe.exists(), "tests/c_abi/abi_run is built by __graft_entry__.build()"
    cu = [0, 37, 101, 102, 232]
    w = workloads.text_inputs(list(np.diff(cu)), 8, 2, seed=17)
    w.update(gate=True, theta=1e7)
    w["qkv"].contiguous().view(torch.int16).numpy().tofile(tmp_path / "qkv.bin")
    w["q_norm"].numpy().astype(np.float32).tofile(tmp_path / "qn.bin")
    w["k_norm"].numpy().astype(np.float32).tofile(tmp_path / "kn.bin")
    w["pos3"].numpy().astype(np.int32).tofile(tmp_path / "pos3.bin")
    res = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr + res.stdout
    T = cu[-1]
    got = np.fromfile(tmp_path / "out.bin", dtype=np.uint16).reshape(T, 8 * 256)
    got_s = np.fromfile(tmp_path / "out_sched.bin", dtype=np.uint16).reshape(T, 8 * 256)
    assert np.array_equal(got, got_s), "the host schedule changed the output bytes"
    f = (got.astype(np.uint32) << 16).view(np.float32)
    assert_close(f, oracle_text(w), what="C caller")
