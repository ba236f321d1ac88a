"""The library's host code under AddressSanitizer: libclef_hip_attn.so is rebuilt host-only
with `-Xarch_host -fsanitize=address` (device code unchanged) and tests/c_abi/host_asan.c drives every
host-only entry point over seeded random and edge-case inputs with exactly sized buffers, and the
GGUF reader over well-formed, truncated and byte-corrupted files. Any out-of-bounds access or use
after free aborts the run with a report. CPU only; no GPU call is made."""
import os
import random
import shutil
import subprocess
from pathlib import Path

import pytest

from cleffa_amd import build
from tests.gguf import writer as gw

ROOT = Path(__file__).resolve().parents[1]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANG = "/opt/rocm/llvm/bin/clang"

pytestmark = pytest.mark.skipif(not (Path(HIPCC).exists() and Path(CLANG).exists()), reason="ROCm toolchain not found")


def _gguf_cases(tmp):
    good = tmp / "good.gguf"
    gw.clef_attention_model(str(good), H=64, nh=2, nkv=1, hd=256, layer_types=(0, 1), vis_heads=1, seed=3)
    data = good.read_bytes()
    paths = [good]
    rng = random.Random(7)
    # truncations across the header, the metadata, the tensor table and the data
    cuts = sorted({1, 3, 4, 8, 16, 23, 24, 32} | {rng.randrange(1, len(data)) for _ in range(40)})
    for c in cuts:
        p = tmp / f"cut{c}.gguf"
        p.write_bytes(data[:c])
        paths.append(p)
    # single-byte corruptions in the first 4 KiB (header, counts, lengths, offsets, types)
    for i in range(120):
        b = bytearray(data)
        pos = rng.randrange(0, min(len(b), 4096))
        b[pos] = rng.choice([0x00, 0xff, 0x7f, 0x80, b[pos] ^ (1 << rng.randrange(8))])
        p = tmp / f"flip{i}.gguf"
        p.write_bytes(bytes(b))
        paths.append(p)
    (tmp / "empty.gguf").write_bytes(b"")
    paths.append(tmp / "empty.gguf")
    paths.append(tmp / "missing.gguf")
    return paths


def test_host_entry_points_under_asan(tmp_path):
    lib = tmp_path / "libclef_hip_attn.so"
    cmd = build.hipcc_command(out=lib)
    i = cmd.index("-O3")
    cmd[i:i + 1] = ["-O1", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    syms = subprocess.run(["nm", "-D", str(lib)], capture_output=True, text=True).stdout
    assert "__asan_report_load" in syms, "the library was not built with AddressSanitizer"
    exe = tmp_path / "host_asan"
    res = subprocess.run([CLANG, "-std=c99", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
                          "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"), "-I", "/opt/rocm/include",
                          str(ROOT / "tests" / "c_abi" / "host_asan.c"), "-L", str(tmp_path), "-lclef_hip_attn",
                          f"-Wl,-rpath,{tmp_path}", "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    files = _gguf_cases(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1")
    res = subprocess.run([str(exe), *map(str, files)], capture_output=True, text=True, env=env, timeout=600)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-6000:])
    assert res.stdout.startswith("ok "), res.stdout
