"""Builds the HIP shared library in-tree (hipcc, gfx950). Used by __graft_entry__.build()."""
import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
LIB = ROOT / "libclef_hip_attn.so"
SOURCES = [ROOT / "csrc" / "attn_api.hip", ROOT / "csrc" / "prefix_cache.hip", ROOT / "csrc" / "omni_api.hip", ROOT / "csrc" / "records.cpp",
           ROOT / "csrc" / "gemm_api.cpp", ROOT / "csrc" / "gguf_layer.cpp"]
# the measurement utility bench.py uses, kept out of the engine-facing library
BENCH_LIB = ROOT / "libclef_hip_bench.so"
BENCH_SOURCES = [ROOT / "csrc" / "mfma_ceiling.hip"]
DEPS = SOURCES + BENCH_SOURCES + [ROOT / "csrc" / "attn_kernels.h", ROOT / "csrc" / "attn_params.h", ROOT / "csrc" / "attn_text.h",
                  ROOT / "csrc" / "attn_vis.h", ROOT / "csrc" / "omni_attn.h", ROOT / "csrc" / "attn_text_f32.h", ROOT / "csrc" / "gguf_view.h",
                  REPO / "include" / "clef_hip_attn.h"]


def hipcc_command(out=LIB, sources=None, libs=("-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib")):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    sources = SOURCES if sources is None else sources
    return [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
            # packed fp32 VALU ops are kept out of the generated code (see DESIGN notes)
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", str(REPO / "include"), "-I", str(ROOT / "csrc"),
            *[str(s) for s in sources], *libs, "-o", str(out)]


# A C caller of the library (tests/c_abi/abi_run.c): the boundary as the engine links it.
C_CALLER = REPO / "tests" / "c_abi" / "abi_run"


def c_caller_command():
    return [os.environ.get("CC", "gcc"), "-std=c99", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
            "-I", str(REPO / "include"), "-I", "/opt/rocm/include", str(C_CALLER) + ".c",
            "-L", str(ROOT), "-lclef_hip_attn", "-L/opt/rocm/lib", "-lamdhip64",
            "-Wl,-rpath,$ORIGIN/../../cleffa_amd", "-Wl,-rpath,/opt/rocm/lib", "-o", str(C_CALLER)]


def build(verbose=False):
    """Compiles libclef_hip_attn.so, libclef_hip_bench.so and the C caller test program; always
    recompiles."""
    for cmd in (hipcc_command(), hipcc_command(BENCH_LIB, BENCH_SOURCES, ()), c_caller_command()):
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + res.stderr[-4000:])
        if verbose:
            print(" ".join(cmd))
    return LIB


def stale():
    if not LIB.exists():
        return True
    t = LIB.stat().st_mtime
    return any(p.stat().st_mtime > t for p in DEPS)


if __name__ == "__main__":
    print(build(verbose=True))
