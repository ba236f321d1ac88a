"""Builds the HIP shared library in-tree (hipcc, gfx950). Used by __graft_entry__.build()."""
import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
LIB = ROOT / "libclef_hip_attn.so"
SOURCES = [ROOT / "csrc" / "attn_api.hip", ROOT / "csrc" / "prefix_cache.hip", ROOT / "csrc" / "omni_api.hip", ROOT / "csrc" / "records.cpp",
           ROOT / "csrc" / "gemm_api.cpp", ROOT / "csrc" / "mfma_ceiling.hip"]
DEPS = SOURCES + [ROOT / "csrc" / "attn_kernels.h", ROOT / "csrc" / "attn_params.h", ROOT / "csrc" / "attn_text.h",
                  ROOT / "csrc" / "attn_vis.h", ROOT / "csrc" / "omni_attn.h",
                  REPO / "include" / "clef_hip_attn.h"]


def hipcc_command(out=LIB):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    return [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
            # packed fp32 VALU ops are kept out of the generated code (see DESIGN notes)
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", str(REPO / "include"), "-I", str(ROOT / "csrc"),
            *[str(s) for s in SOURCES], "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib",
            "-o", str(out)]


def build(verbose=False):
    """Compiles libclef_hip_attn.so; always recompiles."""
    cmd = hipcc_command()
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
