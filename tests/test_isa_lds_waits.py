"""Static check of the built kernels' gfx950 assembly: no register that an inline-asm LDS read
(`ds_read_*` inside an asm statement) is still filling may be read, copied or overwritten before
an `s_waitcnt lgkmcnt(N)` covers that read.

The kernels issue LDS operand reads as inline asm and wait for them with separate asm waits, so
that the reads run ahead of the products they feed. The compiler sees the asm output as defined
when the read statement ends; if it copies or spills that register before the wait (it did once,
for the gate chunks of the text epilogue: `v_mov_b64` of a ring register between its read and
its wait), the copy holds stale data whenever the read has not landed yet. Tests on the GPU pass
or fail on such a race by timing; this scan finds it in the code. Compiled here with hipcc, no GPU.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "cleffa_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]$", tok)
    if m:
        return {f"{m.group(1)}{k}" for k in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {tok} if re.match(r"[va]\d+$", tok) else set()


def lds_wait_hazards(lines):
    """Linear scan of one kernel's assembly. LDS-counter operations (asm ds_reads with their
    destination registers, compiler ds ops and scalar loads as placeholders) are queued in issue
    order; `s_waitcnt lgkmcnt(N)` retires all but the newest N. Any other instruction that names a
    register of a queued asm read is reported. Past an unconditional branch, the queue restarts at
    the next label (its predecessors are elsewhere in the listing)."""
    pending, found = [], []
    in_asm = dead = False
    for n, line in enumerate(lines):
        if "ASMSTART" in line:
            in_asm = True
            continue
        if "ASMEND" in line:
            in_asm = False
            continue
        if line.startswith(".LBB") and dead:
            pending, dead = [], False
        t = line.split(";")[0].strip()
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        op = t.split()[0]
        dead = op in ("s_branch", "s_endpgm", "s_setpc_b64")
        args = [a.strip() for a in t[len(op):].split(",")]
        m = re.search(r"lgkmcnt\((\d+)\)", t)
        if op == "s_waitcnt":
            if m:
                keep = int(m.group(1))
                pending = pending[len(pending) - keep:] if keep else []
            continue
        if op.startswith("ds_read") or op.startswith("ds_load"):
            srcs = set().union(*[_regs(a) for a in args[1:]])
            if any(p & srcs for p in pending):
                found.append((n, t))
            pending.append(_regs(args[0]) if in_asm else set())
            continue
        if op.startswith("ds_") or op.startswith("s_load") or op.startswith("s_buffer_load"):
            pending.append(set())
            continue
        used = set().union(*[_regs(a) for a in args])
        if any(p & used for p in pending):
            found.append((n, t))
    return found


def test_scanner_catches_a_copy_before_the_wait():
    good = ["\t;;#ASMSTART", "\tds_read_b128 v[8:11], v2", "\t;;#ASMEND", "\t;;#ASMSTART",
            "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND", "\tv_mov_b32 v0, v8"]
    bad = ["\t;;#ASMSTART", "\tds_read_b128 v[8:11], v2", "\t;;#ASMEND", "\tv_mov_b64_e32 v[0:1], v[10:11]",
           "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND"]
    ahead = ["\t;;#ASMSTART", "\tds_read_b128 v[8:11], v2", "\t;;#ASMEND", "\t;;#ASMSTART",
             "\tds_read_b128 v[12:15], v3", "\t;;#ASMEND", "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(1)",
             "\t;;#ASMEND", "\tv_mov_b32 v0, v8", "\tv_mov_b32 v1, v12"]
    assert lds_wait_hazards(good) == []
    assert len(lds_wait_hazards(bad)) == 1
    assert [t for _, t in lds_wait_hazards(ahead)] == ["v_mov_b32 v1, v12"]


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not found")
@pytest.mark.parametrize("src", ["attn_api.hip", "omni_api.hip"])
def test_asm_lds_reads_are_waited_before_use(src, tmp_path):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-c", "--save-temps",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", str(REPO / "include"), "-I", str(CSRC), str(CSRC / src), "-o", str(tmp_path / "k.o")]
    res = subprocess.run(cmd, cwd=tmp_path, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    asm = next(tmp_path.glob("*gfx950.s")).read_text()
    kernels = re.findall(r"^\s*\.type\s+(_Z\w+),@function", asm, re.M)
    assert kernels, "no kernels in the assembly"
    report = {}
    for k in kernels:
        i = asm.index(k + ":")
        j = asm.index(".Lfunc_end", i)
        bad = lds_wait_hazards(asm[i:j].split("\n"))
        if bad:
            report[k] = bad[:4]
    assert not report, f"LDS read registers used before their wait: {report}"
