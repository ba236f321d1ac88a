"""FP32 text mode (qkv_type CLEF_HIP_QKV_F32: the reference's FP32 attention kernels,
metal/clef.metal:250-654, dispatched at clef_metal.m:1330-1413) against the float64 oracle and
the oracle's scalar FP32 restatement, through the C ABI.

Bound (the FP32 kernels' own, bench/vision_attention_bench.m:144-157 style): max-abs error
against float64 within max(5e-5, 2x the FP32 control's), mean-abs within 2x the control's."""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, workloads
from tests.helpers import errors, oracle_text

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _fp32(w, seed=11):
    """The workload with f32 qkv rows: bf16 values given full 24-bit mantissas."""
    g = torch.Generator().manual_seed(seed)
    q = w["qkv"].float()
    q = q * (1.0 + 2.0 ** -9 * torch.randn(q.shape, generator=g))
    return dict(w, qkv=q.contiguous())


def _run(w, out_dtype="f32", ovf=None, plan=None, **kw):
    att = TextAttention(w["nh"], w["nkv"], w["hd"], w["n_rot"], rope_theta=w.get("theta", 1e7))
    plan = plan or AttnPlan(w["cu_seqlens"], causal=True)
    d = lambda t: None if t is None else t.cuda()
    out = att.forward(d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan, out_dtype=out_dtype,
                      gate=w.get("gate", True), ovf=ovf, **kw)
    torch.cuda.synchronize()
    return out, plan


def _check_fp32(got, w, rows=None, what=""):
    want = oracle_text(w, rows=rows)
    ctrl = oracle_text(w, rows=rows, precision="f32")
    mx, mean = errors(got, want)
    cmx, cmean = errors(ctrl, want)
    _say(f"[fp32] {what}: max_abs {mx:.3g} mean_abs {mean:.3g} (f32 control {cmx:.3g} / {cmean:.3g})")
    assert mx <= max(5e-5, 2 * cmx), f"{what}: max_abs {mx:.3g}, control {cmx:.3g}"
    assert mean <= 2 * cmean + 1e-7, f"{what}: mean_abs {mean:.3g}, control {cmean:.3g}"


@pytest.mark.parametrize("name", ["C0", "C1"])
def test_fp32_configs(name):
    _say(f"[fp32] {name}")
    w = _fp32(workloads.config(name, seed=0))
    out, _ = _run(w)
    _check_fp32(out.cpu().numpy(), w, what=name)


def test_fp32_gqa_widths_and_edges():
    """Group sizes 1, 3, 5, 8 (one wave per q head of a group) with ragged records of 1, 2, 15,
    16, 17, 31, 33, 127, 129 tokens: every row offset of the 16-row workgroups and 32-key tiles."""
    lengths = [1, 2, 15, 16, 17, 31, 33, 127, 129]
    for nh, nkv in ((2, 2), (6, 2), (5, 1), (16, 2)):
        _say(f"[fp32] nh {nh} nkv {nkv}")
        w = workloads.text_inputs(lengths, nh, nkv, seed=nh)
        w.update(gate=True, theta=1e7)
        w = _fp32(w)
        out, _ = _run(w)
        _check_fp32(out.cpu().numpy(), w, what=f"{nh}/{nkv}")


def test_fp32_c2_sampled_rows():
    _say("[fp32] C2 sampled rows")
    w = _fp32(workloads.config("C2", seed=0))
    out, _ = _run(w)
    rows = np.array([0, 1, 15, 16, 127, 128, 4095, 8191, 12000, 16383], np.int32)
    _check_fp32(out.cpu().numpy()[rows], w, rows=rows, what="C2")


def test_fp32_packing_invariance_bitwise():
    """Each record's output is bitwise the same packed with others as run alone
    (bench/attention_bench.m:263-308): key tiles start at the record's first key."""
    lengths = [1] * 8 + [2, 9, 31, 32, 33, 63, 65, 263]
    w = _fp32(dict(workloads.text_inputs(lengths, 8, 2, seed=4), gate=True, theta=1e7))
    packed, _ = _run(w)
    cu = w["cu_seqlens"]
    for r, n in enumerate(lengths):
        a, b = int(cu[r]), int(cu[r + 1])
        wr = dict(w, qkv=w["qkv"][a:b].clone(), pos3=w["pos3"][a:b].clone(),
                  cu_seqlens=np.array([0, n], np.int32), lengths=[n])
        alone, _ = _run(wr)
        assert torch.equal(alone.view(torch.int32), packed[a:b].view(torch.int32)), f"record {r} (len {n})"


def test_fp32_16bit_outputs_are_rounded_f32():
    """bf16 / f16 outputs are round-to-nearest-even of the f32 output (act16, clef.metal:98-106)."""
    w = _fp32(dict(workloads.text_inputs([300, 77], 8, 2, seed=6), gate=True, theta=1e7))
    f32, _ = _run(w)
    for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        o, _ = _run(w, out_dtype=dt)
        assert torch.equal(o.view(torch.int16), f32.to(tdt).view(torch.int16)), dt


def test_fp32_f16_overflow_flags_isolated():
    """Odd records' V x 1e5: their f16 outputs saturate and flag the record's first row; the
    other records' outputs are unchanged (bench/attention_bench.m:256-261)."""
    lengths = [100, 150, 64, 200]
    nh, nkv, hd = 8, 2, 256
    w = _fp32(dict(workloads.text_inputs(lengths, nh, nkv, seed=3), gate=False, theta=1e7))
    vcol = 2 * nh * hd + nkv * hd
    cu = w["cu_seqlens"]
    q = w["qkv"].clone()
    for r in (1, 3):
        q[cu[r]:cu[r + 1], vcol:] *= 1e5
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    out, _ = _run(dict(w, qkv=q), out_dtype="f16", ovf=ovf)
    clean, _ = _run(w, out_dtype="f16")
    want = np.zeros(int(cu[-1]), np.int32)
    want[cu[1]] = want[cu[3]] = 1
    assert np.array_equal(ovf.cpu().numpy(), want)
    assert torch.isfinite(out.float()).all()
    for r in (0, 2):
        a, b = cu[r], cu[r + 1]
        assert torch.equal(out[a:b].view(torch.int16), clean[a:b].view(torch.int16))


def test_fp32_prefix_equals_full_pass_bitwise():
    """A prefix-cache pass (queries = a record's last tokens, keys = cached rows + new rows) gives
    bitwise the full pass's rows (tests/test_prefix_attention.m semantics), with the FP32 planes
    of the full pass as the cache."""
    nh, nkv = 8, 2
    full_len, new = 328, 72                 # cached 256 rows (a multiple of 8)
    w = _fp32(dict(workloads.text_inputs([full_len], nh, nkv, seed=8), gate=True, theta=1e7))
    att = TextAttention(nh, nkv, 256, 64, rope_theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    kp, vp = att.planes(plan.kvT, fp32=True)
    d = lambda t: t.cuda()
    full = att.forward(d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan, out_dtype="f32",
                       k_plane=kp, vt_plane=vp, kvT=plan.kvT)
    # prefix pass over the same planes: its prologue rewrites rows 256..327 with the same values
    cq = np.array([0, new], np.int32)
    ck = np.array([0, full_len], np.int32)
    pplan = AttnPlan(cq, ck, causal=True)
    a = full_len - new
    part = att.forward(d(w["qkv"][a:].clone()), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"][a:].clone()), pplan,
                       out_dtype="f32", k_plane=kp, vt_plane=vp, kvT=plan.kvT)
    torch.cuda.synchronize()
    assert torch.equal(part.view(torch.int32), full[a:].view(torch.int32))


@pytest.mark.parametrize("nh,nkv", [(12, 1), (16, 1), (9, 1), (24, 2)])
def test_fp32_wide_groups(nh, nkv):
    """Groups of more than 8 q heads (12 and 16 per kv head; 9, whose second chunk has a spare
    wave; 12 per kv head over two kv heads) run as head chunks, against float64 within the FP32
    bound, with ragged records."""
    _say(f"[fp32] wide group {nh}/{nkv}")
    w = _fp32(dict(workloads.text_inputs([1, 17, 40, 130, 300], nh, nkv, seed=nh), gate=True, theta=1e7))
    out, _ = _run(w)
    _check_fp32(out.cpu().numpy(), w, what=f"{nh}/{nkv}")


def test_fp32_persistent_grid_matches_one_item_per_workgroup(monkeypatch):
    """The persistent grid (CLEF_HIP_F32_PERSISTENT=1: items in snake order, the next item's
    first tile loading during the epilogue) gives bitwise the output of one workgroup per item."""
    _say("[fp32] persistent grid vs one item per workgroup")
    w = _fp32(dict(workloads.text_inputs([700, 33, 129, 1, 260], 24, 4, seed=3), gate=True, theta=1e7))
    one, _ = _run(w)
    monkeypatch.setenv("CLEF_HIP_F32_PERSISTENT", "1")
    out, _ = _run(w)
    assert torch.equal(out.view(torch.int32), one.view(torch.int32))


FP32_GEOMETRIES = [(24, 4), (16, 4), (8, 2), (4, 1), (6, 2), (12, 4), (16, 8), (10, 5), (2, 2), (5, 1), (14, 2),
                   (9, 1), (24, 2), (7, 1)]


@pytest.mark.parametrize("seed", range(24))
def test_fp32_random_pass(seed):
    """Seeded random packed passes in the FP32 mode (ragged records around the 16-row workgroups
    and 32-key tiles; group widths 1-12, split over two waves per head up to 6 and as head chunks
    above 8; with and without the norms, rotary and gate) against float64 within the FP32
    bound."""
    rng = np.random.default_rng(5000 + seed)
    n = int(rng.integers(1, 5))
    lengths = [int(x) for x in rng.choice([1, 2, 15, 16, 17, 31, 33, 64, 65, 127, 129, 300], size=n)]
    nh, nkv = FP32_GEOMETRIES[int(rng.integers(len(FP32_GEOMETRIES)))]
    norm = bool(rng.integers(2))
    n_rot = 64 if norm and rng.integers(3) else 0
    gate = bool(rng.integers(2))
    _say(f"[fp32] random seed {seed}: lengths {lengths} heads {nh}/{nkv} norm {norm} rot {n_rot} gate {gate}")
    w = workloads.text_inputs(lengths, nh, nkv, n_rot=n_rot, seed=seed, norm=norm)
    w.update(gate=gate, theta=1e7)
    w = _fp32(w)
    out, _ = _run(w)
    _check_fp32(out.cpu().numpy(), w, what=f"random {seed}")
