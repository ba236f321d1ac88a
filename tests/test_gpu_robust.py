"""Robustness cases the reference's own tests pin (bench/attention_bench.m, bench/
vision_attention_bench.m), through the C ABI on the GPU:

- stale or NaN contents in the plane slack rows and around the output never reach a result
  (attention_bench.m:132-139 poisons both);
- f16 overflow of the K and Q operands saturates and flags only the record it belongs to, as
  split16 does (clef.metal:857-867), and non-finite V values saturate and flag too;
- the reference's packed layout of 46 records (32 one-token ones) is bitwise packing-invariant,
  overflow flags included (attention_bench.m:263-308), and so are its long layouts
  {8 x 512, 8 x 1,382, 4,510 + 346, 2 x 8,072} (attention_bench.m:310-360), checked against the
  float64 oracle on sampled rows.
"""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, workloads
from tests.helpers import assert_close, gpu_text, oracle_text

pytestmark = pytest.mark.gpu
NAN16 = 0x7FC1   # a NaN in both f16 and bf16


def _say(*a):
    print(*a, flush=True)


def _run(w, planes=None, out=None, out_dtype="bf16", ovf=None, schedule=True, rope_cs=None):
    att = TextAttention(w["nh"], w["nkv"], w["hd"], w["n_rot"], rope_theta=w.get("theta", 1e7))
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    d = lambda t: None if t is None else t.cuda()
    kw = {}
    if planes is not None:
        kw.update(k_plane=planes[0], vt_plane=planes[1], kvT=planes[0].shape[1])
    res = att.forward(d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan, out=out,
                      out_dtype=out_dtype, gate=w.get("gate", True), ovf=ovf, schedule=schedule,
                      rope_cs=rope_cs, **kw)
    torch.cuda.synchronize()
    return res, plan, att


def _bits(t):
    return t.contiguous().view(torch.int16).cpu()


def test_poisoned_planes_and_output_guards():
    """Planes full of NaN (every slack row past a record keeps it) and NaN guard rows around the
    output: the output equals a run on zeroed planes bit for bit, and the guards stay NaN."""
    _say("[poison] text planes + output guards")
    lengths = [1, 63, 64, 65, 129, 300]
    w = workloads.text_inputs(lengths, 8, 2, seed=41)
    w.update(gate=True, theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    kvT, T, E = plan.kvT, plan.T, 8 * 256
    k0 = torch.zeros((2, kvT, 256), dtype=torch.float16, device="cuda")
    v0 = torch.zeros((2, 256, kvT), dtype=torch.bfloat16, device="cuda")
    clean, _, _ = _run(w, planes=(k0, v0))
    kn = torch.full((2, kvT, 256), float("nan"), dtype=torch.float16, device="cuda")
    vn = torch.full((2, 256, kvT), float("nan"), dtype=torch.bfloat16, device="cuda")
    big = torch.full(((T + 8) * E,), NAN16, dtype=torch.int16, device="cuda")
    out = big[4 * E:(4 + T) * E].view(torch.bfloat16).view(T, E)
    cs = torch.full((T, 32, 2), float("nan"), dtype=torch.float32, device="cuda")
    got, _, _ = _run(w, planes=(kn, vn), out=out, rope_cs=cs)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(_bits(got), _bits(clean))
    g = big.cpu().numpy()
    assert (g[:4 * E] == NAN16).all() and (g[(4 + T) * E:] == NAN16).all(), "a guard row was written"


def test_poisoned_vision_planes_and_guards():
    _say("[poison] vision planes + output guards")
    from cleffa_amd import VisionAttention, vision_positions
    grids = [(2, 2), (4, 6), (6, 10)]
    heads, hd = 4, 72
    lens = [a * b for a, b in grids]
    P = sum(lens)
    gen = torch.Generator().manual_seed(5)
    qkv = torch.randn((P, 3 * heads * hd), generator=gen).to(torch.bfloat16).cuda()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pos2 = torch.from_numpy(vision_positions(cu, [b for _, b in grids], 2)).cuda()
    vis = VisionAttention(heads, hd)
    plan = AttnPlan(cu, causal=False)
    E = heads * hd
    scratch = vis.scratch(plan.T, plan.kvT)
    for t in scratch:
        t.zero_()
    clean = vis.forward(qkv, None, pos2, plan, scratch=scratch)
    torch.cuda.synchronize()
    for t in scratch:
        t.fill_(float("nan"))
    big = torch.full(((P + 8) * E,), NAN16, dtype=torch.int16, device="cuda")
    out = big[4 * E:(4 + P) * E].view(torch.bfloat16).view(P, E)
    got = vis.forward(qkv, None, pos2, plan, out=out, scratch=scratch)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(_bits(got), _bits(clean))
    g = big.cpu().numpy()
    assert (g[:4 * E] == NAN16).all() and (g[(4 + P) * E:] == NAN16).all()


def _overflow_case(part):
    """Plain operands (no norms, no rotary), 4 records; record 1 gets a key, a query or a value
    that leaves f16's range (or is NaN). Only record 1's flag rises; the others' bytes stay."""
    lengths = [100, 150, 64, 200]
    w = workloads.text_inputs(lengths, 8, 2, n_rot=0, seed=13, norm=False, outlier_frac=0)
    w.update(gate=True, theta=1e7)
    cu = w["cu_seqlens"]
    nh, nkv, hd = 8, 2, 256
    q = w["qkv"].clone()
    r0, r1 = int(cu[1]), int(cu[2])
    if part == "k":
        q[r0 + 5, 2 * nh * hd + 3] = 1e6                # a key element past 65504
    elif part == "q":
        q[r0 + 7, 2 * hd + 11] = -2e5                   # a query element of head 1
    else:
        q[r0 + 9, 2 * nh * hd + nkv * hd + 17] = float("nan")   # a value element
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    out, _ = gpu_text(dict(w, qkv=q), ovf=ovf)
    clean, _ = gpu_text(w)
    flags = ovf.cpu().numpy()
    want = np.zeros_like(flags)
    want[r0] = 1
    assert np.array_equal(flags, want), np.nonzero(flags)
    assert torch.isfinite(out.float()).all()
    for r in (0, 2, 3):
        a, b = int(cu[r]), int(cu[r + 1])
        assert torch.equal(_bits(out[a:b]), _bits(clean[a:b])), f"record {r} changed"
    return out, clean, r0, r1


@pytest.mark.parametrize("part", ["k", "q", "v"])
def test_operand_overflow_flags_its_record(part):
    _say(f"[split16] {part} overflow")
    _overflow_case(part)


REF_PACKED = [1] * 32 + [2, 3, 4, 5, 6, 7, 8, 9, 31, 32, 33, 63, 65, 263]


@pytest.mark.parametrize("f16", [False, True])
def test_reference_packed_layout_bitwise(f16):
    """attention_bench.m:263-308: 46 records (32 of one token), every odd record's V scaled by
    1e5 in the f16 case; each record's output bytes and flags equal its own run alone."""
    _say(f"[invariance] reference packed layout f16={f16}")
    lengths = REF_PACKED
    w = workloads.text_inputs(lengths, 16, 4, seed=23)
    w.update(gate=False, theta=1e7)
    cu = w["cu_seqlens"]
    nh, nkv, hd = 16, 4, 256
    vcol = 2 * nh * hd + nkv * hd
    q = w["qkv"].clone()
    if f16:
        for i in range(1, len(lengths), 2):
            q[cu[i]:cu[i + 1], vcol:] = (q[cu[i]:cu[i + 1], vcol:].float() * 1e5).to(torch.bfloat16)
    w = dict(w, qkv=q)
    dt = "f16" if f16 else "bf16"
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    packed, _ = gpu_text(w, out_dtype=dt, ovf=ovf)
    packed_b, flags = _bits(packed), ovf.cpu().numpy()
    if f16:
        assert flags[cu[1:-1:2]].all() and flags.sum() == len(lengths) // 2
    else:
        assert flags.sum() == 0
    for r, n in enumerate(lengths):
        a, b = int(cu[r]), int(cu[r + 1])
        alone = dict(w, qkv=q[a:b].clone(), pos3=w["pos3"][a:b].clone(),
                     cu_seqlens=np.array([0, n], np.int32))
        ovf1 = torch.zeros(n, dtype=torch.int32, device="cuda")
        out, _ = gpu_text(alone, out_dtype=dt, ovf=ovf1)
        assert torch.equal(_bits(out), packed_b[a:b]), f"record {r} bytes differ"
        assert np.array_equal(ovf1.cpu().numpy(), flags[a:b]), f"record {r} flags differ"
    if not f16:
        rows = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, np.arange(0, int(cu[-1]), 7)])).astype(np.int32)
        assert_close(packed.float().cpu().numpy()[rows], oracle_text(w, rows=rows), what="reference packed")


def test_many_one_token_records_bitwise():
    """80 one-token records packed around longer ones (200, 70), so one-token records sit at every
    row offset of a 128-row block and of a 64-key tile; each record equals its run alone bit for
    bit (attention_bench.m:263-308 with more one-token records than one block holds)."""
    _say("[invariance] 80 one-token records")
    lengths = [1] * 40 + [200] + [1] * 40 + [70]
    w = workloads.text_inputs(lengths, 8, 2, seed=29)
    w.update(gate=True, theta=1e7)
    cu = w["cu_seqlens"]
    packed, _ = gpu_text(w)
    packed_b = _bits(packed)
    for r, n in enumerate(lengths):
        a, b = int(cu[r]), int(cu[r + 1])
        alone = dict(w, qkv=w["qkv"][a:b].clone(), pos3=w["pos3"][a:b].clone(),
                     cu_seqlens=np.array([0, n], np.int32))
        out, _ = gpu_text(alone)
        assert torch.equal(_bits(out), packed_b[a:b]), f"record {r} (len {n}) bytes differ"
    rows = np.arange(int(cu[-1]), dtype=np.int32)
    assert_close(packed.float().cpu().numpy(), oracle_text(w, rows=rows), what="one-token records")


@pytest.mark.parametrize("lengths", [[512] * 8, [1382] * 8, [4510, 346], [8072, 8072]],
                         ids=["8x512", "8x1382", "4510+346", "2x8072"])
def test_reference_long_layouts(lengths):
    """attention_bench.m:310-360: long records across many key tiles and records sharing a block
    boundary; each record equals its run alone bit for bit; sampled rows against float64."""
    _say(f"[invariance] long layout {lengths}")
    w = workloads.text_inputs(lengths, 16, 4, seed=29, device="cuda")
    w.update(gate=True, theta=1e7)
    cu = w["cu_seqlens"]
    packed, _ = gpu_text(w)
    packed_b = _bits(packed)
    for r, n in enumerate(lengths):
        a, b = int(cu[r]), int(cu[r + 1])
        alone = dict(w, qkv=w["qkv"][a:b].clone(), pos3=w["pos3"][a:b].clone(),
                     cu_seqlens=np.array([0, n], np.int32))
        out, _ = gpu_text(alone)
        assert torch.equal(_bits(out), packed_b[a:b]), f"record {r} bytes differ"
    rng = np.random.default_rng(7)
    T = int(cu[-1])
    rows = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, cu[1:-1] - 1, rng.integers(0, T, 40)])).astype(np.int32)
    want = oracle_text(w, rows=rows)
    assert_close(packed.float().cpu().numpy()[rows], want, what=f"long {lengths}")


def _vision_case(seed=3, grids=((4, 6), (16, 18), (2, 2), (6, 10)), heads=4):
    from cleffa_amd import VisionAttention, vision_positions
    hd = 72
    lens = [a * b for a, b in grids]
    P = sum(lens)
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn((P, 3 * heads * hd), generator=gen).to(torch.bfloat16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pos2 = torch.from_numpy(vision_positions(cu, [b for _, b in grids], 2)).cuda()
    return VisionAttention(heads, hd), AttnPlan(cu, causal=False), qkv, pos2, cu


def test_vision_prologue_forms_agree():
    """The prologue over patches (tok_kv given) and over plane rows (kv_tok) write the same Q
    plane, the same owned K and V^T plane rows and the same output, bit for bit, with the qkv
    bias, over images of 4 to 288 patches (64-row tiles that cross images and end mid-tile)."""
    _say("[vision] prologue over patches = over plane rows")
    vis, plan, qkv, pos2, _ = _vision_case(seed=11, grids=((4, 6), (16, 18), (2, 2), (6, 10), (1, 4)), heads=6)
    E = vis.E
    gen = torch.Generator().manual_seed(12)
    bias = (0.5 * torch.randn(3 * E, generator=gen)).cuda()
    qkv = qkv.cuda()
    res = []
    for rows in (True, False):
        scratch = vis.scratch(plan.T, plan.kvT)
        for s in scratch:
            s.zero_()
        out = vis.forward(qkv, bias, pos2, plan, scratch=scratch, rows_prologue=rows)
        torch.cuda.synchronize()
        res.append((out, scratch))
    (o1, (q1, k1, v1)), (o0, (q0, k0, v0)) = res
    own = torch.from_numpy(np.flatnonzero(plan.kv_tok_host >= 0)).cuda()
    assert torch.equal(_bits(q1), _bits(q0))
    assert torch.equal(_bits(k1[:, own]), _bits(k0[:, own]))
    assert torch.equal(_bits(v1[:, :, own]), _bits(v0[:, :, own]))
    assert torch.equal(_bits(o1), _bits(o0))


def test_vision_row_sums_with_unit_values():
    """V = 1: the output is the row sum of P over the row sum the ones row accumulated, exactly 1
    in f32, across images of 24 to 288 patches (tail tiles included)."""
    _say("[vision] V = 1 row sums")
    vis, plan, qkv, pos2, _ = _vision_case()
    E = vis.E
    q = qkv.clone()
    q[:, 2 * E:] = 1.0
    out = vis.forward(q.cuda(), None, pos2, plan, out_dtype="f32")
    torch.cuda.synchronize()
    err = (out.double() - 1.0).abs().max().item()
    assert err <= 2e-6, err


def test_vision_16bit_outputs_are_rounded_f32():
    """vision_attention_bench.m:159-169: bf16 and f16 outputs equal the f32 output rounded to
    nearest even, bit for bit."""
    _say("[vision] act16 rounding")
    vis, plan, qkv, pos2, _ = _vision_case(seed=8)
    qkv = qkv.cuda()
    f32 = vis.forward(qkv, None, pos2, plan, out_dtype="f32")
    b16 = vis.forward(qkv, None, pos2, plan, out_dtype="bf16")
    f16 = vis.forward(qkv, None, pos2, plan, out_dtype="f16")
    torch.cuda.synchronize()
    assert torch.equal(_bits(f32.to(torch.bfloat16)), _bits(b16))
    assert torch.equal(_bits(f32.to(torch.float16)), _bits(f16))


def test_vision_f16_overflow_flags_isolated():
    """vision_attention_bench.m:170-177: an image whose output leaves f16's range is flagged at
    its first patch and saturates (values scaled by 1e7, so that the average over the image still
    leaves the range); the other images' bytes are unchanged."""
    _say("[vision] f16 overflow flags")
    vis, plan, qkv, pos2, cu = _vision_case(seed=12)
    E = vis.E
    q = qkv.clone()
    a, b = int(cu[1]), int(cu[2])
    q[a:b, 2 * E:] = (q[a:b, 2 * E:].float() * 1e7).to(torch.bfloat16)
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    out = vis.forward(q.cuda(), None, pos2, plan, out_dtype="f16", ovf=ovf)
    clean = vis.forward(qkv.cuda(), None, pos2, plan, out_dtype="f16")
    torch.cuda.synchronize()
    flags = ovf.cpu().numpy()
    want = np.zeros_like(flags)
    want[a] = 1
    assert np.array_equal(flags, want)
    assert torch.isfinite(out.float()).all()
    for r in (0, 2, 3):
        x, y = int(cu[r]), int(cu[r + 1])
        assert torch.equal(_bits(out[x:y]), _bits(clean[x:y])), f"image {r} changed"


def test_large_finite_value_flags_its_record():
    """A finite V element past f16's range (1e5, exact in bf16's range) flags its record, as
    split16 does for the reference's f16 V plane; the other records keep their bytes."""
    _say("[split16] finite v overflow")
    lengths = [100, 150, 64, 200]
    w = workloads.text_inputs(lengths, 8, 2, n_rot=0, seed=14, norm=False, outlier_frac=0)
    w.update(gate=True, theta=1e7)
    cu = w["cu_seqlens"]
    q = w["qkv"].clone()
    r0 = int(cu[1])
    q[r0 + 9, 2 * 8 * 256 + 2 * 256 + 17] = 1e5
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    out, _ = gpu_text(dict(w, qkv=q), ovf=ovf)
    clean, _ = gpu_text(w)
    want = np.zeros(int(cu[-1]), np.int32)
    want[r0] = 1
    assert np.array_equal(ovf.cpu().numpy(), want)
    assert torch.isfinite(out.float()).all()
    for r in (0, 2, 3):
        a, b = int(cu[r]), int(cu[r + 1])
        assert torch.equal(_bits(out[a:b]), _bits(clean[a:b])), f"record {r} changed"


@pytest.mark.parametrize("kind", ["inf_element", "wide_weights"])
def test_normalised_query_overflow(kind):
    """Normalised Q rows follow split16 too. An inf element in one query row (its sum of squares
    is inf) flags only its record and leaves every output finite. q_norm weights large enough
    that 16 max|w| passes f16's range switch the elementwise check on: with one weight of 1e6,
    that dim's normalised element passes 65504 in most rows (|x / rms| > 0.066), so every record
    is flagged."""
    _say(f"[split16] normalised q {kind}")
    lengths = [100, 150, 64, 200]
    nh, nkv, hd = 8, 2, 256
    w = workloads.text_inputs(lengths, nh, nkv, n_rot=64, seed=15, norm=True, outlier_frac=0)
    w.update(gate=True, theta=1e7)
    cu = w["cu_seqlens"]
    T = int(cu[-1])
    ovf = torch.zeros(T, dtype=torch.int32, device="cuda")
    clean, _ = gpu_text(w)
    if kind == "inf_element":
        q = w["qkv"].clone()
        r0 = int(cu[1])
        q[r0 + 7, 2 * hd + 11] = float("inf")     # head 1's query, record 1
        out, _ = gpu_text(dict(w, qkv=q), ovf=ovf)
        want = np.zeros(T, np.int32)
        want[r0] = 1
        assert np.array_equal(ovf.cpu().numpy(), want), np.nonzero(ovf.cpu().numpy())
        assert torch.isfinite(out.float()).all()
        for r in (0, 2, 3):
            a, b = int(cu[r]), int(cu[r + 1])
            assert torch.equal(_bits(out[a:b]), _bits(clean[a:b])), f"record {r} changed"
    else:
        qn = w["q_norm"].clone()
        qn[5] = 1e6
        out, _ = gpu_text(dict(w, q_norm=qn), ovf=ovf)
        flags = ovf.cpu().numpy()
        want = np.zeros(T, np.int32)
        want[np.asarray(cu[:-1])] = 1
        assert np.array_equal(flags, want), np.nonzero(flags)
        assert torch.isfinite(out.float()).all()
        # weights below the bound (here 1,000: 16,000 < 65504) flag nothing and change no bits
        # against a pass that takes the elementwise path only because of the bound
        ovf.zero_()
        qn[5] = 1000.0
        gpu_text(dict(w, q_norm=qn), ovf=ovf)
        assert not ovf.cpu().numpy().any()
