"""Seeded sweep over random packed passes, each against the float64 oracle: record counts and
lengths (1 to 700 tokens, so ragged blocks, one-token records and records under and over one
128-row block), GQA geometries, with and without the q/k norms, rotary and gate, and host
schedules over random workgroup counts (so passes with fewer items than workgroups split their
blocks in halves, and others do not). Every case is also run with one workgroup per item and
must give the same bytes. Random prefix passes must reproduce a full pass's rows bitwise, and
random image mixes the vision oracle (bench/attention_bench.m:263-360 and
bench/vision_attention_bench.m:126-177 vary the layout in the same spirit)."""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, VisionAttention, rope_inv_freq, vision_positions, workloads
from oracle import oracle
from tests.helpers import assert_close, oracle_text

pytestmark = pytest.mark.gpu

GEOMETRIES = [(24, 4), (16, 4), (8, 2), (4, 1), (6, 2), (12, 4), (16, 8), (10, 5), (32, 4), (8, 8), (2, 1)]


def _say(*a):
    print(*a, flush=True)


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 6))
    lengths = [int(x) for x in rng.choice([1, 2, 15, 64, 65, 127, 128, 129, 200, 300, 700], size=n)]
    if sum(lengths) > 900:
        lengths = lengths[:1]
    nh, nkv = GEOMETRIES[int(rng.integers(len(GEOMETRIES)))]
    norm = bool(rng.integers(2))
    n_rot = 64 if norm and rng.integers(3) else 0
    gate = bool(rng.integers(2))
    n_wg = int(rng.choice([8, 37, 64, 256, 1000]))
    return lengths, nh, nkv, norm, n_rot, gate, n_wg


@pytest.mark.parametrize("seed", range(40))
def test_random_text_pass(seed):
    lengths, nh, nkv, norm, n_rot, gate, n_wg = _case(seed)
    _say(f"[sweep] seed {seed}: lengths {lengths} heads {nh}/{nkv} norm {norm} rot {n_rot} gate {gate} n_wg {n_wg}")
    w = workloads.text_inputs(lengths, nh, nkv, n_rot=n_rot, seed=seed, norm=norm, outlier_frac=0.0 if not norm else 0.02)
    w.update(gate=gate, theta=1e7)
    att = TextAttention(nh, nkv, 256, n_rot, rope_theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    d = lambda t: None if t is None else t.cuda()
    args = (d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan)
    sched = att.forward(*args, gate=gate, schedule=n_wg)
    whole = att.forward(*args, gate=gate, schedule=False)
    torch.cuda.synchronize()
    assert torch.equal(sched.view(torch.int16), whole.view(torch.int16)), "schedule and static order differ"
    assert_close(sched.float().cpu().numpy(), oracle_text(w), what=f"seed {seed}")


@pytest.mark.parametrize("seed", range(10))
def test_random_prefix_pass_equals_full_pass(seed):
    """Records whose first rows are already in the planes (a prefix pass: each record's last
    tokens as queries, all its tokens as keys) give bitwise the rows of the full pass that wrote
    those planes (tests/test_prefix_attention.m semantics)."""
    rng = np.random.default_rng(2000 + seed)
    n = int(rng.integers(1, 4))
    nh, nkv = GEOMETRIES[int(rng.integers(len(GEOMETRIES)))]
    # key offsets must be multiples of 8: every record but the last is a multiple of 8 long
    full = [8 * int(rng.integers(2, 50)) for _ in range(n - 1)] + [int(rng.integers(9, 400))]
    new = [int(rng.integers(1, f)) for f in full]
    n_wg = int(rng.choice([8, 37, 256]))   # few workgroups: small blocks packed; many: split
    _say(f"[sweep] prefix seed {seed}: full {full} new {new} heads {nh}/{nkv} n_wg {n_wg}")
    w = workloads.text_inputs(full, nh, nkv, seed=seed)
    att = TextAttention(nh, nkv, 256, 64, rope_theta=1e7)
    ck = np.concatenate([[0], np.cumsum(full)]).astype(np.int32)
    cq = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    plan_full, plan_new = AttnPlan(ck, ck, causal=True), AttnPlan(cq, ck, causal=True)
    kvT = max(plan_full.kvT, plan_new.kvT)
    kp, vt = att.planes(kvT)
    qkv, p3, qn, kn = w["qkv"].cuda(), w["pos3"].cuda(), w["q_norm"].cuda(), w["k_norm"].cuda()
    ref = att.forward(qkv, qn, kn, p3, plan_full, k_plane=kp, vt_plane=vt, kvT=kvT)
    pick = torch.from_numpy(np.concatenate([np.arange(ck[r + 1] - new[r], ck[r + 1]) for r in range(n)])).cuda()
    part = att.forward(qkv[pick].contiguous(), qn, kn, p3[pick].contiguous(), plan_new, k_plane=kp, vt_plane=vt,
                       kvT=kvT, schedule=n_wg)
    torch.cuda.synchronize()
    assert torch.equal(part.view(torch.int16), ref[pick].view(torch.int16))


@pytest.mark.parametrize("seed", range(4))
def test_random_vision_pass(seed):
    rng = np.random.default_rng(3000 + seed)
    n = int(rng.integers(1, 4))
    grids = [(2 * int(rng.integers(1, 9)), 2 * int(rng.integers(1, 9))) for _ in range(n)]
    heads = int(rng.choice([2, 4, 16]))
    _say(f"[sweep] vision seed {seed}: grids {grids} heads {heads}")
    hd = 72
    lens = [a * b for a, b in grids]
    P = sum(lens)
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn((P, 3 * heads * hd), generator=g).to(torch.bfloat16)
    bias = (0.1 * torch.randn((3 * heads * hd,), generator=g)).float() if seed % 2 else None
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pos2 = vision_positions(cu, [b for _, b in grids], 2)
    vis = VisionAttention(heads, hd)
    plan = AttnPlan(cu, causal=False)
    Q, K, V = oracle.vis_prep(qkv.float().numpy(), heads, hd, None if bias is None else bias.numpy(), pos2,
                              rope_inv_freq(10000.0, hd // 2))
    want = oracle.attention(Q, K, V, cu, None, False, hd ** -0.5, None)
    out = vis.forward(qkv.cuda(), None if bias is None else bias.cuda(), torch.from_numpy(pos2).cuda(), plan)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), want, what=f"vision seed {seed}")


@pytest.mark.parametrize("foreign", ["other_plan", "other_n_wg", "other_nkv"])
def test_foreign_schedule_runs_static_order(foreign):
    """A schedule built for another plan (same block count and heads, but short blocks that the
    other plan packs several heads to an item), for another workgroup count, or for another kv
    head count is refused by the kernel's header check: the pass runs the static order and gives
    bitwise the output of a pass without a schedule."""
    lengths, other = [40, 40, 200], [100, 100, 200]
    nh, nkv, n_wg = 24, 4, 64
    _say(f"[sweep] foreign schedule: {foreign}")
    w = workloads.text_inputs(lengths, nh, nkv, n_rot=64, seed=3)
    w.update(gate=True, theta=1e7)
    att = TextAttention(nh, nkv, 256, 64, rope_theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    alien = AttnPlan(np.concatenate([[0], np.cumsum(other)]).astype(np.int32), causal=True)
    assert alien.n_blk == plan.n_blk
    if foreign == "other_plan":
        plan.schedule = lambda nh_, nkv_, n: alien.schedule(nh_, nkv_, n)
    elif foreign == "other_n_wg":
        plan.schedule = lambda nh_, nkv_, n: AttnPlan.schedule(plan, nh_, nkv_, n + 8)
    else:
        plan.schedule = lambda nh_, nkv_, n: AttnPlan.schedule(plan, nh_, 2 * nkv_ if nkv_ < nh_ else nkv_, n)
    d = lambda t: t.cuda()
    args = (d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan)
    got = att.forward(*args, gate=True, schedule=n_wg)
    whole = att.forward(*args, gate=True, schedule=False)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), whole.view(torch.int16))
    assert_close(got.float().cpu().numpy(), oracle_text(w), what=f"foreign schedule {foreign}")
