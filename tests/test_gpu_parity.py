"""HIP path vs the float64 CPU oracle on the BASELINE configurations (bf16 outputs, north_star
tolerance max-abs 2e-2 / mean-abs 2e-3), through the C ABI (libclef_hip_attn.so)."""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, VisionAttention, rope_inv_freq, vision_positions, workloads
from oracle import oracle
from tests.helpers import assert_close, gpu_text, oracle_text

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("name", ["C0", "C1"])
def test_config_full(name):
    _say(f"[parity] {name} seed=0")
    w = workloads.config(name, seed=0)
    out, plan = gpu_text(w)
    want = oracle_text(w)
    mx, mean = assert_close(out.float().cpu().numpy(), want, what=name)
    _say(f"[parity] {name}: max_abs {mx:.3g} mean_abs {mean:.3g} blocks {plan.n_blk}")


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_c1_more_seeds(seed):
    """C1 at other seeds: its 2% outlier channels make some rows sharp, where bf16-rounded K
    scores miss the max-abs bound (0.022-0.024 on two of these seeds, in a CPU emulation) and
    the f16 Q/K operands keep it (0.008-0.013)."""
    _say(f"[parity] C1 seed={seed}")
    w = workloads.config("C1", seed=seed)
    out, _ = gpu_text(w)
    mx, mean = assert_close(out.float().cpu().numpy(), oracle_text(w), what=f"C1 seed {seed}")
    _say(f"[parity] C1 seed {seed}: max_abs {mx:.3g} mean_abs {mean:.3g}")


def test_c2_sampled_rows():
    """C2 (16,384-token causal request): float64 oracle on 96 sampled rows, every head."""
    _say("[parity] C2 sampled rows")
    w = workloads.config("C2", seed=0, device="cuda")
    out, _ = gpu_text(w)
    rng = np.random.default_rng(3)
    rows = np.unique(np.concatenate([[0, 1, 127, 128, 16383], rng.integers(0, 16384, 91)])).astype(np.int32)
    want = oracle_text(w, rows=rows)
    got = out.float().cpu().numpy()[rows]
    mx, mean = assert_close(got, want, what="C2")
    _say(f"[parity] C2: max_abs {mx:.3g} mean_abs {mean:.3g}")


def test_c3_prefix():
    _say("[parity] C3 prefix")
    w = workloads.config("C3", seed=0)
    nh, nkv, hd = w["nh"], w["nkv"], w["hd"]
    att = TextAttention(nh, nkv, hd, 64, rope_theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], w["cu_seqlens_k"], causal=True)
    kp = w["k_cache"].cuda().half().contiguous()   # the K plane is f16; bf16 values convert exactly
    vt = w["v_cache"].cuda().transpose(1, 2).contiguous()
    kvT = kp.shape[1]
    out = att.forward(w["qkv"].cuda(), w["q_norm"].cuda(), w["k_norm"].cuda(), w["pos3"].cuda(), plan,
                      k_plane=kp, vt_plane=vt, kvT=kvT)
    torch.cuda.synchronize()
    # oracle: the cache plus the new tokens' prepared K/V at their kv rows
    inv = rope_inv_freq(1e7, 64)
    Q, Kn, Vn, G = oracle.text_prep(w["qkv"].float().numpy(), nh, nkv, hd, 64, w["q_norm"].numpy(),
                                    w["k_norm"].numpy(), w["pos3"].numpy(), inv)
    K = w["k_cache"].double().numpy().copy()
    V = w["v_cache"].double().numpy().copy()
    cq, ck = w["cu_seqlens"], w["cu_seqlens_k"]
    for r in range(len(cq) - 1):
        n = cq[r + 1] - cq[r]
        dst = ck[r + 1] - n
        K[:, dst:dst + n] = Kn[:, cq[r]:cq[r] + n]
        V[:, dst:dst + n] = Vn[:, cq[r]:cq[r] + n]
    want = oracle.attention(Q, K, V, cq, ck, True, hd ** -0.5, G)
    mx, mean = assert_close(out.float().cpu().numpy(), want, what="C3")
    # the prologue wrote exactly the new rows into the cache and left the cached rows alone
    kp_h = kp.float().cpu().numpy()
    for r in range(len(cq) - 1):
        n = cq[r + 1] - cq[r]
        cached = ck[r + 1] - n - ck[r]
        assert np.array_equal(kp_h[:, ck[r]:ck[r] + cached], w["k_cache"].half().float().numpy()[:, ck[r]:ck[r] + cached])
    _say(f"[parity] C3: max_abs {mx:.3g} mean_abs {mean:.3g}")


def test_c4_vision():
    _say("[parity] C4 vision")
    w = workloads.config("C4", seed=0)
    heads, hd = w["heads"], w["hd"]
    vis = VisionAttention(heads, hd)
    plan = AttnPlan(w["cu_seqlens"], causal=False)
    out = vis.forward(w["qkv"].cuda(), w["bias"].cuda(), w["pos2"].cuda(), plan)
    torch.cuda.synchronize()
    Q, K, V = oracle.vis_prep(w["qkv"].float().numpy(), heads, hd, w["bias"].numpy(), w["pos2"].numpy(),
                              rope_inv_freq(10000.0, hd // 2))
    want = oracle.attention(Q, K, V, w["cu_seqlens"], None, False, hd ** -0.5, None)
    mx, mean = assert_close(out.float().cpu().numpy(), want, what="C4")
    _say(f"[parity] C4: max_abs {mx:.3g} mean_abs {mean:.3g}")


EDGE_LENGTHS = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 257, 300]


def test_edge_lengths_packed():
    _say("[parity] edge lengths")
    w = workloads.text_inputs(EDGE_LENGTHS, 8, 2, seed=11)
    w.update(gate=True, theta=1e7)
    out, _ = gpu_text(w)
    assert_close(out.float().cpu().numpy(), oracle_text(w), what="edge lengths")


@pytest.mark.parametrize("nh,nkv", [(16, 8), (10, 5)])
def test_more_than_four_kv_heads(nh, nkv):
    """More kv heads than the K/V prologue's K waves load at once (4): its second round of loads
    (8 kv heads), and a last round with one kv head (5), against float64."""
    _say(f"[parity] {nh}/{nkv} heads")
    w = workloads.text_inputs([1, 63, 130, 300], nh, nkv, seed=nh)
    w.update(gate=True, theta=1e7)
    out, _ = gpu_text(w)
    assert_close(out.float().cpu().numpy(), oracle_text(w), what=f"{nh}/{nkv}")


def test_text_bidirectional_packed():
    """A bidirectional text pass (plan causal=False) through the tensor core: each record's rows
    see all its keys, including the blocks of more than 64 rows that run as paired halves;
    against float64, and one-workgroup-per-item order bitwise equal to the scheduled grid."""
    _say("[parity] text bidirectional")
    w = workloads.text_inputs([200, 1, 65, 130], 12, 2, seed=21)
    w.update(gate=True, theta=1e7)
    out, _ = gpu_text(w, causal=False)
    assert_close(out.float().cpu().numpy(), oracle_text(w, causal=False), what="bidirectional")
    alone, _ = gpu_text(w, causal=False, schedule=False)
    assert torch.equal(out.cpu().view(torch.int16), alone.cpu().view(torch.int16))


def test_packing_invariance_bitwise():
    """Each record's output equals the same record run alone, bit for bit
    (bench/attention_bench.m:263-308)."""
    _say("[invariance] packing")
    lengths = [33, 1, 200, 64, 129, 7, 300]
    w = workloads.text_inputs(lengths, 8, 2, seed=5)
    w.update(gate=True, theta=1e7)
    packed, _ = gpu_text(w)
    packed = packed.cpu()
    cu = w["cu_seqlens"]
    for r, n in enumerate(lengths):
        a, b = int(cu[r]), int(cu[r + 1])
        alone = dict(w, qkv=w["qkv"][a:b].contiguous(), pos3=w["pos3"][a:b].contiguous(),
                     cu_seqlens=np.array([0, n], np.int32))
        out, _ = gpu_text(alone)
        assert torch.equal(out.cpu().view(torch.int16), packed[a:b].view(torch.int16)), f"record {r} differs"


def test_causal_no_leak():
    """Changing values after a cut leaves earlier outputs unchanged (ref/mps_sdpa_causal.py:51-65)."""
    _say("[invariance] causal leak")
    w = workloads.text_inputs([700], 8, 2, seed=9)
    w.update(gate=True, theta=1e7)
    base, _ = gpu_text(w)
    nh, nkv, hd = 8, 2, 256
    vcol = 2 * nh * hd + nkv * hd
    for cut in (1, 2, 7, 17, 350):
        q = w["qkv"].clone()
        q[cut:, vcol:] += 4
        out, _ = gpu_text(dict(w, qkv=q))
        assert torch.equal(out[:cut].cpu().view(torch.int16), base[:cut].cpu().view(torch.int16)), f"leak at cut {cut}"


def test_row_sums_exact():
    """With V = 1 and no gate, O = sum(P)/l = 1 to fp32 rounding: l sums the rounded P."""
    _say("[invariance] row sums")
    w = workloads.text_inputs([1000, 77, 513], 8, 2, seed=4)
    w.update(gate=False, theta=1e7)
    nh, nkv, hd = 8, 2, 256
    q = w["qkv"].clone()
    q[:, 2 * nh * hd + nkv * hd:] = 1.0
    out, _ = gpu_text(dict(w, qkv=q), out_dtype="f32")
    err = (out.double() - 1.0).abs().max().item()
    assert err <= 2e-6, err


def test_constant_values_and_single_token():
    _say("[invariance] constant V / T=1")
    w = workloads.text_inputs([1, 513], 8, 2, seed=8)
    w.update(gate=True, theta=1e7)
    nh, nkv, hd = 8, 2, 256
    q = w["qkv"].clone()
    vcol = 2 * nh * hd + nkv * hd
    q[:, vcol:] = 0.75
    out, _ = gpu_text(dict(w, qkv=q), out_dtype="f32")
    gate = torch.stack([q[:, h * 2 * hd + hd:h * 2 * hd + 2 * hd].float() for h in range(nh)], 1).reshape(q.shape[0], -1)
    want = 0.75 * torch.sigmoid(gate.double())
    assert (out.double().cpu() - want).abs().max().item() <= 1e-5


def test_bf16_is_rounded_f32():
    """bf16 output = round-to-nearest-even of the f32 output (vision_attention_bench.m:159-169)."""
    _say("[act16] bf16 rounding")
    w = workloads.text_inputs([300, 129], 8, 2, seed=2)
    w.update(gate=True, theta=1e7)
    f32, _ = gpu_text(w, out_dtype="f32")
    b16, _ = gpu_text(w, out_dtype="bf16")
    assert torch.equal(f32.to(torch.bfloat16).view(torch.int16), b16.view(torch.int16))
    f16, _ = gpu_text(w, out_dtype="f16")
    assert torch.equal(f32.to(torch.float16).view(torch.int16), f16.view(torch.int16))


def test_f16_overflow_flags_isolated():
    """Records whose output leaves f16 range are flagged at their first row and saturate; the
    other records' outputs are unchanged (bench/attention_bench.m:256-261)."""
    _say("[act16] overflow flags")
    lengths = [100, 150, 64, 200]
    w = workloads.text_inputs(lengths, 8, 2, seed=3)
    w.update(gate=False, theta=1e7)
    nh, nkv, hd = 8, 2, 256
    vcol = 2 * nh * hd + nkv * hd
    cu = w["cu_seqlens"]
    q = w["qkv"].clone()
    for r in (1, 3):
        q[cu[r]:cu[r + 1], vcol:] *= 1e5
    ovf = torch.zeros(int(cu[-1]), dtype=torch.int32, device="cuda")
    out, _ = gpu_text(dict(w, qkv=q), out_dtype="f16", ovf=ovf)
    clean, _ = gpu_text(w, out_dtype="f16")
    flags = ovf.cpu().numpy()
    want = np.zeros_like(flags)
    want[cu[1]] = want[cu[3]] = 1
    assert np.array_equal(flags, want)
    assert torch.isfinite(out.float()).all()
    for r in (0, 2):
        a, b = cu[r], cu[r + 1]
        assert torch.equal(out[a:b].view(torch.int16), clean[a:b].view(torch.int16))


def test_rope_table_accuracy():
    """cos/sin the K/V prologue writes for the Q prologue: within 2e-7 of float64 cos/sin of the
    float32 angle pos * inv_freq (the angle cleffa forms in float, clef.metal:282), for
    positions up to 16,383 on every interleaved M-RoPE axis."""
    _say("[parity] rope table")
    T = 4096
    rng = np.random.default_rng(9)
    pos = np.stack([np.arange(T) * 4 % 16384, rng.integers(0, 16384, T), np.arange(T)[::-1]], 1).astype(np.int32)
    w = workloads.text_inputs([T], 4, 1, seed=2, positions=pos)
    att = TextAttention(4, 1, 256, 64, rope_theta=1e7)
    plan = AttnPlan(w["cu_seqlens"], causal=True)
    cs = att.rope_table(T)
    att.forward(w["qkv"].cuda(), w["q_norm"].cuda(), w["k_norm"].cuda(), w["pos3"].cuda(), plan,
                stage="prep", rope_cs=cs)
    torch.cuda.synchronize()
    inv = rope_inv_freq(1e7, 64)
    ang = (pos[:, np.arange(32) % 3].astype(np.float32) * inv[None, :]).astype(np.float64)
    got = cs.cpu().numpy()
    assert np.abs(got[..., 0] - np.cos(ang)).max() <= 2e-7
    assert np.abs(got[..., 1] - np.sin(ang)).max() <= 2e-7


def test_vision_mixed_images_and_f16():
    """Images of different grids (2x2, 4x6, 6x10, 16x18: patch counts that are not multiples of
    16 or 64), no bias, bf16 and f16 outputs, against the float64 oracle."""
    _say("[parity] vision mixed grids")
    grids = [(2, 2), (4, 6), (6, 10), (16, 18)]
    heads, hd = 4, 72
    lens = [a * b for a, b in grids]
    P = sum(lens)
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn((P, 3 * heads * hd), generator=g).to(torch.bfloat16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pos2 = vision_positions(cu, [b for _, b in grids], 2)
    vis = VisionAttention(heads, hd)
    plan = AttnPlan(cu, causal=False)
    Q, K, V = oracle.vis_prep(qkv.float().numpy(), heads, hd, None, pos2, rope_inv_freq(10000.0, hd // 2))
    want = oracle.attention(Q, K, V, cu, None, False, hd ** -0.5, None)
    for dt in ("bf16", "f16"):
        out = vis.forward(qkv.cuda(), None, torch.from_numpy(pos2).cuda(), plan, out_dtype=dt)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), want, what=f"vision {dt}")


@pytest.mark.parametrize("nh,nkv,lengths", [
    (24, 4, [1160, 890, 730, 425, 472, 136, 179, 104]),   # C1 shape: 864 items over the CUs
    (12, 4, [300, 77, 1030]),                              # heads not a multiple of 8: plain snake order
    (4, 1, [40, 3]),                                       # fewer items than CUs
    (16, 4, [1024]),                                       # C0-like: every block split in halves
    (8, 2, [700, 130, 64, 65, 1]),                         # halves only for blocks > 64 rows
])
def test_persistent_grid_matches_one_item_per_workgroup(nh, nkv, lengths, monkeypatch):
    """The host schedule (clef_hip_attn_schedule over the CUs), the persistent grid's static
    order and one workgroup per item give the same bytes: each item's arithmetic does not depend
    on where or in which order it runs."""
    _say(f"[invariance] persistent grid nh={nh} nkv={nkv} lengths={lengths}")
    w = workloads.text_inputs(lengths, nh, nkv, seed=31)
    w.update(gate=True, theta=1e7)
    a, _ = gpu_text(w)                                   # host schedule
    monkeypatch.setenv("CLEF_HIP_TEXT_PERSISTENT", "1")
    b, _ = gpu_text(w, schedule=False)                   # persistent grid, static order
    monkeypatch.setenv("CLEF_HIP_TEXT_PERSISTENT", "0")
    c, _ = gpu_text(w, schedule=False)                   # one workgroup per item
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    if sum(lengths) <= 1500:
        assert_close(a.float().cpu().numpy(), oracle_text(w), what="persistent grid")
