"""The QKV projection with the fused K/V prologue (clef_hip_qkv_gemm), on the GPU:

- the product against a float64 product of the same bf16 operands, within the fp32 summation
  bound plus half a bf16 ulp of the rounding (as tests/test_gemm.py bounds the library GEMM);
- the planes, rope_cs and overflow flags its epilogue writes are bitwise those of the separate
  K/V prologue (clef_hip_attn_prep_kv) run on the same qkv rows, for fresh and prefix passes, so
  the attention core that follows gives bitwise the output of the unfused step;
- the whole fused step (GEMM, then core) against the float64 oracle at the bf16 tolerance.
"""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, workloads
from tests.helpers import assert_close, oracle_text

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _operands(T, H, nh, nkv, seed, scale=None):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    row = 2 * nh * 256 + 2 * nkv * 256
    X = torch.randn(T, H, generator=g, device="cuda").bfloat16()
    # weights scaled so that qkv entries are about N(0, 1), as the attention tests' inputs are
    W = ((scale or H ** -0.5) * torch.randn(row, H, generator=g, device="cuda")).bfloat16()
    return X, W


def _plan_inputs(lengths, nh, seed):
    w = workloads.text_inputs(lengths, nh, 1, seed=seed)   # norm weights and positions only
    return w["q_norm"].cuda(), w["k_norm"].cuda(), w["pos3"].cuda(), w["cu_seqlens"]


@pytest.mark.parametrize("T,H,nh,nkv", [(1, 64, 2, 1), (300, 1024, 8, 2), (4096, 5120, 24, 4), (777, 2048, 12, 4)])
def test_product_within_fp32_bound(T, H, nh, nkv):
    _say(f"[qkv_gemm] product T={T} H={H} heads {nh}/{nkv}")
    X, W = _operands(T, H, nh, nkv, seed=T + H)
    att = TextAttention(nh, nkv, 256, 64)
    plan = AttnPlan(np.array([0, T], np.int32), causal=True)
    qkv = att.project(X, W, plan, prologue=False)
    torch.cuda.synchronize()
    rows = torch.arange(T, device="cuda") if T <= 1024 else torch.randperm(T, device="cuda")[:512]
    ref = X[rows].double() @ W.double().T
    mag = X[rows].double().abs() @ W.double().abs().T
    bound = (H + 1) * 2.0 ** -24 * mag
    ulp = torch.where(ref.abs() > 0, 2.0 ** (torch.floor(torch.log2(ref.abs())) - 8), torch.zeros_like(ref))
    err = (qkv[rows].double() - ref).abs()
    assert (err <= bound + ulp).all(), f"max excess {(err - bound - ulp).max().item():.3g}"


def _prep_vs_fused(lengths, nh, nkv, H, seed, cu_k=None, big=None):
    q_norm, k_norm, pos3, cu = _plan_inputs(lengths, nh, seed)
    T = int(cu[-1])
    X, W = _operands(T, H, nh, nkv, seed)
    if big is not None:   # (pass row, "k" or "v"): that row's keys or values leave f16's range
        row, part = big
        c0 = 2 * nh * 256 + (0 if part == "k" else nkv * 256)
        X[row, 5] = 3e4
        W[c0:c0 + nkv * 256, 5] = 100.0
        q_norm = k_norm = None   # plain keys: normalised ones stay within 16 max|w|
    att = TextAttention(nh, nkv, 256, 64)
    plan = AttnPlan(cu, causal=True, cu_k=cu_k)
    kvT = plan.kvT
    fill = lambda dt, shape: torch.full(shape, 7.0, dtype=dt, device="cuda")
    # both pairs of planes start from the same contents, so rows the pass does not own must match too
    kp_f, vp_f = fill(torch.float16, (nkv, kvT, 256)), fill(torch.bfloat16, (nkv, 256, kvT))
    kp_u, vp_u = kp_f.clone(), vp_f.clone()
    cs_f, cs_u = att.rope_table(T), att.rope_table(T)
    ov_f = torch.zeros(T, dtype=torch.int32, device="cuda")
    ov_u = ov_f.clone()
    qkv = att.project(X, W, plan, q_norm, k_norm, pos3, k_plane=kp_f, vt_plane=vp_f, ovf=ov_f, rope_cs=cs_f)
    qkv_plain = att.project(X, W, plan, prologue=False)
    att.forward(qkv_plain, q_norm, k_norm, pos3, plan, k_plane=kp_u, vt_plane=vp_u, ovf=ov_u, rope_cs=cs_u, stage="prep")
    out_f = att.forward(qkv, q_norm, k_norm, pos3, plan, k_plane=kp_f, vt_plane=vp_f, rope_cs=cs_f, stage="core")
    out_u = att.forward(qkv_plain, q_norm, k_norm, pos3, plan, k_plane=kp_u, vt_plane=vp_u, rope_cs=cs_u, stage="core")
    torch.cuda.synchronize()
    assert torch.equal(qkv.view(torch.int16), qkv_plain.view(torch.int16)), "the product depends on the prologue"
    assert torch.equal(kp_f.view(torch.int16), kp_u.view(torch.int16)), "K planes differ"
    assert torch.equal(vp_f.view(torch.int16), vp_u.view(torch.int16)), "V^T planes differ"
    assert torch.equal(cs_f[:T], cs_u[:T]), "rope_cs differs"
    assert torch.equal(ov_f, ov_u), "overflow flags differ"
    assert torch.equal(out_f.view(torch.int16), out_u.view(torch.int16)), "core outputs differ"
    return qkv, out_f, ov_f, q_norm, k_norm, pos3, cu


@pytest.mark.parametrize("lengths,nh,nkv,H", [
    ([1160, 890, 730, 425, 472, 136, 179, 104], 24, 4, 1024),   # C1's records
    ([1, 2, 127, 128, 129, 300], 8, 2, 512),                     # ragged records, a 1-token one
    ([64], 4, 1, 256),
])
def test_fused_prologue_equals_separate_prologue(lengths, nh, nkv, H):
    _say(f"[qkv_gemm] fused vs separate prologue {lengths} heads {nh}/{nkv} H={H}")
    _prep_vs_fused(lengths, nh, nkv, H, seed=len(lengths))


def test_fused_prologue_prefix_pass_keeps_cached_rows():
    """A prefix pass: each record's new rows land after its cached rows (kv rows cu_k, each
    record's first a multiple of 8); the cached rows (here the fill value) are left as they are,
    as the separate prologue leaves them."""
    _say("[qkv_gemm] prefix pass")
    full = [8 * 25, 8 * 41, 293]
    new = [100, 37, 256]
    ck = np.concatenate([[0], np.cumsum(full)]).astype(np.int32)
    _prep_vs_fused(new, 8, 2, 512, seed=9, cu_k=ck)


@pytest.mark.parametrize("where", ["k", "v"])
def test_fused_prologue_overflow_flags(where):
    """An activation row that drives one record's keys or values past f16's range: both
    prologues flag the same record (at its first pass row) and saturate alike."""
    _say(f"[qkv_gemm] overflow in {where}")
    lengths = [100, 150, 64]
    row = 100 + 20
    _, _, ovf, *_ = _prep_vs_fused(lengths, 8, 2, 256, seed=3, big=(row, where))
    flags = ovf.cpu().numpy()
    assert flags[100] == 1 and flags.sum() == 1, np.nonzero(flags)


def test_fused_step_matches_oracle():
    """C1's records at 24/4 heads: qkv from the fused GEMM, then the core, against the float64
    oracle run on the same qkv rows, at the bf16 tolerance."""
    _say("[qkv_gemm] fused step vs oracle")
    lengths = [1160, 890, 730, 425, 472, 136, 179, 104]
    qkv, out, _, q_norm, k_norm, pos3, cu = _prep_vs_fused(lengths, 24, 4, 1024, seed=11)
    w = {"qkv": qkv.cpu(), "q_norm": q_norm.cpu(), "k_norm": k_norm.cpu(), "pos3": pos3.cpu(), "cu_seqlens": cu,
         "nh": 24, "nkv": 4, "hd": 256, "n_rot": 64, "gate": True, "theta": 1e7}
    rows = np.sort(np.random.default_rng(0).choice(int(cu[-1]), 256, replace=False))
    assert_close(out.float().cpu().numpy()[rows], oracle_text(w, rows=rows), what="fused step")
