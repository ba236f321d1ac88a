"""Shared test helpers: run the HIP path and the CPU oracle on the same inputs and compare."""
import numpy as np
import torch

from cleffa_amd import AttnPlan, TextAttention, VisionAttention, rope_inv_freq
from oracle import oracle

# north_star tolerance on bf16 outputs against the oracle (fp64 here, stricter than fp32)
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def bf16_round(x):
    """Round-to-nearest-even to bf16, returned as float32 (numpy)."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def oracle_text(w, rows=None, precision="f64", gate=None, causal=True):
    """Oracle output of a text workload dict (fresh pass), [T or rows][nh*hd]."""
    nh, nkv, hd, n_rot = w["nh"], w["nkv"], w["hd"], w["n_rot"]
    qkv = w["qkv"].float().cpu().numpy()
    inv = rope_inv_freq(w.get("theta", 1e7), n_rot) if n_rot else None
    qn = None if w["q_norm"] is None else w["q_norm"].cpu().numpy()
    kn = None if w["k_norm"] is None else w["k_norm"].cpu().numpy()
    Q, K, V, G = oracle.text_prep(qkv, nh, nkv, hd, n_rot, qn, kn, w["pos3"].cpu().numpy(), inv, precision=precision)
    use_gate = w.get("gate", True) if gate is None else gate
    return oracle.attention(Q, K, V, w["cu_seqlens"], None, causal, hd ** -0.5, G if use_gate else None,
                            rows=rows, precision=precision)


def gpu_text(w, out_dtype="bf16", gate=None, causal=True, ovf=None, device="cuda", f16_lim=65504.0,
             schedule=True):
    att = TextAttention(w["nh"], w["nkv"], w["hd"], w["n_rot"], rope_theta=w.get("theta", 1e7), device=device)
    plan = AttnPlan(w["cu_seqlens"], causal=causal, device=device)
    d = lambda t: None if t is None else t.to(device)
    out = att.forward(d(w["qkv"]), d(w["q_norm"]), d(w["k_norm"]), d(w["pos3"]), plan, out_dtype=out_dtype,
                      gate=w.get("gate", True) if gate is None else gate, ovf=ovf, f16_lim=f16_lim,
                      schedule=schedule)
    torch.cuda.synchronize()
    return out, plan


def errors(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    d = np.abs(got - want)
    return float(d.max()), float(d.mean())


def assert_close(got, want, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    mx, mean = errors(got, want)
    assert mx <= max_abs and mean <= mean_abs, f"{what}: max_abs {mx:.3g} (<= {max_abs}), mean_abs {mean:.3g} (<= {mean_abs})"
    return mx, mean
