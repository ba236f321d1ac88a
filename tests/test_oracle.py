"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the HIP path's checker:
against the golden fixtures (PyTorch float64 SDPA + transformers Qwen3.5 modules), against
PyTorch SDPA at runtime on the shapes of the reference's own attention tests
(tests/test_safe_attn.py), and against closed forms (constant values, single key, uniform
scores, row sums)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from cleffa_amd import rope_inv_freq, vision_positions
from oracle import oracle

GOLD = Path(__file__).resolve().parent / "golden"


def _bf16(bits):
    return torch.from_numpy(np.asarray(bits).view(np.int16)).view(torch.bfloat16).float().numpy()


def _text_oracle(z, precision="f64"):
    qkv = _bf16(z["qkv"])
    nh, nkv, hd, n_rot = int(z["nh"]), int(z["nkv"]), int(z["hd"]), int(z["n_rot"])
    qn = z["q_norm"] if z["q_norm"].size else None
    kn = z["k_norm"] if z["k_norm"].size else None
    inv = rope_inv_freq(float(z["theta"]), n_rot) if n_rot else None
    return oracle.text_prep(qkv, nh, nkv, hd, n_rot, qn, kn, z["pos3"], inv, precision=precision)


@pytest.mark.parametrize("name", ["text_gated_small", "text_plain_small"])
def test_text_golden(name):
    z = np.load(GOLD / f"{name}.npz")
    Q, K, V, G = _text_oracle(z)
    hd = int(z["hd"])
    O = oracle.attention(Q, K, V, z["cu_seqlens"], None, True, hd ** -0.5, G if int(z["gate"]) else None)
    # the fixtures' prologue runs in float32 (HF RMSNorm and rotary), the oracle in float64
    np.testing.assert_allclose(O, z["out"], atol=2e-5, rtol=1e-4)


def test_prefix_golden():
    z = np.load(GOLD / "prefix_small.npz")
    Q, Kn, Vn, G = _text_oracle(z)
    K = _bf16(z["k_cache"]).astype(np.float64)
    V = _bf16(z["v_cache"]).astype(np.float64)
    cq, ck, cached = z["cu_seqlens"], z["cu_seqlens_k"], z["cached"]
    for r in range(len(cq) - 1):
        n = cq[r + 1] - cq[r]
        K[:, ck[r] + cached[r]: ck[r] + cached[r] + n] = Kn[:, cq[r]:cq[r + 1]]
        V[:, ck[r] + cached[r]: ck[r] + cached[r] + n] = Vn[:, cq[r]:cq[r + 1]]
    O = oracle.attention(Q, K, V, cq, ck, True, 1 / 16, G)
    np.testing.assert_allclose(O, z["out"], atol=2e-5, rtol=1e-4)


def test_vision_golden():
    z = np.load(GOLD / "vision_small.npz")
    heads, hd = int(z["heads"]), int(z["hd"])
    pos2 = vision_positions(z["cu_seqlens"], z["grid_w"], 2)
    np.testing.assert_array_equal(pos2, z["pos2"])
    Q, K, V = oracle.vis_prep(_bf16(z["qkv"]), heads, hd, z["bias"], pos2, rope_inv_freq(10000.0, hd // 2))
    O = oracle.attention(Q, K, V, z["cu_seqlens"], None, False, hd ** -0.5, None)
    np.testing.assert_allclose(O, z["out"], atol=2e-5, rtol=1e-4)


def _sdpa_ref(q, k, v, causal, offset=0):
    """float64 torch SDPA with GQA; causal keeps key <= offset + query."""
    nq, nk = q.shape[2], k.shape[2]
    mask = None
    if causal:
        mask = torch.arange(nk)[None, :] <= offset + torch.arange(nq)[:, None]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)


@pytest.mark.parametrize("nq,nk,causal", [(19, 19, True), (17, 19, False), (9, 9, True), (15, 23, True)])
def test_attention_vs_torch_sdpa(nq, nk, causal):
    """Shapes of tests/test_safe_attn.py (16 q heads over 2 KV heads, hd 8, seeds 5/7/83). With
    nq < nk the queries are a record's last tokens (prefix semantics, metal/clef.metal:709-849)."""
    torch.manual_seed(5)
    q = torch.randn(1, 16, nq, 8, dtype=torch.float64)
    k, v = (torch.randn(1, 2, nk, 8, dtype=torch.float64) for _ in range(2))
    want = _sdpa_ref(q, k, v, causal, nk - nq)[0].transpose(0, 1).reshape(nq, 16 * 8).numpy()
    got = oracle.attention(q[0].numpy(), k[0].numpy(), v[0].numpy(), np.array([0, nq], np.int32),
                           np.array([0, nk], np.int32), causal, 8 ** -0.5)
    np.testing.assert_allclose(got, want, atol=1e-12, rtol=1e-12)


def test_packed_records_match_separate_sdpa():
    torch.manual_seed(83)
    lengths = [1, 7, 19, 3]
    T = sum(lengths)
    q = torch.randn(8, T, 16, dtype=torch.float64)
    k, v = (torch.randn(2, T, 16, dtype=torch.float64) for _ in range(2))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    got = oracle.attention(q.numpy(), k.numpy(), v.numpy(), cu, None, True, 0.25)
    for r in range(len(lengths)):
        a, b = cu[r], cu[r + 1]
        want = _sdpa_ref(q[None, :, a:b], k[None, :, a:b], v[None, :, a:b], True)
        np.testing.assert_allclose(got[a:b], want[0].transpose(0, 1).reshape(b - a, -1).numpy(), atol=1e-12)


def test_constant_values_long_reduction():
    """test_safe_attn.py: uniform scores over 64,000 keys with V = 0.1 give exactly 0.1."""
    q = np.zeros((8, 1, 16))
    k = np.zeros((1, 64000, 16))
    v = np.full((1, 64000, 16), 0.1)
    got = oracle.attention(q, k, v, np.array([0, 1], np.int32), np.array([0, 64000], np.int32), False, 0.25)
    np.testing.assert_allclose(got, 0.1, atol=2e-12)


def test_closed_forms():
    rng = np.random.default_rng(1)
    # one key: output = that value times sigmoid(gate)
    q = rng.normal(size=(4, 1, 32)); k = rng.normal(size=(2, 1, 32)); v = rng.normal(size=(2, 1, 32))
    g = rng.normal(size=(1, 4 * 32))
    got = oracle.attention(q, k, v, np.array([0, 1], np.int32), None, True, 0.1, g)
    want = np.concatenate([v[h // 2, 0] for h in range(4)]) / (1 + np.exp(-g[0]))
    np.testing.assert_allclose(got[0], want, rtol=1e-13)
    # equal scores: the mean of the visible values
    T = 9
    q = np.zeros((2, T, 8)); k = rng.normal(size=(1, T, 8)); v = rng.normal(size=(1, T, 8))
    got = oracle.attention(q, k, v, np.array([0, T], np.int32), None, True, 1.0)
    for t in range(T):
        np.testing.assert_allclose(got[t, :8], v[0, : t + 1].mean(0), rtol=1e-12)
    # rows sum to one: V = 1
    q = rng.normal(size=(4, T, 8)) * 5; k = rng.normal(size=(2, T, 8)); v = np.ones((2, T, 8))
    got = oracle.attention(q, k, v, np.array([0, T], np.int32), None, True, 1.0)
    np.testing.assert_allclose(got, 1.0, atol=1e-14)


def test_text_prologue_matches_hf_at_long_positions():
    """RMSNorm (1+w folded), interleaved M-RoPE on 64 of 256 dims, positions up to 16,383."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    torch.manual_seed(3)
    nh, nkv, hd, T = 2, 1, 256, 6
    qkv = torch.randn(T, 2 * nh * hd + 2 * nkv * hd).to(torch.bfloat16).float()
    w = 0.1 * torch.randn(hd)
    pos = np.array([[0, 0, 0], [1, 5, 9], [700, 701, 702], [8191, 8000, 17], [16383, 2, 16383], [12, 12, 12]], np.int32)
    Q, K, V, G = oracle.text_prep(qkv.numpy(), nh, nkv, hd, 64, (1 + w).numpy(), (1 + w).numpy(), pos,
                                  rope_inv_freq(1e7, 64))
    cfg = Qwen3_5TextConfig(head_dim=hd, rope_parameters={"rope_type": "default", "rope_theta": 1e7,
                                                          "partial_rotary_factor": 0.25, "mrope_section": [11, 11, 10]})
    norm = hf.Qwen3_5RMSNorm(hd, eps=1e-6)
    norm.weight.data = w
    with torch.no_grad():
        q = norm(qkv[:, : 2 * nh * hd].view(T, nh, 2 * hd)[..., :hd]).transpose(0, 1)[None]
        k = norm(qkv[:, 2 * nh * hd: 2 * nh * hd + hd].view(T, 1, hd)).transpose(0, 1)[None]
        cos, sin = hf.Qwen3_5TextRotaryEmbedding(cfg)(q, torch.from_numpy(pos.T.copy()).long()[:, None, :])
        q, k = hf.apply_rotary_pos_emb(q, k, cos, sin)
    np.testing.assert_allclose(Q, q[0].double().numpy(), atol=5e-5)
    np.testing.assert_allclose(K, k[0].double().numpy(), atol=5e-5)
    np.testing.assert_array_equal(V[0], qkv[:, 2 * nh * hd + hd:].numpy())
    np.testing.assert_array_equal(G.reshape(T, nh, hd), qkv[:, : 2 * nh * hd].view(T, nh, 2 * hd)[..., hd:].numpy())


def test_rope_tables_match_hf():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(head_dim=256, rope_parameters={"rope_type": "default", "rope_theta": 1e7,
                                                           "partial_rotary_factor": 0.25})
    want = hf.Qwen3_5TextRotaryEmbedding(cfg).inv_freq.numpy()
    np.testing.assert_allclose(rope_inv_freq(1e7, 64), want, rtol=3e-7)
    want = hf.Qwen3_5VisionRotaryEmbedding(36).inv_freq.numpy()
    np.testing.assert_allclose(rope_inv_freq(10000.0, 36), want, rtol=3e-7)


def test_vision_positions_match_hf():
    from transformers.vision_utils import get_vision_position_ids
    grids = [(4, 6), (2, 2), (32, 32)]
    cu = np.concatenate([[0], np.cumsum([h * w for h, w in grids])]).astype(np.int32)
    got = vision_positions(cu, [w for _, w in grids], 2)
    want = get_vision_position_ids(torch.tensor([[1, h, w] for h, w in grids]), 2).numpy()
    np.testing.assert_array_equal(got, want)


def test_f32_flavour_tracks_f64():
    z = np.load(GOLD / "text_gated_small.npz")
    Q, K, V, G = _text_oracle(z, "f32")
    O32 = oracle.attention(Q, K, V, z["cu_seqlens"], None, True, 1 / 16, G, precision="f32")
    np.testing.assert_allclose(O32, z["out"], atol=5e-5)
