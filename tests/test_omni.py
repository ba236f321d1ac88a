"""Omni decoder attention (hd 128, FP32): the oracle's prep pinned against transformers' Qwen3-Omni
RMSNorm and interleaved M-RoPE, and on the GPU the checks of tests/test_omni_attention.m: FP64
prep and attention tolerances, packed-versus-single byte equality, flat scores, poisoned inputs
reported, the output guard, large positions, f32 angles and a long constant-value row."""
import numpy as np
import pytest
import torch

from cleffa_amd import _lib
from cleffa_amd.omni import OmniAttention, OmniPlan, omni_rope_table
from oracle import oracle

HF = "transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe"


def _hf_prep(qkv, nh, nkv, qn, kn, pos3, exact, theta=1e6, eps=1e-6):
    """Q, K through transformers' Qwen3-Omni modules: RMSNorm(head_dim), the interleaved M-RoPE
    frequency layout (mrope_section 24/20/20) and apply_rotary_pos_emb. exact: angles in float64."""
    import importlib
    hf = importlib.import_module(HF)
    T = qkv.shape[0]
    x = torch.from_numpy(qkv.astype(np.float32)).view(T, nh + 2 * nkv, 128)
    norm = hf.Qwen3OmniMoeThinkerTextRMSNorm(128, eps=eps)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(qn))
        q = norm(x[:, :nh]).double()
        norm.weight.copy_(torch.from_numpy(kn))
        k = norm(x[:, nh:nh + nkv]).double()
    if exact:
        inv = torch.tensor([theta ** (-2.0 * i / 128.0) for i in range(64)], dtype=torch.float64)
        pos = torch.from_numpy(pos3.T.astype(np.float64))            # (3, T)
    else:
        inv = (1.0 / (theta ** (torch.arange(0, 128, 2, dtype=torch.float) / 128))).float()
        pos = torch.from_numpy(pos3.T.astype(np.float32))
    freqs = pos[:, :, None] * inv[None, None, :]                     # (3, T, 64)
    freqs = hf.Qwen3OmniMoeThinkerTextRotaryEmbedding.apply_interleaved_mrope(None, freqs[:, None], [24, 20, 20])[0]
    emb = torch.cat((freqs, freqs), dim=-1).double()
    q, k = hf.apply_rotary_pos_emb(q, k, emb.cos(), emb.sin(), unsqueeze_dim=1)   # cos (T, 1, 128)
    return q.permute(1, 0, 2).numpy(), k.permute(1, 0, 2).numpy()


def _inputs(T, nh, nkv, seed, pos_max=3000):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((T, (nh + 2 * nkv) * 128)).astype(np.float32)
    qn = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    pos3 = rng.integers(0, pos_max, size=(T, 3)).astype(np.int32)
    return qkv, qn, kn, pos3


@pytest.mark.parametrize("exact", [True, False])
def test_oracle_prep_matches_transformers(exact):
    nh, nkv, T = 4, 2, 40
    qkv, qn, kn, pos3 = _inputs(T, nh, nkv, seed=1)
    inv = omni_rope_table(1e6)[:64]
    Q, K, V = oracle.omni_prep(qkv, nh, nkv, qn, kn, pos3, theta=1e6, exact=exact, inv_freq=inv)
    hq, hk = _hf_prep(qkv, nh, nkv, qn, kn, pos3, exact)
    assert np.abs(Q - hq).max() < 2e-6 and np.abs(K - hk).max() < 2e-6
    np.testing.assert_array_equal(V, qkv.reshape(T, nh + 2 * nkv, 128)[:, nh + nkv:].transpose(1, 0, 2))


def test_oracle_prep_axes_and_pairs():
    """Position (p, 0, 0) turns exactly the temporal pairs (i % 3 == 0 below 60, and 60-63); every
    pair (i, i + 64) keeps its length."""
    nh, nkv, T = 1, 1, 3
    qkv, qn, kn, _ = _inputs(T, nh, nkv, seed=2)
    Q0, _, _ = oracle.omni_prep(qkv, nh, nkv, qn, kn, np.zeros((T, 3), np.int32))
    for axis in range(3):
        pos = np.zeros((T, 3), np.int32)
        pos[:, axis] = 77
        Q, _, _ = oracle.omni_prep(qkv, nh, nkv, qn, kn, pos)
        moved = np.abs(Q[0] - Q0[0])[:, :64].max(0) > 1e-9
        want = np.array([(i < 60 and i % 3 == axis) or (i >= 60 and axis == 0) for i in range(64)])
        np.testing.assert_array_equal(moved, want)
        r0 = Q0[0][:, :64] ** 2 + Q0[0][:, 64:] ** 2
        r1 = Q[0][:, :64] ** 2 + Q[0][:, 64:] ** 2
        assert np.abs(r0 - r1).max() < 1e-12


def test_rope_table():
    t = omni_rope_table(1e6)
    f = 1e6 ** (-np.arange(64) * 2 / 128.0)
    assert np.abs(t[64:128].astype(np.float64) + t[128:].astype(np.float64) - f).max() <= 1e-15 * 1
    # the f32 table is C's 1 / powf(theta, 2j / 128) (clef_metal.m:177); libm's powf is within an ulp
    np.testing.assert_allclose(t[:64], 1.0 / 1e6 ** (np.arange(64) * 2 / 128.0), rtol=2.5e-7, atol=0)


def test_plan_blocks():
    p = OmniPlan([0, 33, 33, 40], device="cpu")
    b = p.blocks_host
    assert p.n_blk == 4 and (np.diff(b[:, 4]) <= 0).all()
    assert sorted(map(tuple, b[:, :5].tolist())) == [(0, 16, 0, 0, 16), (16, 16, 16, 0, 32), (32, 1, 32, 0, 33),
                                                      (33, 7, 0, 33, 7)]
    assert p.pairs() == 33 * 34 // 2 + 7 * 8 // 2


def test_abi_rejects_bad_heads():
    import ctypes
    lib = _lib.load()
    a = _lib.OmniAttnArgs()
    a.nh, a.nkv, a.T, a.kvT, a.scale, a.n_blk = 24, 4, 8, 40, 0.1, 1
    err = ctypes.create_string_buffer(256)
    assert not lib.clef_hip_omni_attention(ctypes.byref(a), None, err, 256)
    assert "head counts" in err.value.decode()
    a.nh, a.kvT = 32, 20
    assert not lib.clef_hip_omni_attention(ctypes.byref(a), None, err, 256)
    assert "kvT" in err.value.decode()


# ---------------------------------------------------------------- GPU: tests/test_omni_attention.m

def _sample(i):
    return (np.sin(np.asarray(i, dtype=np.float32) * np.float32(0.37)) * np.float32(0.7)).astype(np.float32)


def _run(length, packed, mode, rope_exact=True, pos_base=0):
    """One case of tests/test_omni_attention.m:run: nh 8, nkv 1; packed puts a 7-token record
    before and a 3-token record after. mode 1 sharp norms, 2 flat scores, 3-5 a NaN / +inf / -inf
    input, 6 flat scores with constant V."""
    nh, nkv = 8, 1
    before, after = (7, 3) if packed else (0, 0)
    T, row = before + length + after, (nh + 2 * nkv) * 128
    starts = np.array([0 if t < before else before if t < before + length else before + length for t in range(T)])
    local = np.arange(T) - starts
    norms = ((8.0 if mode == 1 else 1.0) + _sample(np.arange(256) + 3) * np.float32(0.2)).astype(np.float32)
    qkv = _sample(local[:, None] * row + np.arange(row)[None, :])
    if mode in (2, 6):
        qkv[:, :(nh + nkv) * 128] = 0
    if mode == 6:
        qkv[:, (nh + nkv) * 128:] = (np.float32(0.1234567) + np.arange(128, dtype=np.float32) * np.float32(1e-4))
    if 3 <= mode <= 5:
        qkv[before + length - 1, 0] = {3: np.nan, 4: np.inf, 5: -np.inf}[mode]
    pos3 = np.stack([pos_base + local + 5, pos_base + 2 * local + 1, pos_base + 3 * local + 2], 1).astype(np.int32)
    cu = np.array(sorted({0, before, before + length, T}), np.int32)
    att = OmniAttention(nh, nkv, theta=1e6, rope_exact=rope_exact)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    plan = OmniPlan(cu)
    out = torch.full((T * nh * 128 + 32,), float("nan"), device="cuda")
    o = out[: T * nh * 128].view(T, nh * 128)
    Q, K, V, status = att.prep(d(qkv), d(norms[:128]), d(norms[128:]), d(pos3))
    att.attention(Q, K, V, plan, out=o)
    torch.cuda.synchronize()
    return dict(qkv=qkv, norms=norms, pos3=pos3, cu=cu, before=before, T=T, nh=nh, nkv=nkv,
                Q=Q.cpu().numpy(), K=K.cpu().numpy(), out=out.cpu().numpy(), status=int(status.item()))


def _check_fp64(r, length, sharp, rope_exact):
    nh, nkv, T, before = r["nh"], r["nkv"], r["T"], r["before"]
    inv = omni_rope_table(1e6)[:64]
    Q, K, V = oracle.omni_prep(r["qkv"], nh, nkv, r["norms"][:128], r["norms"][128:], r["pos3"], theta=1e6,
                               exact=rope_exact, inv_freq=inv)
    tol = 1e-5 if sharp else 2e-6
    assert np.abs(r["Q"][:, :T] - Q).max() < tol, "RMS/RoPE mismatch (Q)"
    assert np.abs(r["K"][:, :T] - K).max() < tol, "RMS/RoPE mismatch (K)"
    assert (r["K"][:, T:T + 32] == 0).all(), "kv slack rows not zeroed"
    want = oracle.attention(Q, K, V, r["cu"], None, True, 128 ** -0.5, None)
    got = r["out"][: T * nh * 128].reshape(T, nh * 128)
    err = np.abs(got[before:before + length] - want[before:before + length]).max()
    assert np.isfinite(got).all() and err < (3e-4 if sharp else 3e-6), f"attention FP64 max err {err:.3g}"
    assert np.isnan(r["out"][T * nh * 128:]).all(), "output guard overwritten"
    return err


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_omni_fp64_and_packing(mode):
    print(f"[omni] mode {mode}", flush=True)
    for length in (1, 31, 32, 33, 127, 128, 129):
        single, packed = _run(length, False, mode), _run(length, True, mode)
        assert single["status"] == 0 and packed["status"] == 0
        _check_fp64(single, length, mode == 1, True)
        _check_fp64(packed, length, mode == 1, True)
        n = length * 8 * 128
        b = packed["before"] * 8 * 128
        assert np.array_equal(single["out"][:n].view(np.uint32), packed["out"][b:b + n].view(np.uint32)), \
            f"packing changed output bytes at length {length}"


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [3, 4, 5])
def test_omni_nonfinite_reported(mode):
    print(f"[omni] poison mode {mode}", flush=True)
    for length, packed in ((1, False), (33, True)):
        r = _run(length, packed, mode)
        t = r["before"] + length - 1
        assert not np.isfinite(r["Q"][0, t, 0]), "non-finite Q was hidden"
        assert r["status"] != 0, "non-finite attention was not reported"


@pytest.mark.gpu
def test_omni_large_positions_and_f32_angles():
    print("[omni] large positions", flush=True)
    for mode in (0, 1):
        for length in (1, 65, 129):
            single, packed = _run(length, False, mode, pos_base=65000), _run(length, True, mode, pos_base=65000)
            _check_fp64(single, length, mode == 1, True)
            n, b = length * 8 * 128, packed["before"] * 8 * 128
            assert np.array_equal(single["out"][:n].view(np.uint32), packed["out"][b:b + n].view(np.uint32))
    _check_fp64(_run(33, False, 0, rope_exact=False), 33, False, False)
    _check_fp64(_run(33, True, 1, rope_exact=False), 33, True, False)


@pytest.mark.gpu
def test_omni_long_flat():
    """8,193 keys of one constant V row: every output equals that row within 6e-8, and the
    packed run matches the single one byte for byte."""
    print("[omni] long flat", flush=True)
    res = []
    for packed in (False, True):
        r = _run(8193, packed, 6)
        T, b = r["T"], r["before"]
        got = r["out"][: T * 8 * 128].reshape(T, 8, 128)[b:b + 8193]
        want = r["qkv"][b, (8 + 1) * 128:]
        assert np.abs(got - want[None, None, :]).max() < 6e-8, "long accumulation lost constant values"
        res.append(got.copy())
    assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))
