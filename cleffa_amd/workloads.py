"""Seeded synthetic workloads for the prefill attention path (the BASELINE configurations).

C0  one causal sequence of 1,024 tokens, 16/4 heads, hd 256, plain SDPA operands (no norm,
    no rotary, no gate), Q/K/V ~ N(0,1) rounded to bf16.
C1  packed varlen causal micro-batch: 8 records, lengths ~ U[64,1024] rescaled to 4,096 tokens,
    24/4 heads, hd 256, q/k RMSNorm weights 1+N(0,0.1), rotary on 64 dims (theta 1e7),
    sigmoid gate logits N(0,1), Q/K ~ N(0,1) with 2% of channels x8.
C2  one causal request of 16,384 tokens, 24/4, same prologue/epilogue as C1.
C3  prefix-cache continuation: 4 records x (2,048 cached K/V rows + 512 new queries at
    positions 2,048..2,559), 16/4 heads, hd 256.
C4  vision: 4 images x 1,024 patches (32x32 grid), bidirectional, 16 heads, hd 72, 2-D rotary.
S   a batch of short records: 256 records x 16 tokens (4,096 tokens), 24/4 heads, hd 256, C1's
    prologue and gate (not a BASELINE configuration: the serving case of many short prompts).

Record lengths come from a numpy PCG64 stream so they are identical on every machine; the
tensor values come from a torch generator on the target device.
"""
import numpy as np
import torch

from .attention import vision_positions


def c1_lengths(seed=0, n=8, total=4096, lo=64, hi=1024):
    """n lengths drawn uniform in [lo, hi], rescaled to sum to exactly `total`."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(lo, hi + 1, size=n).astype(np.float64)
    exact = raw * total / raw.sum()
    lengths = np.maximum(np.floor(exact).astype(np.int64), 1)
    short = total - int(lengths.sum())
    order = np.argsort(-(exact - np.floor(exact)), kind="stable")
    for i in range(abs(short)):
        lengths[order[i % n]] += 1 if short > 0 else -1
    assert int(lengths.sum()) == total
    return [int(x) for x in lengths]


def cu_seqlens(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def column_scales(nh, nkv, hd, seed, outlier_frac=0.02, outlier_scale=8.0):
    """Per-column scale of the qkv rows: 1, or outlier_scale on a random outlier_frac of the query
    and key channels."""
    row = 2 * nh * hd + 2 * nkv * hd
    rng = np.random.default_rng(seed + 7)
    cols = np.zeros(row, dtype=np.float32) + 1.0
    qcols = (np.arange(nh)[:, None] * 2 * hd + np.arange(hd)[None, :]).ravel()
    kcols = 2 * nh * hd + np.arange(nkv * hd)
    for c in (qcols, kcols):
        pick = rng.random(c.size) < outlier_frac
        cols[c[pick]] = outlier_scale
    return cols


def qkv_projection(T, nh, nkv, hd=256, H=5120, seed=0, device="cpu", outlier_frac=0.02, outlier_scale=8.0):
    """Operands of the QKV GEMM whose product has the distribution text_inputs gives the qkv rows
    directly: X [T][H] ~ N(0, 1) and W [row][H] ~ N(0, 1 / H) (so each product entry is about
    N(0, 1)), with the same outlier channels scaled. Both bf16."""
    g = _gen(device, seed + 101)
    X = torch.randn((T, H), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    W = torch.randn((2 * nh * hd + 2 * nkv * hd, H), generator=g, device=device, dtype=torch.float32) * H ** -0.5
    if outlier_frac > 0:
        W *= torch.from_numpy(column_scales(nh, nkv, hd, seed, outlier_frac, outlier_scale)).to(device)[:, None]
    return X, W.to(torch.bfloat16)


def text_inputs(lengths, nh, nkv, hd=256, n_rot=64, seed=0, device="cpu", norm=True,
                outlier_frac=0.02, outlier_scale=8.0, positions=None):
    """Fused qkv rows [T][2*nh*hd + 2*nkv*hd] (bf16), norm weights, pos3 and cu_seqlens.
    positions: [T] (one position per token) or [T][3] (temporal, row, column)."""
    T = int(sum(lengths))
    row = 2 * nh * hd + 2 * nkv * hd
    g = _gen(device, seed)
    qkv = torch.randn((T, row), generator=g, device=device, dtype=torch.float32)
    if outlier_frac > 0:
        qkv *= torch.from_numpy(column_scales(nh, nkv, hd, seed, outlier_frac, outlier_scale)).to(device)
    qkv = qkv.to(torch.bfloat16)
    q_norm = k_norm = None
    if norm:
        q_norm = (1.0 + 0.1 * torch.randn((hd,), generator=g, device=device)).float()
        k_norm = (1.0 + 0.1 * torch.randn((hd,), generator=g, device=device)).float()
    if positions is None:
        positions = np.concatenate([np.arange(n) for n in lengths]) if T else np.zeros(0)
    positions = np.asarray(positions, dtype=np.int32)
    if positions.ndim == 1:   # text tokens: the same position on all three M-RoPE axes
        positions = np.repeat(positions[:, None], 3, axis=1)
    pos3 = torch.from_numpy(np.ascontiguousarray(positions)).to(device)
    return {"qkv": qkv, "q_norm": q_norm, "k_norm": k_norm, "pos3": pos3,
            "cu_seqlens": cu_seqlens(lengths), "lengths": list(lengths), "nh": nh, "nkv": nkv,
            "hd": hd, "n_rot": n_rot, "row": row}


def config(name, seed=0, device="cpu"):
    """Inputs of one BASELINE configuration."""
    if name == "C0":
        w = text_inputs([1024], 16, 4, n_rot=0, seed=seed, device=device, norm=False, outlier_frac=0)
        w.update(gate=False, theta=1e7)
        return w
    if name == "C1":
        w = text_inputs(c1_lengths(seed), 24, 4, seed=seed, device=device)
        w.update(gate=True, theta=1e7)
        return w
    if name == "C2":
        w = text_inputs([16384], 24, 4, seed=seed, device=device, outlier_frac=0)
        w.update(gate=True, theta=1e7)
        return w
    if name == "S":
        w = text_inputs([16] * 256, 24, 4, seed=seed, device=device)
        w.update(gate=True, theta=1e7)
        return w
    if name == "C3":
        return prefix_inputs(seed=seed, device=device)
    if name == "C4":
        return vision_inputs(seed=seed, device=device)
    raise KeyError(name)


def prefix_inputs(n_req=4, cached=2048, new=512, nh=16, nkv=4, hd=256, seed=0, device="cpu"):
    """C3: cached K/V rows (already normalised and rotated) plus the new tokens' qkv rows."""
    w = text_inputs([new] * n_req, nh, nkv, hd=hd, seed=seed, device=device, outlier_frac=0,
                    positions=np.concatenate([cached + np.arange(new)] * n_req))
    g = _gen(device, seed + 1)
    # cached keys and values in the plane layouts: K [nkv][Tk][hd], V [nkv][Tk][hd]
    Tk = n_req * (cached + new)
    w["k_cache"] = torch.randn((nkv, Tk, hd), generator=g, device=device).to(torch.bfloat16)
    w["v_cache"] = torch.randn((nkv, Tk, hd), generator=g, device=device).to(torch.bfloat16)
    w["cu_seqlens_k"] = cu_seqlens([cached + new] * n_req)
    w.update(gate=True, theta=1e7, cached=cached, new=new)
    return w


def vision_inputs(n_img=4, grid=32, heads=16, hd=72, seed=0, device="cpu", bias=True):
    """C4: packed images' qkv rows [P][3*heads*hd] (bf16) + bias, cu_seqlens, (row, col) positions."""
    P = n_img * grid * grid
    E = heads * hd
    g = _gen(device, seed)
    qkv = torch.randn((P, 3 * E), generator=g, device=device).to(torch.bfloat16)
    b = (0.1 * torch.randn((3 * E,), generator=g, device=device)).float() if bias else None
    cu = cu_seqlens([grid * grid] * n_img)
    pos2 = vision_positions(cu, [grid] * n_img, merge=2)
    return {"qkv": qkv, "bias": b, "pos2": torch.from_numpy(pos2.copy()).to(device), "cu_seqlens": cu,
            "heads": heads, "hd": hd, "grid": grid, "n_img": n_img}


def flops(pairs, hd, nh):
    """Algorithmic attention flops: QK^T and PV, 2 flops per multiply-add each."""
    return 4.0 * hd * nh * pairs
