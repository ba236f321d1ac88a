"""Writes the golden fixtures under tests/golden/ from independent library implementations.

The reference ships no golden vectors for its attention path (its tests build inputs with a hash
generator and check against a float64 loop, bench/attention_bench.m:93-104, 200-245). These
fixtures are computed with PyTorch's float64 scaled_dot_product_attention and the installed
transformers Qwen3.5 modules (Qwen3_5RMSNorm, Qwen3_5TextRotaryEmbedding with interleaved M-RoPE,
apply_rotary_pos_emb, Qwen3_5VisionRotaryEmbedding, get_vision_position_ids,
apply_rotary_pos_emb_vision) - the semantics cleffa's oracles run (ref/safe_attn.py,
ref/oracle.py) - and never with this repository's oracle, so they pin it.

Run from the repository root: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
from transformers.vision_utils import get_vision_position_ids

HERE = Path(__file__).resolve().parent


def bf16_bits(x):
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def rounded(x):
    return x.to(torch.bfloat16).to(torch.float32)


def text_prep(qkv, nh, nkv, hd, n_rot, w_q, w_k, pos3, theta):
    """HF Qwen3.5 gated attention prologue on fused rows [T][2*nh*hd + 2*nkv*hd] (float32)."""
    T = qkv.shape[0]
    qg = qkv[:, : 2 * nh * hd].view(T, nh, 2 * hd)
    q, gate = qg[..., :hd], qg[..., hd:].reshape(T, nh * hd)
    k = qkv[:, 2 * nh * hd: 2 * nh * hd + nkv * hd].view(T, nkv, hd)
    v = qkv[:, 2 * nh * hd + nkv * hd:].view(T, nkv, hd)
    if w_q is not None:
        qn, kn = hf.Qwen3_5RMSNorm(hd, eps=1e-6), hf.Qwen3_5RMSNorm(hd, eps=1e-6)
        qn.weight.data, kn.weight.data = w_q.clone(), w_k.clone()
        q, k = qn(q), kn(k)
    q, k = q.transpose(0, 1)[None], k.transpose(0, 1)[None]     # [1, heads, T, hd]
    if n_rot:
        cfg = Qwen3_5TextConfig(head_dim=hd, rope_parameters={
            "rope_type": "default", "rope_theta": theta, "partial_rotary_factor": n_rot / hd,
            "mrope_section": [11, 11, 10]})
        rot = hf.Qwen3_5TextRotaryEmbedding(cfg)
        cos, sin = rot(q, torch.from_numpy(pos3.T.copy()).long()[:, None, :])
        q, k = hf.apply_rotary_pos_emb(q, k, cos, sin)
    return q[0].double(), k[0].double(), v.transpose(0, 1).double(), gate.double()


def sdpa_records(Q, K, V, cu_q, cu_k, causal):
    """float64 SDPA per record (GQA); query j of a record with L cached keys sees keys <= L + j."""
    nh, hd = Q.shape[0], Q.shape[2]
    out = torch.zeros(Q.shape[1], nh * hd, dtype=torch.float64)
    for r in range(len(cu_q) - 1):
        q = Q[:, cu_q[r]:cu_q[r + 1]][None]
        k, v = K[:, cu_k[r]:cu_k[r + 1]][None], V[:, cu_k[r]:cu_k[r + 1]][None]
        nq, nk = q.shape[2], k.shape[2]
        mask = None
        if causal:
            mask = torch.arange(nk)[None, :] <= (nk - nq) + torch.arange(nq)[:, None]
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
        out[cu_q[r]:cu_q[r + 1]] = o[0].transpose(0, 1).reshape(nq, nh * hd)
    return out


def text_case(name, lengths, nh, nkv, n_rot, norm, gate, seed, positions=None):
    hd, theta = 256, 1e7
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    row = 2 * nh * hd + 2 * nkv * hd
    qkv = rounded(torch.randn(T, row, generator=g))
    w_q = 0.1 * torch.randn(hd, generator=g) if norm else None
    w_k = 0.1 * torch.randn(hd, generator=g) if norm else None
    if positions is None:
        # distinct temporal / row / column positions so the interleaved axis choice matters
        base = np.concatenate([np.arange(n) for n in lengths])
        positions = np.stack([base, 2 * base + 1, 3 * base + 2], 1)
    pos3 = np.ascontiguousarray(positions, dtype=np.int32)
    Q, K, V, G = text_prep(qkv, nh, nkv, hd, n_rot, w_q, w_k, pos3, theta)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    O = sdpa_records(Q, K, V, cu, cu, True)
    if gate:
        O = O * torch.sigmoid(G)
    np.savez_compressed(HERE / f"{name}.npz", qkv=bf16_bits(qkv), nh=nh, nkv=nkv, hd=hd, n_rot=n_rot,
                        theta=theta, gate=int(gate), cu_seqlens=cu, pos3=pos3,
                        q_norm=(1.0 + w_q).numpy().astype(np.float32) if norm else np.zeros(0, np.float32),
                        k_norm=(1.0 + w_k).numpy().astype(np.float32) if norm else np.zeros(0, np.float32),
                        out=O.numpy().astype(np.float32))


def prefix_case(name, cached, new, nh, nkv, seed):
    hd, n_rot, theta = 256, 64, 1e7
    g = torch.Generator().manual_seed(seed)
    row = 2 * nh * hd + 2 * nkv * hd
    T = sum(new)
    qkv = rounded(torch.randn(T, row, generator=g))
    w_q, w_k = 0.1 * torch.randn(hd, generator=g), 0.1 * torch.randn(hd, generator=g)
    pos = np.concatenate([L + np.arange(n) for L, n in zip(cached, new)])
    pos3 = np.ascontiguousarray(np.stack([pos, pos, pos], 1), dtype=np.int32)
    Qn, Kn, Vn, G = text_prep(qkv, nh, nkv, hd, n_rot, w_q, w_k, pos3, theta)
    lens_k = [L + n for L, n in zip(cached, new)]
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)   # record starts: multiples of 8
    assert all(x % 8 == 0 for x in cu_k[:-1])
    Tk = int(cu_k[-1])
    Kc = rounded(torch.randn(nkv, Tk, hd, generator=g)).double()
    Vc = rounded(torch.randn(nkv, Tk, hd, generator=g)).double()
    K, V = Kc.clone(), Vc.clone()
    cu_q = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    for r, (L, n) in enumerate(zip(cached, new)):
        K[:, cu_k[r] + L: cu_k[r] + L + n] = Kn[:, cu_q[r]:cu_q[r + 1]]
        V[:, cu_k[r] + L: cu_k[r] + L + n] = Vn[:, cu_q[r]:cu_q[r + 1]]
    O = sdpa_records(Qn, K, V, cu_q, cu_k, True)
    O = O * torch.sigmoid(G)
    np.savez_compressed(HERE / f"{name}.npz", qkv=bf16_bits(qkv), nh=nh, nkv=nkv, hd=hd, n_rot=n_rot,
                        theta=theta, gate=1, cu_seqlens=cu_q, pos3=pos3, cached=np.array(cached, np.int32),
                        cu_seqlens_k=cu_k, k_cache=bf16_bits(Kc.float()), v_cache=bf16_bits(Vc.float()),
                        q_norm=(1.0 + w_q).numpy().astype(np.float32), k_norm=(1.0 + w_k).numpy().astype(np.float32),
                        out=O.numpy().astype(np.float32))


def vision_case(name, grids, heads, seed):
    hd, merge = 72, 2
    g = torch.Generator().manual_seed(seed)
    E = heads * hd
    lens = [h * w for h, w in grids]
    P = sum(lens)
    qkv = rounded(torch.randn(P, 3 * E, generator=g))
    bias = 0.1 * torch.randn(3 * E, generator=g)
    thw = torch.tensor([[1, h, w] for h, w in grids])
    pos = get_vision_position_ids(thw, merge)                       # [P, 2] (row, column)
    rope = hf.Qwen3_5VisionRotaryEmbedding(hd // 2)
    freqs = rope(pos)                                                # [P, hd/2]
    emb = torch.cat((freqs, freqs), dim=-1)
    x = (qkv + bias).view(P, 3, heads, hd)
    q, k = hf.apply_rotary_pos_emb_vision(x[:, 0], x[:, 1], emb.cos(), emb.sin())
    v = x[:, 2]
    Q, K, V = (t.transpose(0, 1).double() for t in (q, k, v))       # [heads, P, hd]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    O = sdpa_records(Q, K, V, cu, cu, False)
    np.savez_compressed(HERE / f"{name}.npz", qkv=bf16_bits(qkv), bias=bias.numpy().astype(np.float32),
                        heads=heads, hd=hd, cu_seqlens=cu, grid_w=np.array([w for _, w in grids], np.int32),
                        pos2=pos.numpy().astype(np.int32), out=O.numpy().astype(np.float32))


@torch.no_grad()
def main():
    torch.manual_seed(0)
    text_case("text_gated_small", [1, 23, 46], nh=4, nkv=2, n_rot=64, norm=True, gate=True, seed=11)
    text_case("text_plain_small", [50], nh=4, nkv=1, n_rot=0, norm=False, gate=False, seed=12)
    prefix_case("prefix_small", cached=[37, 64], new=[11, 16], nh=4, nkv=2, seed=13)
    vision_case("vision_small", grids=[(4, 4), (6, 4)], heads=2, seed=14)
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
