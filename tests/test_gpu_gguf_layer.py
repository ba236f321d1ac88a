"""One full-attention layer driven from a clef GGUF: the layer's weights bound through
clef_hip_gguf_attn_layer (clef.c:180-256), then QKV GEMM -> prefill attention -> o_proj into the
residual on the GPU. Each stage is checked against float64 products of the arrays the test wrote
into the file, so a transposed or misplaced weight fails."""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, rope_inv_freq
from cleffa_amd.gemm import gemm
from cleffa_amd.gguf import GgufFile
from oracle import oracle
from tests.gguf import writer as gw
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)


def test_attention_layer_from_gguf(tmp_path):
    print("[gguf] layer from file", flush=True)
    H, nh, nkv, hd = 512, 4, 2, 256
    path = tmp_path / "layer.gguf"
    arrays, _ = gw.clef_attention_model(path, H=H, nh=nh, nkv=nkv, hd=hd, layer_types=(0, 1), seed=3)
    with GgufFile(path) as g:
        c = g.attn_config()
        w_qkv, w_o, qn, kn = g.attn_layer(1)
        torch.cuda.synchronize()
    # the device copies are the written bytes
    assert torch.equal(w_qkv.cpu().view(torch.int16), _bf16(arrays["blk.1.attn_qkv.weight"]).view(torch.int16))
    assert torch.equal(w_o.cpu().view(torch.int16), _bf16(arrays["blk.1.attn_output.weight"]).view(torch.int16))
    assert torch.equal(qn.cpu(), torch.from_numpy(arrays["blk.1.attn_q_norm.weight"]))

    lengths = [300, 77, 129]
    T = sum(lengths)
    gen = torch.Generator().manual_seed(9)
    X = torch.randn(T, H, generator=gen).bfloat16()
    R = torch.randn(T, H, generator=gen)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    pos = np.concatenate([np.arange(n) for n in lengths]).astype(np.int32)
    pos3 = torch.from_numpy(np.repeat(pos[:, None], 3, axis=1).copy())

    # QKV GEMM with the file's W
    qkv = gemm(X.cuda(), w_qkv, out="bf16")
    torch.cuda.synchronize()
    Wq = _bf16(arrays["blk.1.attn_qkv.weight"]).double()
    ref = X.double() @ Wq.T
    bound = (X.double().abs() @ Wq.abs().T) * (H + 1) * 2.0 ** -24
    ulp = torch.where(ref.abs() > 0, 2.0 ** (torch.floor(torch.log2(ref.abs())) - 7), torch.zeros_like(ref))
    assert ((qkv.cpu().double() - ref).abs() <= bound + ulp).all()

    # prefill attention with the file's norm weights, on the GPU's own qkv rows
    att = TextAttention(c.nh, c.nkv, c.hd, c.n_rot, eps=c.eps, rope_theta=c.rope_theta)
    plan = AttnPlan(cu, causal=True)
    A = att.forward(qkv, qn, kn, pos3.cuda(), plan)
    torch.cuda.synchronize()
    Q, K, V, G = oracle.text_prep(qkv.float().cpu().numpy(), nh, nkv, hd, c.n_rot, arrays["blk.1.attn_q_norm.weight"],
                                  arrays["blk.1.attn_k_norm.weight"], pos3.numpy(), rope_inv_freq(c.rope_theta, c.n_rot),
                                  eps=c.eps)
    want = oracle.attention(Q, K, V, cu, None, True, hd ** -0.5, G)
    assert_close(A.float().cpu().numpy(), want, what="attention from GGUF weights")

    # o_proj into the residual with the file's W_o
    Y = R.clone().cuda()
    gemm(A, w_o, Y=Y, out="f32", acc=True)
    torch.cuda.synchronize()
    Wo = _bf16(arrays["blk.1.attn_output.weight"]).double()
    ref = R.double() + A.cpu().double() @ Wo.T
    bound = (A.cpu().double().abs() @ Wo.abs().T) * (nh * hd + 1) * 2.0 ** -24 + 2.0 ** -23 * ref.abs()
    assert ((Y.cpu().double() - ref).abs() <= bound).all()


def test_vision_layer_from_gguf(tmp_path):
    print("[gguf] vision layer from file", flush=True)
    path = tmp_path / "vis.gguf"
    arrays, _ = gw.clef_attention_model(path, vis_heads=2, layer_types=(1,), seed=4)
    with GgufFile(path) as g:
        w_qkv, b_qkv, w_o, b_o = g.vis_layer(0, heads=2)
        torch.cuda.synchronize()
    assert torch.equal(w_qkv.cpu().view(torch.int16), _bf16(arrays["v.blk.0.attn_qkv.weight"]).view(torch.int16))
    assert torch.equal(b_qkv.cpu(), torch.from_numpy(arrays["v.blk.0.attn_qkv.bias"]))
    assert torch.equal(w_o.cpu().view(torch.int16), _bf16(arrays["v.blk.0.attn_out.weight"]).view(torch.int16))
    assert torch.equal(b_o.cpu(), torch.from_numpy(arrays["v.blk.0.attn_out.bias"]))
