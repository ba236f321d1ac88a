"""HIP path against the committed golden fixtures (PyTorch float64 SDPA + transformers Qwen3.5
prologue, written by tests/golden/make_golden.py), through the C ABI: gated and plain text
passes, a prefix-cache continuation with cu_seqlens_k, and the vision encoder's attention."""
from pathlib import Path

import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, VisionAttention, vision_positions
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def _bf16(bits, device="cuda"):
    return torch.from_numpy(np.asarray(bits).view(np.int16).copy()).view(torch.bfloat16).to(device)


def _text_inputs(z):
    nh, nkv, hd, n_rot = int(z["nh"]), int(z["nkv"]), int(z["hd"]), int(z["n_rot"])
    att = TextAttention(nh, nkv, hd, n_rot, rope_theta=float(z["theta"]))
    norm = lambda k: torch.from_numpy(z[k]).cuda() if z[k].size else None
    return att, _bf16(z["qkv"]), norm("q_norm"), norm("k_norm"), torch.from_numpy(z["pos3"]).cuda()


@pytest.mark.parametrize("name", ["text_gated_small", "text_plain_small"])
def test_text_golden(name):
    print(f"[golden] {name}", flush=True)
    z = np.load(GOLD / f"{name}.npz")
    att, qkv, qn, kn, pos = _text_inputs(z)
    plan = AttnPlan(z["cu_seqlens"], causal=True)
    out = att.forward(qkv, qn, kn, pos, plan, gate=bool(z["gate"]))
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), z["out"], what=name)


def test_prefix_golden():
    print("[golden] prefix_small", flush=True)
    z = np.load(GOLD / "prefix_small.npz")
    att, qkv, qn, kn, pos = _text_inputs(z)
    plan = AttnPlan(z["cu_seqlens"], z["cu_seqlens_k"], causal=True)
    kvT = plan.kvT
    Tk = int(z["cu_seqlens_k"][-1])
    kp, vt = att.planes(kvT)
    kp.zero_(), vt.zero_()
    kp[:, :Tk] = _bf16(z["k_cache"])
    vt[:, :, :Tk] = _bf16(z["v_cache"]).transpose(1, 2)
    before = kp.clone()
    out = att.forward(qkv, qn, kn, pos, plan, k_plane=kp, vt_plane=vt, kvT=kvT)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), z["out"], what="prefix")
    # cached rows untouched, new rows written at the end of each record
    ck, cq, cached = z["cu_seqlens_k"], z["cu_seqlens"], z["cached"]
    for r in range(len(cq) - 1):
        a = int(ck[r]); L = int(cached[r])
        assert torch.equal(kp[:, a:a + L], before[:, a:a + L])
        assert not torch.equal(kp[:, a + L:int(ck[r + 1])], before[:, a + L:int(ck[r + 1])])


def test_vision_golden():
    print("[golden] vision_small", flush=True)
    z = np.load(GOLD / "vision_small.npz")
    vis = VisionAttention(int(z["heads"]), int(z["hd"]))
    pos2 = torch.from_numpy(vision_positions(z["cu_seqlens"], z["grid_w"], 2)).cuda()
    plan = AttnPlan(z["cu_seqlens"], causal=False)
    out = vis.forward(_bf16(z["qkv"]), torch.from_numpy(z["bias"]).cuda(), pos2, plan)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), z["out"], what="vision")
