"""clef_hip_vis_attention_noalloc (the vision step on the library's static device scratch)
against clef_hip_vis_attention on caller-owned planes: bitwise equal outputs and overflow flags,
on two calls in a row, the second smaller, and the size limit rejected before any launch."""
import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, VisionAttention, _lib, vision_positions

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _case(grids, heads, seed, scale=1.0):
    lens = [a * b for a, b in grids]
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((sum(lens), 3 * heads * 72), generator=g) * scale).to(torch.bfloat16)
    bias = torch.randn((3 * heads * 72,), generator=g) * 0.1
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pos2 = vision_positions(cu, [b for _, b in grids], 2)
    return qkv.cuda(), bias.cuda(), torch.from_numpy(pos2).cuda(), AttnPlan(cu, causal=False)


@pytest.mark.parametrize("out_dtype", ["bf16", "f16"])
def test_noalloc_matches_caller_planes(out_dtype):
    heads = 16
    vis = VisionAttention(heads, 72)
    # first call: four images (2,304 patches); second: one small image, so stale scratch rows
    # from the first call lie past every key the second reads
    for grids, seed in (([(16, 18), (32, 40), (24, 24), (6, 10)], 5), ([(4, 6)], 6)):
        _say(f"[no_alloc] {out_dtype} grids {grids} heads {heads}")
        qkv, bias, pos2, plan = _case(grids, heads, seed, scale=30.0 if out_dtype == "f16" else 1.0)
        ovf_ref = torch.zeros(plan.T, dtype=torch.int32, device="cuda")
        ovf_new = torch.zeros(plan.T, dtype=torch.int32, device="cuda")
        ref = vis.forward(qkv, bias, pos2, plan, out_dtype=out_dtype, ovf=ovf_ref)
        new = vis.forward(qkv, bias, pos2, plan, out_dtype=out_dtype, ovf=ovf_new, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(new.view(torch.int16), ref.view(torch.int16)), f"{grids}: outputs differ"
        assert torch.equal(ovf_new, ovf_ref)
        assert torch.isfinite(new.float()).all()


def test_noalloc_rejects_beyond_scratch():
    heads = 16
    vis = VisionAttention(heads, 72)
    qkv, bias, pos2, plan = _case([(4, 4)], heads, 7)
    # 16 heads x (P + 2 kvT) x 144 bytes above 64 MiB: a plan this large is refused before launch
    P = 10_000
    big = torch.empty((P, 3 * heads * 72), dtype=torch.bfloat16, device="cuda")
    pos = torch.zeros((P, 2), dtype=torch.int32, device="cuda")
    bplan = AttnPlan(np.array([0, P], np.int32), causal=False)
    assert heads * (P + 2 * bplan.kvT) * 144 > _lib.VIS_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="scratch"):
        vis.forward(big, None, pos, bplan, noalloc=True)
    # the library stays usable after the refusal
    ref = vis.forward(qkv, bias, pos2, plan)
    new = vis.forward(qkv, bias, pos2, plan, noalloc=True)
    torch.cuda.synchronize()
    assert torch.equal(new.view(torch.int16), ref.view(torch.int16))
