"""Prefix-cache entry planes: the capacity policy (clef_metal.m:762-775) on the host, and on the
GPU the growth copy plus cached-versus-full exactness of prefix passes through a growing entry
(tests/test_prefix_attention.m: a record computed in pieces against its own cache equals the same
record computed in one pass)."""
import ctypes

import numpy as np
import pytest
import torch

from cleffa_amd import AttnPlan, TextAttention, _lib, workloads
from cleffa_amd.prefix_cache import PrefixEntry


def _cap(rows, cur, hd=256):
    return _lib.load().clef_hip_prefix_capacity(rows, cur, hd)


def test_capacity_policy():
    assert _cap(0, 0) == 0 and _cap(1, 0) == 1024 and _cap(1024, 0) == 1024 and _cap(1025, 0) == 2048
    assert _cap(900, 1024) == 1024                      # fits: unchanged
    assert _cap(1025, 1024) == 2048                     # at least a quarter more, rounded to 1024
    assert _cap(4097, 4096) == 5120                     # 4096 + 1024, already a multiple of 1024
    assert _cap(9000, 8192) == 10240                    # max(9000, 8192 + 2048)
    assert _cap(20000, 4096) == 20480                   # a big jump takes what is asked for
    for cur in (0, 1024, 3072, 65536):
        for rows in (cur + 1, cur + 700, 3 * cur + 5):
            c = _cap(rows, cur)
            assert c >= rows and c % 1024 == 0 and c >= cur + cur // 4


def test_capacity_limits():
    assert _cap(-1, 0) == -1
    assert _cap(8387584, 0) == 8387584                   # largest cap with 32-bit plane offsets at hd 256
    assert _cap(8387585, 0) == -1
    assert _lib.load().clef_hip_prefix_plane_bytes(4, 256, 2048) == 4 * 2048 * 256 * 2


@pytest.mark.parametrize("args,msg", [
    ((0, 0, 1024, 16, 16, 2048, 4, 256, 10), "source planes"),
    ((16, 16, 1024, 16, 16, 2048, 4, 256, 1025), "exceeds a capacity"),
    ((16, 16, 1020, 16, 16, 2048, 4, 256, 10), "multiples of 8"),
    ((16, 16, 1024, 0, 16, 2048, 4, 256, 10), "destination planes"),
    ((16, 16, 1024, 16, 16, 2048, 4, 250, 10), "bad plane shape"),
    ((16, 16, 1024, 24, 16, 2048, 4, 256, 10), "destination planes"),   # misaligned
])
def test_copy_argument_errors(args, msg):
    lib = _lib.load()
    err = ctypes.create_string_buffer(256)
    assert not lib.clef_hip_prefix_copy(*args, None, err, 256)
    assert msg in err.value.decode()


@pytest.mark.gpu
def test_growth_copy_exact():
    print("[prefix] growth copy", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    nkv, hd, src_cap, dst_cap = 3, 256, 1024, 2048
    ks = torch.randn(nkv, src_cap, hd, generator=g, device="cuda").bfloat16()
    vs = torch.randn(nkv, hd, src_cap, generator=g, device="cuda").bfloat16()
    for keep in (1000, 1024, 0, 5):
        kd = torch.full((nkv, dst_cap, hd), float("nan"), device="cuda").bfloat16()
        vd = torch.full((nkv, hd, dst_cap), float("nan"), device="cuda").bfloat16()
        err = ctypes.create_string_buffer(256)
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        ok = _lib.load().clef_hip_prefix_copy(ks.data_ptr(), vs.data_ptr(), src_cap, kd.data_ptr(), vd.data_ptr(),
                                              dst_cap, nkv, hd, keep, s, err, 256)
        _lib.check(ok, err)
        torch.cuda.synchronize()
        wk = torch.zeros_like(kd)
        wk[:, :keep] = ks[:, :keep]
        wv = torch.zeros_like(vd)
        wv[:, :, :keep] = vs[:, :, :keep]
        assert torch.equal(kd.view(torch.int16), wk.view(torch.int16)), f"K keep {keep}"
        assert torch.equal(vd.view(torch.int16), wv.view(torch.int16)), f"V^T keep {keep}"


@pytest.mark.gpu
@pytest.mark.parametrize("T,cuts", [(161, [32]), (1025, [544]), (2049, [512, 1056])])
def test_cached_versus_full_exact(T, cuts):
    """A record computed in pieces (rows [0, c1), [c1, c2), ...) through a prefix entry that
    grows between them equals the record computed in one pass, bit for bit."""
    print(f"[prefix] cached vs full T={T} cuts={cuts}", flush=True)
    nh, nkv, hd = 16, 4, 256
    w = workloads.text_inputs([T], nh, nkv, seed=T)
    d = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    att = TextAttention(nh, nkv, hd, 64, rope_theta=1e7)
    full = att.forward(d["qkv"], d["q_norm"], d["k_norm"], d["pos3"], AttnPlan([0, T], [0, T]))
    entry = PrefixEntry(1, nkv, hd)
    bounds = [0] + cuts + [T]
    pieces = []
    for L, E in zip(bounds[:-1], bounds[1:]):
        entry.reserve(E, keep=L)
        plan = AttnPlan([0, E - L], [0, E])
        pieces.append(att.forward(d["qkv"][L:E].contiguous(), d["q_norm"], d["k_norm"], d["pos3"][L:E].contiguous(),
                                  plan, k_plane=entry.K[0], vt_plane=entry.Vt[0], kvT=entry.cap))
    torch.cuda.synchronize()
    got = torch.cat(pieces)
    assert entry.cap >= T and entry.cap % 1024 == 0
    assert torch.equal(got.view(torch.int16), full.view(torch.int16))
