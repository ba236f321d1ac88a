"""The projections either side of the path (clef_metal.m:463-499 clef_metal_gemm): bf16 X and W,
f32 accumulation, bf16 or f32 Y, and accumulation into an f32 residual, against a float64
product of the same operands."""
import ctypes

import numpy as np
import pytest
import torch

from cleffa_amd import _lib
from cleffa_amd.gemm import gemm


@pytest.mark.parametrize("args,msg", [
    ((4, 0, 8), "bad GEMM shape"),
    ((4, 8, 8, "y3"), "bad y_type"),
    ((4, 8, 8, "bf16acc"), "accumulation needs an f32 Y"),
])
def test_gemm_argument_errors(args, msg):
    lib = _lib.load()
    err = ctypes.create_string_buffer(256)
    T, N, K = args[:3]
    y_type, acc = 0, 0
    if len(args) > 3:
        y_type, acc = {"y3": (3, 0), "bf16acc": (1, 1)}[args[3]]
    assert not lib.clef_hip_gemm(T, N, K, 16, 16, 16, y_type, acc, None, 0, None, err, 256)
    assert msg in err.value.decode()


def _ref(X, W):
    return X.double() @ W.double().T


def _bound(X, W):
    """fp32 summation bound gamma_K * (|X| |W|^T) plus the rounding of the f32 result."""
    K = X.shape[1]
    mag = X.double().abs() @ W.double().abs().T
    return K * 2.0 ** -24 * mag + 2.0 ** -24 * mag


@pytest.mark.gpu
@pytest.mark.parametrize("T,N,K", [(1, 128, 256), (33, 1000, 520), (4096, 14336, 5120), (777, 5120, 6144)])
def test_gemm_f32_and_bf16(T, N, K):
    print(f"[gemm] T={T} N={N} K={K}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(T + N + K)
    X = torch.randn(T, K, generator=g, device="cuda").bfloat16()
    W = (0.05 * torch.randn(N, K, generator=g, device="cuda")).bfloat16()
    ref = _ref(X, W)
    bound = _bound(X, W)
    y32 = gemm(X, W, out="f32")
    torch.cuda.synchronize()
    assert ((y32.double() - ref).abs() <= bound).all(), "f32 result outside the fp32 summation bound"
    y16 = gemm(X, W, out="bf16")
    torch.cuda.synchronize()
    # bf16 of the f32 accumulation: within half a bf16 ulp of a value inside the bound
    ulp = torch.where(ref.abs() > 0, 2.0 ** (torch.floor(torch.log2(ref.abs())) - 7), torch.zeros_like(ref))
    assert ((y16.double() - ref).abs() <= bound + ulp).all(), "bf16 result off by more than one bf16 ulp"


@pytest.mark.gpu
def test_gemm_accumulates_into_residual():
    print("[gemm] accumulate", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    T, N, K = 300, 640, 6144
    X = torch.randn(T, K, generator=g, device="cuda").bfloat16()
    W = (0.02 * torch.randn(N, K, generator=g, device="cuda")).bfloat16()
    R = torch.randn(T, N, generator=g, device="cuda")
    want = R.double() + _ref(X, W)
    Y = R.clone()
    gemm(X, W, Y=Y, out="f32", acc=True)
    ws = torch.empty(32 << 20, dtype=torch.uint8, device="cuda")
    Y2 = R.clone()
    gemm(X, W, Y=Y2, out="f32", acc=True, workspace=ws)
    torch.cuda.synchronize()
    bound = _bound(X, W) + 2.0 ** -23 * want.abs()
    assert ((Y.double() - want).abs() <= bound).all()
    assert ((Y2.double() - want).abs() <= bound).all()


@pytest.mark.gpu
def test_gemm_first_call_captured_then_timed():
    """A shape first met under graph capture takes hipBLASLt's first candidate (nothing can be
    timed); the next uncaptured call times the candidates and replaces it; both graphs replay
    correctly, each replay checked against the float64 product with eager work in between."""
    print("[gemm] capture, then timed", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    T, N, K = 257, 1536, 1024   # a shape no other test uses
    X = torch.randn(T, K, generator=g, device="cuda").bfloat16()
    W = (0.05 * torch.randn(N, K, generator=g, device="cuda")).bfloat16()
    ws = torch.empty(32 << 20, dtype=torch.uint8, device="cuda")
    ref, bound = _ref(X, W), _bound(X, W)
    Yb = torch.empty(T, N, device="cuda", dtype=torch.bfloat16)
    ulp = torch.where(ref.abs() > 0, 2.0 ** (torch.floor(torch.log2(ref.abs())) - 7), torch.zeros_like(ref))
    graphs = []
    for rnd in range(2):
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            gemm(X, W, Y=Yb, out="bf16", workspace=ws)
        graphs.append(gr)
        if rnd == 0:   # an uncaptured call: times the candidates, replaces the captured choice
            Yb.zero_()
            gemm(X, W, Y=Yb, out="bf16", workspace=ws)
            torch.cuda.synchronize()
            assert ((Yb.double() - ref).abs() <= bound + ulp).all(), "timed call"
    for gr in graphs:
        for _ in range(3):
            Yb.fill_(float("nan"))
            gr.replay()
            torch.cuda.synchronize()
            assert ((Yb.double() - ref).abs() <= bound + ulp).all(), "graph replay"
            torch.mm(X.float(), W.float().T)   # eager work between replays
