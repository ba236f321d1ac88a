"""Y (+)= X . W^T for the projections either side of the attention path (clef_metal.m:463-499):
the QKV GEMM writing the bf16 qkv rows the path reads, and the o_proj accumulating into the f32
residual. Through the C ABI (hipBLASLt inside libclef_hip_attn.so)."""
import ctypes

import torch

from . import _lib
from ._lib import c_void_p  # noqa: F401
from .attention import _err, _stream_handle

Y_F32, Y_BF16 = 0, 1


def gemm(X, W, Y=None, out="bf16", acc=False, workspace=None, stream=None):
    """X [T][K] bf16, W [N][K] bf16 -> Y [T][N] (bf16 or f32); acc adds into an f32 Y."""
    if X.dtype != torch.bfloat16 or W.dtype != torch.bfloat16 or not X.is_contiguous() or not W.is_contiguous():
        raise ValueError("X and W must be contiguous bf16")
    T, K = X.shape
    N, K2 = W.shape
    if K2 != K:
        raise ValueError(f"inner dims differ: X has {K}, W has {K2}")
    y_type = Y_BF16 if out == "bf16" else Y_F32
    dt = torch.bfloat16 if y_type == Y_BF16 else torch.float32
    if Y is None:
        if acc:
            raise ValueError("acc needs the Y to add into")
        Y = torch.empty(T, N, dtype=dt, device=X.device)
    if Y.shape != (T, N) or Y.dtype != dt or not Y.is_contiguous():
        raise ValueError(f"Y must be contiguous {dt} [{T}][{N}]")
    ws = 0 if workspace is None else workspace.numel() * workspace.element_size()
    err = _err()
    ok = _lib.load().clef_hip_gemm(T, N, K, X.data_ptr(), W.data_ptr(), Y.data_ptr(), y_type, int(acc),
                                   None if workspace is None else workspace.data_ptr(), ws, _stream_handle(stream),
                                   err, len(err))
    _lib.check(ok, err)
    return Y
