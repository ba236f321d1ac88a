"""cleffa_amd: MI355X-native prefill attention for cleffa (HIP kernels behind a C ABI).

The compute lives in libclef_hip_attn.so (include/clef_hip_attn.h); this package holds the
host-side layer above it: plans, plane allocation and the calls.
"""
from ._lib import OUT_BF16, OUT_F16, OUT_F32, load  # noqa: F401
from .attention import AttnPlan, TextAttention, VisionAttention, init_device, rope_inv_freq, vision_positions  # noqa: F401

__all__ = ["AttnPlan", "TextAttention", "VisionAttention", "init_device", "rope_inv_freq",
           "vision_positions", "load", "OUT_BF16", "OUT_F16", "OUT_F32"]
