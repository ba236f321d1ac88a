"""ctypes binding of libclef_hip_attn.so (the C ABI declared in include/clef_hip_attn.h).

The library is the product: there is no Python or CPU fallback. Loading fails loudly when the
shared library has not been built.
"""
import ctypes
import os
from ctypes import POINTER, c_bool, c_char_p, c_float, c_int, c_int32, c_size_t, c_uint16, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("CLEF_HIP_ATTN_LIB") or Path(__file__).resolve().parent / "libclef_hip_attn.so")

OUT_BF16, OUT_F16, OUT_F32 = 0, 1, 2
QKV_BF16, QKV_F32 = 0, 1
VIS_SCRATCH_BYTES = 64 << 20
BLOCK_Q = 128
KV_ALIGN = 8
BLOCK_INTS = 8

# Every symbol include/clef_hip_attn.h declares.
EXPORTS = (
    "clef_hip_attn_version", "clef_hip_attn_wave_size", "clef_hip_attn_init",
    "clef_hip_attn_plan_max_blocks", "clef_hip_attn_plan", "clef_hip_attn_sched_size",
    "clef_hip_attn_schedule",
    "clef_hip_rope_inv_freq", "clef_hip_vis_positions", "clef_hip_attn_prep_kv",
    "clef_hip_attn_core", "clef_hip_attn_prefill", "clef_hip_vis_attention", "clef_hip_vis_attention_noalloc",
    "clef_hip_record_positions", "clef_hip_pack_batch",
    "clef_hip_gemm", "clef_hip_qkv_gemm",
    "clef_hip_omni_rope_table", "clef_hip_omni_prep", "clef_hip_omni_plan_max_blocks",
    "clef_hip_omni_plan", "clef_hip_omni_attention",
    "clef_hip_prefix_capacity", "clef_hip_prefix_plane_bytes", "clef_hip_prefix_copy",
    "clef_hip_gguf_open", "clef_hip_gguf_close", "clef_hip_gguf_tensor_count", "clef_hip_gguf_tensor_at",
    "clef_hip_gguf_find_tensor", "clef_hip_gguf_get_u32", "clef_hip_gguf_get_f32", "clef_hip_gguf_attn_config",
    "clef_hip_gguf_attn_layer", "clef_hip_gguf_vis_layer",
)

GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
MAX_LAYERS = 128


class GgufTensorInfo(ctypes.Structure):
    _fields_ = [("n_dims", ctypes.c_uint32), ("type", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("data", c_void_p)]


class AttnConfig(ctypes.Structure):
    _fields_ = [("n_layer", c_int), ("H", c_int), ("nh", c_int), ("nkv", c_int), ("hd", c_int), ("n_rot", c_int),
                ("eps", c_float), ("rope_theta", c_float), ("layer_full", c_int32 * MAX_LAYERS)]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("nh", c_int), ("nkv", c_int), ("hd", c_int), ("n_rot", c_int),
        ("eps", c_float), ("scale", c_float),
        ("T", c_int), ("row", c_int),
        ("qkv", c_void_p), ("q_norm", c_void_p), ("k_norm", c_void_p), ("pos3", c_void_p),
        ("inv_freq", c_void_p), ("rope_cs", c_void_p), ("k_plane", c_void_p), ("vt_plane", c_void_p),
        ("kvT", c_int), ("blocks", c_void_p), ("n_blk", c_int),
        ("kv_tok", c_void_p),
        ("kv_rows", c_int), ("causal", c_int), ("gate", c_int),
        ("out", c_void_p), ("out_type", c_int), ("f16_lim", c_float), ("ovf", c_void_p),
        ("trace", c_void_p), ("sched", c_void_p), ("n_wg", c_int),
        ("seq_start", c_void_p), ("qkv_type", c_int), ("tok_kv", c_void_p),
    ]


class VisArgs(ctypes.Structure):
    _fields_ = [
        ("P", c_int), ("heads", c_int), ("hd", c_int), ("scale", c_float),
        ("qkv", c_void_p), ("bias", c_void_p), ("pos2", c_void_p), ("inv_freq", c_void_p),
        ("q_plane", c_void_p), ("k_plane", c_void_p), ("vt_plane", c_void_p), ("kvT", c_int),
        ("blocks", c_void_p), ("n_blk", c_int), ("kv_tok", c_void_p), ("kv_rows", c_int),
        ("out", c_void_p), ("out_type", c_int), ("f16_lim", c_float), ("ovf", c_void_p),
        ("tok_kv", c_void_p),
    ]


class OmniPrepArgs(ctypes.Structure):
    _fields_ = [
        ("nh", c_int), ("nkv", c_int), ("T", c_int), ("kvT", c_int), ("eps", c_float), ("rope_exact", c_int),
        ("qkv", c_void_p), ("q_norm", c_void_p), ("k_norm", c_void_p), ("pos3", c_void_p), ("freq", c_void_p),
        ("q_plane", c_void_p), ("k_plane", c_void_p), ("v_plane", c_void_p), ("status", c_void_p),
    ]


class OmniAttnArgs(ctypes.Structure):
    _fields_ = [
        ("nh", c_int), ("nkv", c_int), ("T", c_int), ("kvT", c_int), ("scale", c_float),
        ("q_plane", c_void_p), ("k_plane", c_void_p), ("v_plane", c_void_p), ("blocks", c_void_p),
        ("n_blk", c_int), ("out", c_void_p),
    ]


_lib = None


def load():
    """Returns the loaded library; raises if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m cleffa_amd.build` "
                           "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.clef_hip_attn_version.restype = c_int
    lib.clef_hip_attn_wave_size.restype = c_int
    lib.clef_hip_attn_init.argtypes = [c_char_p, c_size_t]
    lib.clef_hip_attn_init.restype = c_bool
    lib.clef_hip_record_positions.argtypes = [c_int, POINTER(c_int32), POINTER(c_int32), POINTER(c_int32), POINTER(c_int32),
                                              c_int, c_int, POINTER(c_int32), c_char_p, c_size_t]
    lib.clef_hip_record_positions.restype = c_bool
    lib.clef_hip_pack_batch.argtypes = [POINTER(c_int32), ctypes.c_void_p, c_int, c_int, ctypes.c_long, POINTER(c_int32)]
    lib.clef_hip_pack_batch.restype = c_int
    lib.clef_hip_gemm.argtypes = [c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_size_t,
                                  c_void_p, c_char_p, c_size_t]
    lib.clef_hip_gemm.restype = c_bool
    lib.clef_hip_qkv_gemm.argtypes = [c_int, c_void_p, c_void_p, POINTER(AttnArgs), c_void_p, c_void_p, c_char_p, c_size_t]
    lib.clef_hip_qkv_gemm.restype = c_bool
    lib.clef_hip_omni_rope_table.argtypes = [c_float, POINTER(c_float)]
    lib.clef_hip_omni_rope_table.restype = None
    lib.clef_hip_omni_prep.argtypes = [POINTER(OmniPrepArgs), c_void_p, c_char_p, c_size_t]
    lib.clef_hip_omni_prep.restype = c_bool
    lib.clef_hip_omni_plan_max_blocks.argtypes = [c_int, c_int]
    lib.clef_hip_omni_plan_max_blocks.restype = c_int
    lib.clef_hip_omni_plan.argtypes = [POINTER(c_int32), c_int, POINTER(c_int32), c_int, POINTER(c_int),
                                       c_char_p, c_size_t]
    lib.clef_hip_omni_plan.restype = c_bool
    lib.clef_hip_omni_attention.argtypes = [POINTER(OmniAttnArgs), c_void_p, c_char_p, c_size_t]
    lib.clef_hip_omni_attention.restype = c_bool
    lib.clef_hip_prefix_capacity.argtypes = [c_int, c_int, c_int]
    lib.clef_hip_prefix_capacity.restype = c_int
    lib.clef_hip_prefix_plane_bytes.argtypes = [c_int, c_int, c_int]
    lib.clef_hip_prefix_plane_bytes.restype = c_size_t
    lib.clef_hip_prefix_copy.argtypes = [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                         c_void_p, c_char_p, c_size_t]
    lib.clef_hip_prefix_copy.restype = c_bool
    lib.clef_hip_gguf_open.argtypes = [c_char_p, POINTER(c_void_p), c_char_p, c_size_t]
    lib.clef_hip_gguf_open.restype = c_bool
    lib.clef_hip_gguf_close.argtypes = [c_void_p]
    lib.clef_hip_gguf_close.restype = None
    lib.clef_hip_gguf_tensor_count.argtypes = [c_void_p]
    lib.clef_hip_gguf_tensor_count.restype = c_int
    lib.clef_hip_gguf_tensor_at.argtypes = [c_void_p, c_int, POINTER(GgufTensorInfo), c_char_p, c_size_t]
    lib.clef_hip_gguf_tensor_at.restype = c_bool
    lib.clef_hip_gguf_find_tensor.argtypes = [c_void_p, c_char_p, POINTER(GgufTensorInfo)]
    lib.clef_hip_gguf_find_tensor.restype = c_bool
    lib.clef_hip_gguf_get_u32.argtypes = [c_void_p, c_char_p, POINTER(ctypes.c_uint32)]
    lib.clef_hip_gguf_get_u32.restype = c_bool
    lib.clef_hip_gguf_get_f32.argtypes = [c_void_p, c_char_p, POINTER(c_float)]
    lib.clef_hip_gguf_get_f32.restype = c_bool
    lib.clef_hip_gguf_attn_config.argtypes = [c_void_p, POINTER(AttnConfig), c_char_p, c_size_t]
    lib.clef_hip_gguf_attn_config.restype = c_bool
    lib.clef_hip_gguf_attn_layer.argtypes = [c_void_p, POINTER(AttnConfig), c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_char_p, c_size_t]
    lib.clef_hip_gguf_attn_layer.restype = c_bool
    lib.clef_hip_gguf_vis_layer.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_char_p, c_size_t]
    lib.clef_hip_gguf_vis_layer.restype = c_bool
    lib.clef_hip_attn_plan_max_blocks.argtypes = [c_int, c_int]
    lib.clef_hip_attn_plan_max_blocks.restype = c_int
    lib.clef_hip_attn_plan.argtypes = [POINTER(c_int32), POINTER(c_int32), c_int, c_int,
                                       POINTER(c_int32), c_int, POINTER(c_int32), c_int,
                                       POINTER(c_int32), c_int,
                                       POINTER(c_int), POINTER(c_int), c_char_p, c_size_t]
    lib.clef_hip_attn_plan.restype = c_bool
    lib.clef_hip_attn_sched_size.argtypes = [c_int, c_int, c_int]
    lib.clef_hip_attn_sched_size.restype = c_int
    lib.clef_hip_attn_schedule.argtypes = [POINTER(c_int32), c_int, c_int, c_int, c_int, POINTER(c_int32), c_int,
                                           c_char_p, c_size_t]
    lib.clef_hip_attn_schedule.restype = c_bool
    lib.clef_hip_rope_inv_freq.argtypes = [c_float, c_int, POINTER(c_float)]
    lib.clef_hip_rope_inv_freq.restype = None
    lib.clef_hip_vis_positions.argtypes = [POINTER(c_int32), c_int, POINTER(c_int32), c_int,
                                           POINTER(c_int32), c_char_p, c_size_t]
    lib.clef_hip_vis_positions.restype = c_bool
    for name in ("clef_hip_attn_prep_kv", "clef_hip_attn_core", "clef_hip_attn_prefill"):
        fn = getattr(lib, name)
        fn.argtypes = [POINTER(AttnArgs), c_void_p, c_char_p, c_size_t]
        fn.restype = c_bool
    for name in ("clef_hip_vis_attention", "clef_hip_vis_attention_noalloc"):
        fn = getattr(lib, name)
        fn.argtypes = [POINTER(VisArgs), c_void_p, c_char_p, c_size_t]
        fn.restype = c_bool
    _lib = lib
    return lib


def load_bench():
    """The measurement utility library (clef_hip_mfma_ceiling), built beside the product."""
    path = LIB_PATH.parent / "libclef_hip_bench.so"
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run `python -m cleffa_amd.build`")
    lib = ctypes.CDLL(str(path))
    lib.clef_hip_mfma_ceiling.argtypes = [c_int, c_int, c_void_p, c_size_t, POINTER(ctypes.c_double),
                                          POINTER(ctypes.c_double), c_char_p, c_size_t]
    lib.clef_hip_mfma_ceiling.restype = c_bool
    return lib


def check(ok, err):
    if not ok:
        raise RuntimeError(err.value.decode(errors="replace") or "hip: unknown error")
