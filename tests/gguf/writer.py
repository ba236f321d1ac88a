"""A GGUF v3 writer for tests (the container tools/convert.py writes through the gguf package,
which is not installed here): header, typed metadata, tensor table, aligned data."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def bf16_bits(a):
    """float32 array -> bf16 bit patterns (round to nearest even), uint16."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def write(path, kvs, tensors, alignment=32):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, array)] with the array's shape in
    row-major order (ne is the reversed shape). Returns the absolute data offsets."""
    if alignment != 32:
        kvs = [("general.alignment", U32, alignment)] + list(kvs)
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs))
    meta = b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kvs)
    infos, blobs, off = b"", [], 0
    rel = []
    for name, gt, arr in tensors:
        arr = np.ascontiguousarray(arr)
        ne = list(arr.shape[::-1])
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", gt, off)
        data = arr.tobytes()
        rel.append(off)
        blobs.append((off, data))
        off = (off + len(data) + alignment - 1) // alignment * alignment
    pre = head + meta + infos
    data_start = (len(pre) + alignment - 1) // alignment * alignment
    buf = bytearray(pre + b"\0" * (data_start - len(pre)))
    for o, d in blobs:
        end = data_start + o
        if len(buf) < end:
            buf += b"\0" * (end - len(buf))
        buf[end:end + len(d)] = d
    with open(path, "wb") as f:
        f.write(bytes(buf))
    return [data_start + o for o in rel]


def clef_attention_model(path, H=128, nh=4, nkv=2, hd=256, layer_types=(0, 1, 1), vis_heads=2, seed=0,
                         alignment=32, extra_kvs=()):
    """A clef GGUF holding the attention-side tensors of every full-attention layer (and a
    DeltaNet stand-in for the others), a vision attention layer, and the geometry keys."""
    rng = np.random.default_rng(seed)
    n_attn = 2 * nh * hd + 2 * nkv * hd
    kvs = [("general.architecture", STRING, "clef"),
           ("general.name", STRING, "synthetic"),
           ("clef.block_count", U32, len(layer_types)),
           ("clef.embedding_length", U32, H),
           ("clef.attention.head_count", U32, nh),
           ("clef.attention.head_count_kv", U32, nkv),
           ("clef.attention.key_length", U32, hd),
           ("clef.rope.dimension_count", U32, 64),
           ("clef.attention.layer_norm_rms_epsilon", F32, 1e-6),
           ("clef.rope.freq_base", F32, 1e7),
           ("clef.layer_types", ARRAY, (I32, list(layer_types))),
           ("tokenizer.tokens", ARRAY, (STRING, ["<a>", "bb", "ccc"])),
           ("clef.nested", ARRAY, (ARRAY, [(U8, [1, 2]), (U8, [3])])),
           ("clef.flag", BOOL, True),
           ("clef.big", U64, 1 << 40),
           ("clef.f64", F64, 0.5)] + list(extra_kvs)
    tensors, arrays = [], {}
    for l, full in enumerate(layer_types):
        if full:
            t = {f"blk.{l}.attn_qkv.weight": (GGML_BF16, bf16_bits(0.05 * rng.standard_normal((n_attn, H)))),
                 f"blk.{l}.attn_output.weight": (GGML_BF16, bf16_bits(0.05 * rng.standard_normal((H, nh * hd)))),
                 f"blk.{l}.attn_q_norm.weight": (GGML_F32, (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)),
                 f"blk.{l}.attn_k_norm.weight": (GGML_F32, (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))}
        else:
            t = {f"blk.{l}.ssm_a": (GGML_F32, rng.standard_normal(8).astype(np.float32))}
        t[f"blk.{l}.attn_norm.weight"] = (GGML_F32, rng.standard_normal(H).astype(np.float32))
        for k, (gt, a) in t.items():
            tensors.append((k, gt, a))
            arrays[k] = a
    E = 72 * vis_heads
    for k, gt, a in [("v.blk.0.attn_qkv.weight", GGML_BF16, bf16_bits(0.05 * rng.standard_normal((3 * E, E)))),
                     ("v.blk.0.attn_qkv.bias", GGML_F32, (0.1 * rng.standard_normal(3 * E)).astype(np.float32)),
                     ("v.blk.0.attn_out.weight", GGML_BF16, bf16_bits(0.05 * rng.standard_normal((E, E)))),
                     ("v.blk.0.attn_out.bias", GGML_F32, (0.1 * rng.standard_normal(E)).astype(np.float32)),
                     ("token_embd.weight", GGML_F16, rng.standard_normal((5, H)).astype(np.float16))]:
        tensors.append((k, gt, a))
        arrays[k] = a
    offsets = write(path, kvs, tensors, alignment)
    return arrays, dict(zip([t[0] for t in tensors], offsets))
