"""GGUF weight binding (clef_hip_gguf_*): the library's reader against the reference's own reader
(clef_gguf.c, compiled from its sources into oracle/_ref when they are present) and against what
the test wrote, on well-formed, malformed and truncated files; then the attention geometry and
per-layer binding checks of clef.c:27-59 and 180-256."""
import ctypes
import os

import numpy as np
import pytest

from cleffa_amd import _lib
from cleffa_amd.gguf import GgufFile
from oracle import oracle
from tests.gguf import writer as gw


class _Str(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("len", ctypes.c_uint64)]


class _RefTensor(ctypes.Structure):   # gguf_tensor (clef_gguf.h)
    _fields_ = [("name", _Str), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4), ("type", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]


class _RefFile(ctypes.Structure):     # gguf_file (clef_gguf.h)
    _fields_ = [("fd", ctypes.c_int), ("base", ctypes.c_void_p), ("size", ctypes.c_uint64), ("n_kv", ctypes.c_uint64),
                ("n_tensors", ctypes.c_uint64), ("kv", ctypes.c_void_p), ("tensors", ctypes.POINTER(_RefTensor)),
                ("data_offset", ctypes.c_uint64)]


def _ref_lib():
    if not oracle.REF_GGUF.exists():
        return None
    lib = ctypes.CDLL(str(oracle.REF_GGUF))
    lib.gguf_open.argtypes = [ctypes.POINTER(_RefFile), ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    lib.gguf_open.restype = ctypes.c_bool
    lib.gguf_close.argtypes = [ctypes.POINTER(_RefFile)]
    lib.gguf_get_u32.argtypes = [ctypes.POINTER(_RefFile), ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]
    lib.gguf_get_u32.restype = ctypes.c_bool
    lib.gguf_get_f32.argtypes = [ctypes.POINTER(_RefFile), ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]
    lib.gguf_get_f32.restype = ctypes.c_bool
    return lib


def _ref_table(lib, path):
    """(ok, [(name, n_dims, ne, type, offset, nbytes)]) from the reference reader."""
    f = _RefFile()
    err = ctypes.create_string_buffer(256)
    if not lib.gguf_open(ctypes.byref(f), str(path).encode(), err, 256):
        return False, None
    rows = []
    for i in range(f.n_tensors):
        t = f.tensors[i]
        # the library hands names out NUL-terminated: compare up to the first NUL
        name = ctypes.string_at(t.name.ptr, t.name.len).split(b"\0")[0][:511].decode("utf-8", "surrogateescape")
        rows.append((name, t.n_dims, tuple(t.ne), t.type, t.offset, t.nbytes))
    lib.gguf_close(ctypes.byref(f))
    return True, rows


def _our_table(path):
    try:
        g = GgufFile(path)
    except RuntimeError:
        return False, None
    rows = [(n, i.n_dims, tuple(i.ne), i.type, i.offset, i.nbytes) for n, i in g.tensors()]
    g.close()
    return True, rows


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "clef.gguf"
    arrays, offsets = gw.clef_attention_model(path)
    return path, arrays, offsets


def test_reader_reads_what_was_written(model):
    path, arrays, offsets = model
    with GgufFile(path) as g:
        names = [n for n, _ in g.tensors()]
        assert names == list(arrays)
        for n, info in g.tensors():
            assert info.offset == offsets[n]
            a = arrays[n]
            assert tuple(info.ne[d] for d in range(info.n_dims)) == a.shape[::-1]
            assert np.array_equal(g.tensor(n), a.view(g.tensor(n).dtype))
        assert g.u32("clef.attention.head_count") == 4 and g.u32("clef.block_count") == 3
        assert g.u32("clef.big") is None   # a u64 is not a u32
        assert g.f32("clef.rope.freq_base") == np.float32(1e7)
        c = g.attn_config()
        assert (c.n_layer, c.H, c.nh, c.nkv, c.hd, c.n_rot) == (3, 128, 4, 2, 256, 64)
        assert c.eps == np.float32(1e-6) and list(c.layer_full[:3]) == [0, 1, 1]


@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_matches_reference_reader(tmp_path, alignment):
    lib = _ref_lib()
    if lib is None:
        pytest.skip("reference sources not present (oracle/_ref not built)")
    path = tmp_path / "m.gguf"
    gw.clef_attention_model(path, alignment=alignment, seed=alignment)
    ok_r, ref = _ref_table(lib, path)
    ok_o, ours = _our_table(path)
    assert ok_r and ok_o and ours == ref
    # scalar lookups agree
    f = _RefFile()
    err = ctypes.create_string_buffer(64)
    assert lib.gguf_open(ctypes.byref(f), str(path).encode(), err, 64)
    with GgufFile(path) as g:
        for key in ("clef.block_count", "clef.attention.head_count_kv", "clef.big", "missing"):
            v = ctypes.c_uint32()
            r = lib.gguf_get_u32(ctypes.byref(f), key.encode(), ctypes.byref(v))
            assert (v.value if r else None) == g.u32(key)
        for key in ("clef.rope.freq_base", "clef.attention.layer_norm_rms_epsilon", "clef.block_count"):
            v = ctypes.c_float()
            r = lib.gguf_get_f32(ctypes.byref(f), key.encode(), ctypes.byref(v))
            assert (v.value if r else None) == g.f32(key)
    lib.gguf_close(ctypes.byref(f))


def test_malformed_files_agree_with_reference(tmp_path, model):
    """Truncations at every 7th byte of the header and tables, and single-byte corruptions of
    the counts, lengths, types and offsets: both readers accept or refuse together, and agree on
    the table of every accepted file."""
    lib = _ref_lib()
    path, _, _ = model
    blob = path.read_bytes()
    rng = np.random.default_rng(1)
    data_start = min(_our_table(path)[1], key=lambda r: r[4])[4]
    cases = [blob[:n] for n in range(0, data_start + 64, 7)]
    for _ in range(300):
        b = bytearray(blob)
        pos = int(rng.integers(0, data_start))
        b[pos] = int(rng.integers(0, 256))
        cases.append(bytes(b))
    # counts far beyond the file, a bad magic, a bad version, a zero / non-power-of-two alignment
    b = bytearray(blob); b[8:16] = (1 << 62).to_bytes(8, "little"); cases.append(bytes(b))
    b = bytearray(blob); b[16:24] = (1 << 40).to_bytes(8, "little"); cases.append(bytes(b))
    b = bytearray(blob); b[0] = 0; cases.append(bytes(b))
    b = bytearray(blob); b[4] = 2; cases.append(bytes(b))
    refused = 0
    for i, c in enumerate(cases):
        p = tmp_path / f"c{i}.gguf"
        p.write_bytes(c)
        ok_o, ours = _our_table(p)
        if not ok_o:
            refused += 1
        if lib is not None:
            ok_r, ref = _ref_table(lib, p)
            assert ok_o == ok_r, f"case {i}: reference {'accepts' if ok_r else 'refuses'}, library does not"
            if ok_o:
                assert ours == ref, f"case {i}: tables differ"
        os.unlink(p)
    assert refused > 100


@pytest.mark.parametrize("alignment", [0, 48])
def test_bad_alignment_refused(tmp_path, alignment):
    path = tmp_path / "a.gguf"
    gw.write(path, [("general.alignment", gw.U32, alignment)], [("x", gw.GGML_F32, np.zeros(4, np.float32))])
    with pytest.raises(RuntimeError, match="alignment"):
        GgufFile(path)


def test_unsupported_tensor_type_and_rank_refused(tmp_path):
    p = tmp_path / "q.gguf"
    gw.write(p, [], [("q", 2, np.zeros(4, np.uint8))])   # a quantized type
    with pytest.raises(RuntimeError, match="tensor table"):
        GgufFile(p)
    p2 = tmp_path / "r.gguf"
    gw.write(p2, [], [("r", gw.GGML_F32, np.zeros((1, 1, 1, 1, 2), np.float32))])
    with pytest.raises(RuntimeError, match="tensor table"):
        GgufFile(p2)


def test_config_errors(tmp_path):
    p = tmp_path / "c.gguf"
    gw.clef_attention_model(p, layer_types=(1, 2))
    with GgufFile(p) as g, pytest.raises(RuntimeError, match="unknown type 2"):
        g.attn_config()
    p = tmp_path / "d.gguf"
    gw.write(p, [("general.architecture", gw.STRING, "llama")], [])
    with GgufFile(p) as g, pytest.raises(RuntimeError, match="not a clef"):
        g.attn_config()
    p = tmp_path / "e.gguf"
    gw.clef_attention_model(p, nh=3, nkv=2, layer_types=(1,))
    with GgufFile(p) as g, pytest.raises(RuntimeError, match="multiple"):
        g.attn_config()


def test_layer_binding_checks(tmp_path, model):
    """The per-layer binding refuses a DeltaNet layer, a missing tensor and a wrong shape or type
    before copying anything (no GPU call is reached)."""
    path, _, _ = model
    lib = _lib.load()
    err = ctypes.create_string_buffer(256)
    with GgufFile(path) as g:
        c = g.attn_config()
        assert not lib.clef_hip_gguf_attn_layer(g._h, ctypes.byref(c), 0, None, None, None, None, None, err, 256)
        assert b"not a full-attention layer" in err.value
        assert not lib.clef_hip_gguf_attn_layer(g._h, ctypes.byref(c), 3, None, None, None, None, None, err, 256)
        assert b"out of range" in err.value
        c.nh = 8   # geometry that does not match the stored tensors
        assert not lib.clef_hip_gguf_attn_layer(g._h, ctypes.byref(c), 1, None, None, None, None, None, err, 256)
        assert b"blk.1.attn_qkv.weight" in err.value and b"expected type 30" in err.value
        assert not lib.clef_hip_gguf_vis_layer(g._h, 0, 3, None, None, None, None, None, err, 256)
        assert b"v.blk.0.attn_qkv.weight" in err.value
        assert not lib.clef_hip_gguf_vis_layer(g._h, 1, 2, None, None, None, None, None, err, 256)
        assert b"missing tensor v.blk.1" in err.value
    # a norm stored as BF16 instead of F32
    p = tmp_path / "t.gguf"
    arrays, _ = gw.clef_attention_model(p, layer_types=(1,))
    tensors = [(k, gw.GGML_BF16 if k.endswith("q_norm.weight") else
                (gw.GGML_BF16 if a.dtype == np.uint16 else (gw.GGML_F16 if a.dtype == np.float16 else gw.GGML_F32)),
                gw.bf16_bits(a) if k.endswith("q_norm.weight") else a) for k, a in arrays.items()]
    kvs = [("general.architecture", gw.STRING, "clef"), ("clef.block_count", gw.U32, 1),
           ("clef.embedding_length", gw.U32, 128), ("clef.attention.head_count", gw.U32, 4),
           ("clef.attention.head_count_kv", gw.U32, 2), ("clef.attention.key_length", gw.U32, 256),
           ("clef.rope.dimension_count", gw.U32, 64), ("clef.attention.layer_norm_rms_epsilon", gw.F32, 1e-6),
           ("clef.rope.freq_base", gw.F32, 1e7), ("clef.layer_types", gw.ARRAY, (gw.I32, [1]))]
    gw.write(p, kvs, tensors)
    with GgufFile(p) as g:
        c = g.attn_config()
        assert not lib.clef_hip_gguf_attn_layer(g._h, ctypes.byref(c), 0, None, None, None, None, None, err, 256)
        assert b"attn_q_norm.weight has type 30" in err.value


def _raw_gguf(meta_blobs, tensor_blobs=b"", n_tensors=0, tail=b"\0" * 64):
    """A GGUF from already-encoded metadata entries (key + type + value bytes) and tensor entries."""
    import struct
    return struct.pack("<IIQQ", 0x46554747, 3, n_tensors, len(meta_blobs)) + b"".join(meta_blobs) + tensor_blobs + tail


def _entry(key, t, value_bytes):
    import struct
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<I", t) + value_bytes


def _arr(et, n, body=b""):
    import struct
    return struct.pack("<IQ", et, n) + body


@pytest.mark.parametrize("case", ["str_depth1", "str_depth2", "str_depth3", "arr_depth3_scalars", "arr_depth3_strings",
                                  "empty_bad_elem", "one_bad_elem", "bad_scalar_type", "align_i32", "align_u32_64",
                                  "misaligned_offset", "overlap", "huge_count_scalars", "rank5", "zero_extent"])
def test_edge_files_agree_with_reference(tmp_path, case):
    """Hand-built files at the edges of the acceptance rules: array nesting (strings and arrays
    inside at most two arrays), empty arrays of an unknown element type, an alignment key of the
    wrong type, tensor offsets that are unaligned or overlap. Both readers decide alike and, where
    they accept, give the same table."""
    import struct
    s = lambda x: struct.pack("<Q", len(x)) + x
    strs = lambda *xs: b"".join(s(x) for x in xs)
    tensor = lambda name, dims, t, off: s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", t, off)
    expect = None
    meta, tens, nt = [], b"", 0
    if case == "str_depth1":
        meta = [_entry("a", 9, _arr(8, 2, strs(b"x", b"yy")))]; expect = True
    elif case == "str_depth2":
        meta = [_entry("a", 9, _arr(9, 1, _arr(8, 1, strs(b"x"))))]; expect = True
    elif case == "str_depth3":
        meta = [_entry("a", 9, _arr(9, 1, _arr(9, 1, _arr(8, 1, strs(b"x")))))]; expect = False
    elif case == "arr_depth3_scalars":
        meta = [_entry("a", 9, _arr(9, 1, _arr(9, 1, _arr(4, 2, b"\0" * 8))))]; expect = True
    elif case == "arr_depth3_strings":
        meta = [_entry("a", 9, _arr(9, 1, _arr(9, 1, _arr(9, 0))))]; expect = True
    elif case == "empty_bad_elem":
        meta = [_entry("a", 9, _arr(77, 0))]; expect = True
    elif case == "one_bad_elem":
        meta = [_entry("a", 9, _arr(77, 1, b"\0" * 8))]; expect = False
    elif case == "bad_scalar_type":
        meta = [_entry("a", 13, b"\0" * 8)]; expect = False
    elif case == "align_i32":   # not a u32: the default 32 applies
        meta = [_entry("general.alignment", 5, struct.pack("<i", 48))]; tens = tensor(b"t", [4], 0, 0); nt = 1; expect = True
    elif case == "align_u32_64":
        meta = [_entry("general.alignment", 4, struct.pack("<I", 64))]; tens = tensor(b"t", [4], 0, 0); nt = 1; expect = True
    elif case == "misaligned_offset":
        tens = tensor(b"t", [3], 30, 6) + tensor(b"u", [2], 0, 3); nt = 2; expect = True
    elif case == "overlap":
        tens = tensor(b"t", [8], 0, 0) + tensor(b"u", [8], 0, 4); nt = 2; expect = True
    elif case == "huge_count_scalars":
        meta = [_entry("a", 9, _arr(10, 1 << 61))]; expect = False
    elif case == "rank5":
        tens = tensor(b"t", [1, 1, 1, 1, 1], 0, 0); nt = 1; expect = False
    elif case == "zero_extent":
        tens = tensor(b"t", [4, 0], 0, 0); nt = 1; expect = False
    p = tmp_path / "e.gguf"
    p.write_bytes(_raw_gguf(meta, tens, nt, tail=b"\0" * 256))
    ok_o, ours = _our_table(p)
    assert ok_o == expect
    lib = _ref_lib()
    if lib is not None:
        ok_r, ref = _ref_table(lib, p)
        assert ok_r == ok_o
        if ok_o:
            assert ours == ref
