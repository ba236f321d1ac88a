"""Host-side producers of the attention path's inputs, through the C ABI: M-RoPE positions of a
record with image / video-frame spans (clef_record.c:938-962) and the server's micro-batch
packing (clef_server.c:311-327)."""
import ctypes

import numpy as np

from . import _lib


def _i32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def record_positions(T, spans=(), merge=2, given=None):
    """pos3 [T][3] int32 of one record. spans: (token start, grid_h, grid_w) per vision span in
    token order (grid sizes in patches, before the merge). given: the record's own [T][3]
    positions (an Omni record's), copied as they are."""
    lib = _lib.load()
    sp = np.asarray(spans, dtype=np.int32).reshape(-1, 3)
    start, gh, gw = (np.ascontiguousarray(sp[:, i]) for i in range(3))
    pos3 = np.zeros((max(T, 1), 3), dtype=np.int32)
    if given is not None:
        given = np.ascontiguousarray(given, dtype=np.int32)
        if given.shape != (T, 3):
            raise ValueError(f"given positions have shape {given.shape}, expected ({T}, 3)")
    err = ctypes.create_string_buffer(256)
    ok = lib.clef_hip_record_positions(int(T), None if given is None else _i32p(given), _i32p(start), _i32p(gh),
                                       _i32p(gw), len(sp), int(merge), _i32p(pos3), err, len(err))
    _lib.check(ok, err)
    return pos3[:T]


def pack_batch(lengths, keyed=None, max_batch=64, max_tokens=16384):
    """Records taken from the head of a FIFO queue for one micro-batch: (n, cu_seqlens[n + 1])."""
    lib = _lib.load()
    ln = np.ascontiguousarray(lengths, dtype=np.int32)
    ky = None if keyed is None else np.ascontiguousarray(keyed, dtype=np.uint8)
    cu = np.zeros(len(ln) + 1, dtype=np.int32)
    n = lib.clef_hip_pack_batch(_i32p(ln), None if ky is None else ky.ctypes.data, len(ln), int(max_batch),
                                int(max_tokens), _i32p(cu))
    return n, cu[: n + 1].copy()
