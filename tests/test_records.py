"""Host producers of the path's inputs (C ABI, no GPU): M-RoPE positions of records with image
and video-frame spans against transformers' Qwen3.5 get_rope_index, and the server's FIFO
micro-batch packing on the cases its own comments name (clef_server.c:311-327)."""
import types

import numpy as np
import pytest
import torch

from cleffa_amd.records import pack_batch, record_positions


def _hf_positions(T, spans, merge=2):
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    ids = torch.zeros(1, T, dtype=torch.long)
    types_ = torch.zeros(1, T, dtype=torch.int32)
    grids = []
    for start, gh, gw in spans:
        n = (gh // merge) * (gw // merge)
        types_[0, start:start + n] = 1
        grids.append([1, gh, gw])
    fake = types.SimpleNamespace(config=types.SimpleNamespace(vision_config=types.SimpleNamespace(spatial_merge_size=merge)))
    fake.get_vision_position_ids = lambda *a, **k: hf.Qwen3_5Model.get_vision_position_ids(fake, *a, **k)
    pos, _ = hf.Qwen3_5Model.get_rope_index(fake, ids, types_, image_grid_thw=torch.tensor(grids) if grids else None)
    return pos[:, 0].T.numpy().astype(np.int32)


@pytest.mark.parametrize("T,spans", [
    (7, []),
    (30, [(3, 4, 6)]),                          # 2 x 3 merged grid after 3 text tokens
    (60, [(0, 8, 4), (9, 2, 2), (20, 6, 10)]),  # image first, one text token between spans, a wide grid
    (400, [(5, 32, 32), (300, 4, 8), (330, 4, 8), (360, 4, 8)]),   # an image, then video frames with text between
])
def test_positions_match_hf_get_rope_index(T, spans):
    np.testing.assert_array_equal(record_positions(T, spans), _hf_positions(T, spans))


def test_text_only_positions_count_up():
    np.testing.assert_array_equal(record_positions(5), np.repeat(np.arange(5, dtype=np.int32)[:, None], 3, 1))


@pytest.mark.parametrize("T,spans,msg", [
    (10, [(2, 3, 4)], "multiple of the merge"),
    (10, [(2, 8, 8)], "runs past"),
    (20, [(2, 2, 2), (2, 2, 2)], "inside or before"),
    (10, [(12, 2, 2)], "past the record"),
])
def test_position_errors(T, spans, msg):
    with pytest.raises(RuntimeError, match=msg):
        record_positions(T, spans)


def test_pack_fifo_within_budget():
    n, cu = pack_batch([100, 200, 300, 400], max_batch=8, max_tokens=600)
    assert n == 3 and cu.tolist() == [0, 100, 300, 600]   # the budget is inclusive


def test_pack_head_always_taken_and_runs_alone_when_oversized():
    n, cu = pack_batch([5000, 10, 10], max_batch=8, max_tokens=1000)
    assert n == 1 and cu.tolist() == [0, 5000]


def test_pack_stops_at_first_misfit_fifo():
    n, _ = pack_batch([500, 600, 10], max_batch=8, max_tokens=1000)
    assert n == 1   # the small third request waits behind the second (no reordering)


def test_pack_max_batch():
    n, cu = pack_batch([1] * 10, max_batch=4, max_tokens=1 << 20)
    assert n == 4 and cu.tolist() == [0, 1, 2, 3, 4]


def test_pack_keyed_requests_run_alone():
    assert pack_batch([10, 10, 10], keyed=[1, 0, 0], max_batch=8)[0] == 1
    assert pack_batch([10, 10, 10], keyed=[0, 0, 1], max_batch=8)[0] == 2
    assert pack_batch([], max_batch=8)[0] == 0


def test_adjacent_spans_stay_separate():
    # clef_record.c:947-956 walks images one by one, so two 1x1 merged grids back to back take
    # positions 0 and 1 (transformers would read them as one 1x2 run of vision tokens).
    np.testing.assert_array_equal(record_positions(3, [(0, 2, 2), (1, 2, 2)]),
                                  [[0, 0, 0], [1, 1, 1], [2, 2, 2]])


def test_given_positions_are_copied():
    """A record that carries its own positions (clef_record.c:939-942, r->pos3: an Omni record's
    precomputed [T][3]) gets them back as they are; spans are not read."""
    rng = np.random.default_rng(3)
    given = rng.integers(-5, 1000, size=(7, 3)).astype(np.int32)
    np.testing.assert_array_equal(record_positions(7, [(0, 2, 2)], given=given), given)
    np.testing.assert_array_equal(record_positions(0, given=np.zeros((0, 3), np.int32)), np.zeros((0, 3), np.int32))
    with pytest.raises(ValueError, match="expected"):
        record_positions(7, given=given[:5])
