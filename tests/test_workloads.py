"""Synthetic BASELINE workloads: shapes and the C1 length draw."""
import numpy as np

from cleffa_amd import workloads


def test_c1_lengths():
    for seed in range(20):
        lengths = workloads.c1_lengths(seed)
        assert len(lengths) == 8 and sum(lengths) == 4096 and min(lengths) >= 1
    assert workloads.c1_lengths(0) == workloads.c1_lengths(0)


def test_config_shapes():
    w = workloads.config("C1")
    assert w["qkv"].shape == (4096, 2 * 24 * 256 + 2 * 4 * 256)
    assert w["pos3"].shape == (4096, 3) and int(w["cu_seqlens"][-1]) == 4096
    w = workloads.config("C3")
    assert w["qkv"].shape[0] == 2048 and w["k_cache"].shape == (4, 10240, 256)
    assert int(w["pos3"][0, 0]) == 2048 and int(w["pos3"][-1, 0]) == 2559
    w = workloads.config("C4")
    assert w["qkv"].shape == (4096, 3 * 16 * 72) and w["pos2"].shape == (4096, 2)
    assert int(w["pos2"].max()) == 31
    w = workloads.config("C0")
    assert w["q_norm"] is None and w["n_rot"] == 0 and not w["gate"]
