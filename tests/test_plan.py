"""Host-side plan builder (clef_hip_attn_plan, the block list of clef_metal.m:1243-1257 and the
packing of clef.c:470-497): coverage, key ranges, order and kv-row layout. Runs on the CPU."""
import numpy as np
import pytest

from cleffa_amd import AttnPlan
from cleffa_amd._lib import BLOCK_Q, KV_ALIGN


def _check_plan(cu_q, cu_k, causal):
    plan = AttnPlan(cu_q, cu_k, causal=causal, device="cpu")
    b = plan.blocks_host
    T = int(cu_q[-1])
    seen = np.zeros(T, np.int32)
    for e in b:
        q_row0, nq, q_pos0, k_row0, k_len, flag_row, rec, _ = (int(x) for x in e)
        assert 1 <= nq <= BLOCK_Q
        seen[q_row0:q_row0 + nq] += 1
        lq = cu_q[rec + 1] - cu_q[rec]
        lk = lq if cu_k is None else cu_k[rec + 1] - cu_k[rec]
        L = lk - lq
        i0 = q_row0 - cu_q[rec]
        assert i0 % BLOCK_Q == 0 and q_pos0 == L + i0 and flag_row == cu_q[rec]
        assert k_len == (min(lk, L + i0 + nq) if causal else lk)
        if cu_k is not None:
            assert k_row0 == cu_k[rec]
        # whole 64-key tiles from the record's first key stay inside the planes
        assert k_row0 + -(-lk // 64) * 64 <= plan.kv_rows
    assert (seen == 1).all(), "every pass row in exactly one block"
    assert (np.diff(b[:, 4]) <= 0).all(), "blocks ordered longest first"
    # pass row -> kv row: a record's tokens are its last keys, in order
    for r in range(len(cu_q) - 1):
        rows = plan.tok_kv_host[cu_q[r]:cu_q[r + 1]]
        lq = cu_q[r + 1] - cu_q[r]
        lk = lq if cu_k is None else cu_k[r + 1] - cu_k[r]
        k0 = rows[0] - (lk - lq) if lq else None
        if lq:
            assert (np.diff(rows) == 1).all()
            if cu_k is None:
                assert k0 % KV_ALIGN == 0
            else:
                assert k0 == cu_k[r]
    # plane row -> pass row: the exact inverse of tok_kv, -1 everywhere else
    inv = np.full(plan.kv_rows, -1, np.int32)
    inv[plan.tok_kv_host] = np.arange(T, dtype=np.int32)
    np.testing.assert_array_equal(plan.kv_tok_host, inv)
    return plan


@pytest.mark.parametrize("lengths", [[1], [1160, 890, 730, 425, 472, 136, 179, 104], [127, 128, 129, 1, 256],
                                     [0, 5, 0, 300], [16384]])
@pytest.mark.parametrize("causal", [True, False])
def test_fresh_plans(lengths, causal):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    plan = _check_plan(cu, None, causal)
    assert plan.n_blk == sum(-(-n // BLOCK_Q) for n in lengths)


def test_prefix_plan():
    cu_q = np.array([0, 512, 1024, 1536, 2048], np.int32)
    cu_k = np.array([0, 2560, 5120, 7680, 10240], np.int32)
    plan = _check_plan(cu_q, cu_k, True)
    assert plan.kv_rows == 10240
    assert plan.pairs() == 4 * (512 * 2048 + 512 * 513 // 2)


def test_empty_pass():
    plan = AttnPlan(np.array([0], np.int32), device="cpu")
    assert plan.n_blk == 0 and plan.kv_rows == 0


@pytest.mark.parametrize("cu_q,cu_k,msg", [
    ([0, 5, 3], None, "decreases"),
    ([1, 5], None, "start at 0"),
    ([0, 10], [0, 5], "keys for"),
    ([0, 4, 8], [0, 12, 20], "not a multiple of 8"),
])
def test_plan_errors(cu_q, cu_k, msg):
    with pytest.raises(RuntimeError, match=msg):
        AttnPlan(np.array(cu_q, np.int32), None if cu_k is None else np.array(cu_k, np.int32), device="cpu")


def test_pairs_counts_causal_and_bidirectional():
    cu = np.array([0, 3, 10], np.int32)
    assert AttnPlan(cu, device="cpu").pairs() == 6 + 28
    assert AttnPlan(cu, causal=False, device="cpu").pairs() == 9 + 49


def _sched(plan, nh, nkv, n_wg):
    import ctypes
    from cleffa_amd import _lib
    lib = _lib.load()
    n = lib.clef_hip_attn_sched_size(plan.n_blk, nh, n_wg)
    out = np.zeros(max(n, 1), np.int32)
    err = ctypes.create_string_buffer(256)
    b = np.ascontiguousarray(plan.blocks_host, dtype=np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    ok = lib.clef_hip_attn_schedule(p(b), plan.n_blk, nh, nkv, n_wg, p(out), len(out), err, len(err))
    return ok, out, err.value.decode()


def _item_cost(plan, nh, it):
    """An item's modelled cost: its 64-key tiles (a first half's keys end at its last row) + 6."""
    e = plan.blocks_host[(it & ((1 << 28) - 1)) // nh]
    k_len = min(int(e[4]), int(e[2]) + 64) if (it >> 28) & 3 == 1 else int(e[4])
    return (k_len + 63) // 64 + 6


@pytest.mark.parametrize("lengths,nh,nkv,n_wg", [
    ([1160, 890, 730, 425, 472, 136, 179, 104], 24, 4, 256),   # C1: heads split over the 8 XCDs
    ([16384], 24, 4, 256),
    ([512] * 4, 16, 4, 256),                                     # as many items as workgroups
    ([300, 17, 1], 12, 4, 7),                                    # no XCD split
    ([5], 2, 1, 300),                                            # more workgroups than items
    ([1000], 16, 4, 256),                                        # C0-like: blocks split in halves
    ([700, 130, 64, 65, 1], 8, 2, 256),                          # halves only for blocks > 64 rows
    ([16] * 256, 24, 4, 256),                                    # short records: every block packed
])
def test_schedule_covers_items_balanced(lengths, nh, nkv, n_wg):
    """clef_hip_attn_schedule: every (block, head) item exactly once, whole or (when the pass
    has fewer items than workgroups and the block more than 64 rows) as its two 64-row halves;
    each workgroup's items longest first, items of an XCD's heads only on that XCD's workgroups,
    and greedy balance (no workgroup above the mean load by more than one item's cost)."""
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    plan = AttnPlan(cu, causal=True, device="cpu")
    ok, s, err = _sched(plan, nh, nkv, n_wg)
    assert ok, err
    # the header names the plan: its sizes and the fingerprint in word 7 of every block entry
    fp = plan.blocks_host[:, 7]
    assert plan.n_blk == 0 or (fp == fp[0]).all() and fp[0] != 0
    assert s[:8].tolist() == [0x53434844, plan.n_blk, nh, n_wg, nkv, int(fp[0]) if plan.n_blk else s[5], 0, 0]
    s = s[8:]
    off = s[: n_wg + 1]
    items = s[n_wg + 1: n_wg + 1 + off[-1]]
    split_pass = plan.n_blk * nh < n_wg
    group = nh // nkv

    def pack(nq):   # heads per packed item (pack_heads in attn_text.h)
        if split_pass or nq > 64:
            return 1
        wph = -(-nq // 16)
        return next((k for k in range(8 // wph, 1, -1) if group % k == 0), 1)

    pairs = (nh // nkv) % 2 == 0
    want = []
    for it in range(plan.n_blk * nh):
        nq = int(plan.blocks_host[it // nh][1])
        if split_pass and nq > 64:
            want += [it | (1 << 28), it | (2 << 28)]
        elif nq > 64 and pairs:   # the block's halves, each for heads h and h + 1 (bit 30)
            if (it % nh) % 2 == 0:
                want += [it | (1 << 28) | (1 << 30), it | (2 << 28) | (1 << 30)]
        elif pack(nq) > 1:
            if (it % nh) % pack(nq) == 0:
                want.append(it | (3 << 28))
        else:
            want.append(it)
    # every (block, head) exactly once: whole, as two halves, or inside one packed item
    covered = {}
    for it in items.tolist():
        base, code, pair = it & ((1 << 28) - 1), (it >> 28) & 3, (it >> 30) & 1
        heads = range(base % nh, base % nh + pack(int(plan.blocks_host[base // nh][1]))) if code == 3 else \
            [base % nh, base % nh + 1] if pair else [base % nh]
        for h in heads:
            key = (base // nh, h)
            covered[key] = covered.get(key, 0) + (1 if code in (0, 3) else 0.5)
    assert covered == {(b, h): 1 for b in range(plan.n_blk) for h in range(nh)}
    assert off[0] == 0 and (np.diff(off) >= 0).all() and off[-1] == len(want)
    assert sorted(items.tolist()) == sorted(want)
    cost = lambda it: _item_cost(plan, nh, it)
    head = lambda it: (it & ((1 << 28) - 1)) % nh
    xh = nh // 8 if nh % 8 == 0 and ((nh // nkv) % (nh // 8) == 0 or (nh // 8) % (nh // nkv) == 0) else 0
    split = xh and n_wg % 8 == 0
    loads = []
    for b in range(n_wg):
        mine = items[off[b]:off[b + 1]].tolist()
        c = [cost(it) for it in mine]
        assert c == sorted(c, reverse=True)
        if split:   # on an XCD of one of its heads (a packed item may span two)
            for it in mine:
                hk = pack(int(plan.blocks_host[(it & ((1 << 28) - 1)) // nh][1])) if (it >> 28) & 3 == 3 else \
                    2 if (it >> 30) & 1 else 1
                assert head(it) // xh <= b % 8 <= (head(it) + hk - 1) // xh
        loads.append(sum(c))
    groups = 8 if split else 1
    for x in range(groups):
        ld = loads[x::groups]
        mine = [it for b in range(x, n_wg, groups) for it in items[off[b]:off[b + 1]].tolist()]
        tot = sum(cost(it) for it in mine)
        biggest = max([cost(it) for it in mine], default=0)
        assert max(ld) <= tot / len(ld) + biggest
    if split_pass and len(want) <= n_wg and not split:
        assert max(len(items[off[b]:off[b + 1]]) for b in range(n_wg)) == 1
    if len(want) >= n_wg:   # every workgroup has work, also when every item is packed
        assert min(len(items[off[b]:off[b + 1]]) for b in range(n_wg)) >= 1


def test_schedule_errors():
    plan = AttnPlan(np.array([0, 100], np.int32), causal=True, device="cpu")
    ok, _, err = _sched(plan, 6, 4, 8)       # nh not a multiple of nkv
    assert not ok and "bad schedule" in err


def test_schedule_local_search_reaches_c1_bound():
    """C1 (24/4 heads, 256 workgroups): with the 8- and 41/51-row blocks packed several heads to
    an item and the blocks of more than 64 rows run as halves for two heads each, 10,048 tiles of
    modelled cost (tiles + 6 per item); the local search brings every workgroup to at most 41,
    within two tiles of the per-workgroup mean (39.25; a packed item sits on the XCD of its first
    head, so the XCDs' totals differ by a few tiles)."""
    lengths = [1160, 890, 730, 425, 472, 136, 179, 104]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    plan = AttnPlan(cu, causal=True, device="cpu")
    ok, s, err = _sched(plan, 24, 4, 256)
    assert ok, err
    off = s[8:265]
    items = s[265:265 + off[-1]]
    cost = lambda it: _item_cost(plan, 24, it)
    loads = [sum(cost(it) for it in items[off[b]:off[b + 1]]) for b in range(256)]
    assert sum(loads) == 10048 and max(loads) <= 41


def _fnv_fingerprint(blocks):
    """FNV-1a (32-bit, offset basis 2166136261, prime 16777619) over the little-endian bytes of
    words 0-6 of every entry, with bit 0 forced on."""
    h = 2166136261
    for e in np.asarray(blocks, np.int32):
        for byte in e[:7].astype("<i4").tobytes():
            h = ((h ^ byte) * 16777619) & 0xFFFFFFFF
    return np.int32(np.uint32(h | 1).view(np.int32))


def test_plan_fingerprint():
    """Word 7 of every block entry is the FNV-1a fingerprint of the list (textbook FNV-1a, written
    out here); plans that differ in any block differ in it, and the schedule header repeats it."""
    seen = set()
    for lengths in ([1160, 890, 730, 425, 472, 136, 179, 104], [1160, 890, 730, 425, 472, 136, 180, 103],
                    [100, 20], [20, 100], [300]):
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        plan = AttnPlan(cu, causal=True, device="cpu")
        fp = _fnv_fingerprint(plan.blocks_host)
        assert (plan.blocks_host[:, 7] == fp).all()
        seen.add(int(fp))
        ok, s, err = _sched(plan, 24, 4, 256)
        assert ok and s[5] == fp and s[4] == 4
    assert len(seen) == 5
    # FNV-1a known answer: the empty input hashes to the offset basis
    assert _fnv_fingerprint(np.zeros((0, 8), np.int32)) == np.int32(np.uint32(2166136261 | 1).view(np.int32))
