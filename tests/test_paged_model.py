"""Pin the page-table model (oracle/paged.py) with invariants that tie it to
the reference's contiguous cache semantics (kvcache.go:240-388)."""
import copy

import numpy as np
import pytest

import oracle
from oracle.paged import PagedModel, PagedOverflow, PagedPoolExhausted, PagedStateError


def _snapshot(m, layer):
    return (m.table[layer].copy(), list(m.free[layer]), m.len[layer].copy(),
            m.first[layer].copy(), m.pages[layer].copy(), m.pos_offset[layer].copy())


def _same(a, b):
    return all(np.array_equal(x, y) if isinstance(x, np.ndarray) else x == y for x, y in zip(a, b))


def test_rollback_restores_exact_state():
    rng = np.random.default_rng(0)
    for trial in range(50):
        m = PagedModel(1, 16, 64, 4, 16)
        seqs = [0, 1, 2, 3]
        a = rng.integers(0, 40, size=4).tolist()
        m.append(0, seqs, a)
        before = _snapshot(m, 0)
        b = rng.integers(0, 40, size=4).tolist()
        m.append(0, seqs, b)
        for s, n in zip(seqs, b):
            m.rollback(0, s, n)
        # rollback in call order frees pages in reverse of their allocation
        # only when sequences are rolled back last-allocated first; compare
        # the per-sequence state and the free-set, then the exact stack for
        # the reverse order.
        after = _snapshot(m, 0)
        assert np.array_equal(after[0], before[0])
        assert sorted(after[1]) == sorted(before[1])
        m2 = PagedModel(1, 16, 64, 4, 16)
        m2.append(0, seqs, a)
        m2.append(0, seqs, b)
        for s, n in reversed(list(zip(seqs, b))):
            m2.rollback(0, s, n)
        assert _same(_snapshot(m2, 0), before)


def test_contiguous_semantics_single_sequence():
    """gather(seq) equals the bytes a contiguous KVCache holds after the same
    decode appends (KVH*D rows, kvcache.go:407-423 with n=1 per call)."""
    rng = np.random.default_rng(1)
    KVH, D, P = 2, 8, 16
    m = PagedModel(1, P, 8, 1, 8)
    cap = 8 * P
    ref = np.zeros(cap * KVH * D, np.uint16)
    T = 0
    for step in range(70):
        k = rng.normal(size=(KVH, 1, D)).astype(np.float32)
        oracle.kv_copy_into(ref, k, T, 1, KVH * D)
        m.append(0, [0], [1], payloads=[[oracle.bf16_from_f32(k[:, 0, :])]])
        T += 1
    dense = np.stack(m.rows[0][0], axis=1)            # [KVH, T, D]
    image = ref[: T * KVH * D].reshape(T, KVH, D)     # token-major rows
    assert np.array_equal(dense, image.transpose(1, 0, 2))
    # every live token has a distinct (page, slot)
    locs = {m.token_location(0, 0, t) for t in range(T)}
    assert len(locs) == T


def test_evict_compact_preserve_order_and_positions():
    m = PagedModel(2, 16, 40, 2, 10)
    m.append(0, [0, 1], [100, 33], payloads=[list(range(100)), list(range(33))])
    m.append(1, [0, 1], [100, 33], payloads=[list(range(100)), list(range(33))])
    full = 100 // 16
    m.evict(-1, 0, full // 4 + 1)
    assert m.state(0, 0) == {"len": 100 - 32, "first": 2, "pos_offset": 32, "pages": 5}
    rows_before = list(m.rows[0][0])
    live_pages = [m.token_location(0, 0, t)[0] for t in range(0, m.state(0, 0)["len"], 16)]
    m.compact(-1)
    assert m.state(0, 0)["first"] == 0
    assert list(m.table[0][0][:5]) == live_pages and np.all(m.table[0][0][5:] == -1)
    assert m.rows[0][0] == rows_before == list(range(32, 100))
    # all pages accounted for: live + free == pool
    used = sum(int(m.pages[0, s]) for s in range(2))
    assert used + len(m.free[0]) == 40


def test_failures_leave_state_unchanged():
    m = PagedModel(1, 16, 4, 2, 3)
    m.append(0, [0], [20])
    snap = _snapshot(m, 0)
    with pytest.raises(PagedOverflow):
        m.append(0, [0], [29])           # 49 tokens > 3 pages
    assert _same(_snapshot(m, 0), snap)
    with pytest.raises(PagedPoolExhausted):
        m.append(0, [0, 1], [10, 40])    # needs 3 more pages, 2 free
    assert _same(_snapshot(m, 0), snap)
    with pytest.raises(PagedStateError):
        m.rollback(0, 0, 21)
    with pytest.raises(PagedStateError):
        m.evict(0, 0, 2)                 # only one full page
    assert _same(_snapshot(m, 0), snap)


def test_release_and_reset_return_every_page():
    m = PagedModel(1, 16, 16, 3, 8)
    m.append(0, [0, 1, 2], [17, 50, 3])
    m.release(0, 1)
    assert m.state(0, 1) == {"len": 0, "first": 0, "pos_offset": 0, "pages": 0}
    m2 = copy.deepcopy(m)
    m2.reset()
    assert m2.free[0] == list(range(15, -1, -1))


# ---- host spill tier -------------------------------------------------------

def _device_state(m, layer):
    return _snapshot(m, layer) + (m.rows[layer],)


def _fill(m, rng, seqs, lo=20, hi=120):
    n = rng.integers(lo, hi, size=len(seqs)).tolist()
    for layer in range(m.layers):
        m.append(layer, seqs, n, payloads=[[(layer, s, t) for t in range(int(m.len[layer, s]), int(m.len[layer, s]) + k)]
                                          for s, k in zip(seqs, n)])
    return n


def test_spill_is_evict_on_the_device_and_restore_undoes_it():
    rng = np.random.default_rng(7)
    for trial in range(40):
        m = PagedModel(2, 16, 64, 3, 12, host_slots=48)
        _fill(m, rng, [0, 1, 2])
        before = copy.deepcopy(m)
        n = [int(rng.integers(0, int(m.len[0, s]) // 16 + 1)) for s in range(3)]
        e = copy.deepcopy(m)
        m.spill(-1, [0, 1, 2], n)
        for s in range(3):
            e.evict(-1, s, n[s])
        for layer in range(2):
            assert _same(_device_state(m, layer), _device_state(e, layer))
        assert len(m.host_free) == 48 - 2 * sum(n)
        assert [slot for slot, _ in m.spilled[0][0]] == list(range(n[0]))  # slots 0, 1, 2, ... in order
        m.restore(-1, [0, 1, 2], n)
        for layer in range(2):
            for s in range(3):
                assert m.rows[layer][s] == before.rows[layer][s]
                assert m.state(layer, s) == before.state(layer, s)
        assert sorted(m.host_free) == list(range(48))
        # every page is live or free, and the live pages are distinct
        live = [int(p) for s in range(3) for p in m.table[0][s] if p >= 0]
        assert len(set(live)) == len(live) == int(m.pages[0].sum())
        assert len(live) + len(m.free[0]) == 64


def test_restore_moves_live_entries_right_when_the_front_is_short():
    m = PagedModel(1, 16, 32, 1, 8, host_slots=8)
    m.append(0, [0], [80], payloads=[list(range(80))])
    m.spill(0, [0], [3])
    m.compact(0)                         # first = 0: no room in front
    assert m.state(0, 0)["first"] == 0
    live = list(m.table[0][0][:2])
    m.restore(0, [0], [2])
    assert m.state(0, 0) == {"len": 64, "first": 0, "pos_offset": 16, "pages": 4}
    assert list(m.table[0][0][2:4]) == live
    assert m.rows[0][0] == list(range(16, 80))
    m.restore(0, [0], [1])
    assert m.rows[0][0] == list(range(80)) and m.state(0, 0)["pos_offset"] == 0


def test_evict_after_spill_drops_the_spilled_pages():
    m = PagedModel(1, 16, 32, 2, 10, host_slots=6)
    m.append(0, [0, 1], [96, 40])
    m.spill(0, [0], [2])
    m.evict(0, 0, 1)
    assert m.spilled[0][0] == [] and sorted(m.host_free) == list(range(6))
    assert m.state(0, 0)["pos_offset"] == 48
    with pytest.raises(PagedStateError):
        m.restore(0, [0], [1])


def test_spill_and_restore_failures_leave_state_unchanged():
    m = PagedModel(1, 16, 12, 2, 6, host_slots=3)
    m.append(0, [0, 1], [64, 80])
    snap = copy.deepcopy(m)
    with pytest.raises(PagedPoolExhausted):
        m.spill(0, [0, 1], [2, 2])       # 4 slots needed, 3 free
    with pytest.raises(PagedStateError):
        m.spill(0, [0], [5])             # 4 full pages
    assert _same(_device_state(m, 0), _device_state(snap, 0)) and m.host_free == snap.host_free
    m.spill(0, [0, 1], [1, 2])
    snap = copy.deepcopy(m)
    with pytest.raises(PagedStateError):
        m.restore(0, [0], [2])           # one spilled page
    with pytest.raises(PagedStateError):
        m.restore(0, [1, 1], [1, 1])
    m.append(0, [0], [16 * 2])           # first 1 + 5 pages == max_pages
    m.compact(0)
    m.append(0, [0], [16])               # first 0 + 6 pages == max_pages
    snap = copy.deepcopy(m)
    with pytest.raises(PagedOverflow):
        m.restore(0, [0], [1])           # 6 live pages + 1 restored > 6 entries
    assert _same(_device_state(m, 0), _device_state(snap, 0))
    m2 = copy.deepcopy(snap)
    m2.free[0] = []
    with pytest.raises(PagedPoolExhausted):
        m2.restore(0, [1], [1])
    m.release(0, 1)
    assert [s for s, _ in m.spilled[0][1]] == [] and len(m.host_free) == 2
