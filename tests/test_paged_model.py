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
