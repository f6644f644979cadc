"""GPU parity of the paged cache state machine and byte movement.

Every check is bit-exact: cache contents (via the paged gather) against
BF16FromF32 of the appended rows in logical order (the oracle), page tables
and free lists against oracle/paged.py.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle.paged import PagedModel

pytestmark = pytest.mark.gpu


def _kv(gpu, **kw):
    from relux_amd import KVCache
    return KVCache(device=gpu.index, **kw)


def _mla(gpu, **kw):
    from relux_amd import MLACache
    return MLACache(device=gpu.index, **kw)


def test_reference_kvcache_known_answers(gpu):
    """kvcache_test.go:16-106 through the drop-in API."""
    c = _kv(gpu, num_layers=2, max_len=16, num_kv_heads=2, head_dim=64)
    assert c.TotalLen(0) == 0
    k = torch.arange(1, 2 * 64 + 1, dtype=torch.float32, device=gpu).reshape(1, 2, 1, 64)
    c.Append(0, k, k + 1000)
    assert c.TotalLen(0) == 1 and c.TotalLen(1) == 0 and c.TotalLen(7) == 0
    ck, cv = c.View(0)
    assert tuple(ck.shape) == (1, 2, 1, 64)
    want = oracle.round_bf16(k.cpu().numpy())
    assert np.array_equal(ck.float().cpu().numpy(), want)
    assert np.array_equal(cv.float().cpu().numpy(), oracle.round_bf16((k + 1000).cpu().numpy()))
    k2 = torch.arange(9, 9 + 2 * 2 * 64, dtype=torch.float32, device=gpu).reshape(1, 2, 2, 64)
    c.Append(0, k2, k2)
    assert c.TotalLen(0) == 3
    ck, _ = c.View(0)
    full = np.concatenate([k.cpu().numpy(), k2.cpu().numpy()], axis=2)
    assert np.array_equal(ck.float().cpu().numpy(), oracle.round_bf16(full))
    c.Reset()
    assert c.TotalLen(0) == 0 and c.View(0) == (None, None)


def test_errors_mirror_reference_panics(gpu):
    from relux_amd import ReluxError, ReluxPanic
    c = _kv(gpu, num_layers=1, max_len=32, num_kv_heads=1, head_dim=64, max_seqs=2, pool_pages=3)
    x = torch.zeros(1, 1, 20, 64, device=gpu)
    c.Append(0, x, x)
    tab = c.PageTable(0, 0)
    with pytest.raises(ReluxPanic):                 # kvcache.go:282-285
        c.Append(0, torch.zeros(1, 1, 13, 64, device=gpu), torch.zeros(1, 1, 13, 64, device=gpu))
    with pytest.raises(ReluxPanic):                 # kvcache.go:241-243
        c.Append(3, x, x)
    with pytest.raises(ReluxError):                 # pool of 3 pages exhausted
        c.Append(0, torch.zeros(1, 1, 40, 64, device=gpu), torch.zeros(1, 1, 40, 64, device=gpu),
                 seq_ids=[1])
    assert c.TotalLen(0) == 20 and c.PageTable(0, 0) == tab and c.TotalLen(0, 1) == 0
    with pytest.raises(ReluxPanic):                 # K/V shape mismatch
        c.Append(0, x, torch.zeros(1, 1, 19, 64, device=gpu))


@pytest.mark.parametrize("src_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["HSD", "SHD"])
@pytest.mark.parametrize("D", [128, 80])
def test_multi_sequence_append_gather_bit_exact(gpu, src_dtype, layout, D):
    """D 80 is stored padded to 96 dims per head: the padding never shows."""
    rng = np.random.default_rng(11 + D)
    KVH, P, S = 4, 16, 5
    c = _kv(gpu, num_layers=2, max_len=512, num_kv_heads=KVH, head_dim=D, page_tokens=P,
            max_seqs=S, pool_pages=120)
    model = PagedModel(2, P, 120, S, 32)
    logical = {(l, s): [] for l in range(2) for s in range(S)}
    for step in range(6):
        for layer in range(2):
            seqs = [int(s) for s in rng.permutation(S)[: rng.integers(1, S + 1)]]
            n = [int(v) for v in rng.integers(0, 40, size=len(seqs))]
            k_tok = [rng.normal(size=(ni, KVH, D)).astype(np.float32) * 3 for ni in n]
            v_tok = [rng.normal(size=(ni, KVH, D)).astype(np.float32) for ni in n]
            if layout == "SHD":
                kk = np.concatenate(k_tok) if sum(n) else np.zeros((0, KVH, D), np.float32)
                vv = np.concatenate(v_tok) if sum(n) else np.zeros((0, KVH, D), np.float32)
            else:
                kk = np.concatenate([t.transpose(1, 0, 2).reshape(-1) for t in k_tok])
                vv = np.concatenate([t.transpose(1, 0, 2).reshape(-1) for t in v_tok])
            kt = torch.from_numpy(np.ascontiguousarray(kk)).to(gpu).to(src_dtype)
            vt = torch.from_numpy(np.ascontiguousarray(vv)).to(gpu).to(src_dtype)
            c.Append(layer, kt, vt, seq_ids=seqs, n_tok=n, layout=layout)
            model.append(layer, seqs, n)
            for s, kt_, vt_ in zip(seqs, k_tok, v_tok):
                src_k = kt_ if src_dtype == torch.float32 else oracle.round_bf16(kt_)
                src_v = vt_ if src_dtype == torch.float32 else oracle.round_bf16(vt_)
                logical[(layer, s)].append((oracle.bf16_from_f32(src_k), oracle.bf16_from_f32(src_v)))
    for layer in range(2):
        assert c.FreeList(layer) == model.free[layer]
        for s in range(S):
            assert c.TotalLen(layer, s) == model.len[layer, s]
            assert c.PageTable(layer, s) == list(model.table[layer][s])
            ck, cv = c.View(layer, s)
            parts = logical[(layer, s)]
            if not parts or sum(p[0].shape[0] for p in parts) == 0:
                assert ck is None
                continue
            want_k = np.concatenate([p[0] for p in parts]).transpose(1, 0, 2)
            want_v = np.concatenate([p[1] for p in parts]).transpose(1, 0, 2)
            assert np.array_equal(ck.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_k)
            assert np.array_equal(cv.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_v)


@pytest.mark.parametrize("D", [8, 48, 96, 256])
def test_append_gather_other_head_dims(gpu, D):
    """head_dims that are multiples of 8 up to 256 (NewKVCacheSized takes any,
    kvcache.go:66-93; other widths below): stored as 16/32/64/96/128/256 dims, zero padded;
    View returns exactly the appended rows, across pages and two calls."""
    rng = np.random.default_rng(D)
    KVH, P = 2, 16
    c = _kv(gpu, num_layers=1, max_len=128, num_kv_heads=KVH, head_dim=D, page_tokens=P,
            max_seqs=2)
    rows = [[], []]
    for n in ([37, 5], [20, 60]):
        k = rng.normal(size=(sum(n), KVH, D)).astype(np.float32)
        v = rng.normal(size=(sum(n), KVH, D)).astype(np.float32)
        c.Append(0, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), seq_ids=[0, 1],
                 n_tok=n, layout="SHD")
        rows[0].append((k[:n[0]], v[:n[0]]))
        rows[1].append((k[n[0]:], v[n[0]:]))
    for s in range(2):
        ck, cv = c.View(0, s)
        assert tuple(ck.shape) == (1, KVH, sum(r[0].shape[0] for r in rows[s]), D)
        want_k = oracle.bf16_from_f32(np.concatenate([r[0] for r in rows[s]])).transpose(1, 0, 2)
        want_v = oracle.bf16_from_f32(np.concatenate([r[1] for r in rows[s]])).transpose(1, 0, 2)
        assert np.array_equal(ck.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_k)
        assert np.array_equal(cv.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_v)
    c.close()
    from relux_amd import _lib
    for bad in (264, 0):
        with pytest.raises(_lib.ReluxError) as e:
            _kv(gpu, num_layers=1, max_len=16, num_kv_heads=1, head_dim=bad)
        assert e.value.code in (_lib.RLX_ERR_UNSUPPORTED, _lib.RLX_ERR_INVALID)


@pytest.mark.parametrize("dC,dR", [(32, 4), (64, 8), (256, 32), (100, 6)])
def test_mla_append_gather_other_dims(gpu, dC, dR):
    """NewMLACache takes any dC and even dHR (mla_cache.go:38-59): rows are
    stored zero padded in the 512 + 64 layout and View returns exactly the
    appended latents and rope keys."""
    rng = np.random.default_rng(dC + dR)
    c = _mla(gpu, num_layers=1, max_len=256, d_c=dC, d_r=dR, page_tokens=16, max_seqs=2)
    rows = [[], []]
    for n in ([33, 4], [17, 50]):
        cc = rng.normal(size=(sum(n), dC)).astype(np.float32)
        kr = rng.normal(size=(sum(n), dR)).astype(np.float32)
        c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu), seq_ids=[0, 1], n_tok=n)
        rows[0].append((cc[:n[0]], kr[:n[0]]))
        rows[1].append((cc[n[0]:], kr[n[0]:]))
    for s in range(2):
        gc, gk = c.View(0, s)
        want_c = oracle.bf16_from_f32(np.concatenate([r[0] for r in rows[s]]))
        want_k = oracle.bf16_from_f32(np.concatenate([r[1] for r in rows[s]]))
        assert np.array_equal(gc.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_c)
        assert np.array_equal(gk.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_k)
    c.close()
    from relux_amd import _lib
    for dc_, dr_ in ((600, 64), (512, 66), (64, 3)):
        with pytest.raises(_lib.ReluxError):
            _mla(gpu, num_layers=1, max_len=16, d_c=dc_, d_r=dr_)


def test_append_conversion_edge_bits(gpu):
    """NaN / Inf / denormal / tie patterns convert exactly as BF16FromF32."""
    special = np.array([0x7FFFFFFF, 0x7F800001, 0x7FC00000, 0x7F7FFFFF, 0x00000001, 0x00008000,
                        0x00018000, 0x80000000, 0xFF800000, 0x3F800000, 0x3F808000, 0x3F818000,
                        0x807FFFFF, 0x00800000, 0x477FE000, 0xC77FF000], np.uint32)
    D = 64
    vals = np.resize(special, D).view(np.float32)
    c = _kv(gpu, num_layers=1, max_len=16, num_kv_heads=1, head_dim=D)
    k = torch.from_numpy(vals.copy()).to(gpu).reshape(1, 1, 1, D)
    c.Append(0, k, k)
    ck, cv = c.View(0)
    got = ck.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    assert np.array_equal(got, oracle.bf16_from_f32(vals))


def test_rollback_evict_compact_state(gpu):
    rng = np.random.default_rng(12)
    KVH, D, P, S, POOL, MAXP = 2, 64, 16, 4, 64, 20
    c = _kv(gpu, num_layers=2, max_len=MAXP * P, num_kv_heads=KVH, head_dim=D, page_tokens=P,
            max_seqs=S, pool_pages=POOL)
    m = PagedModel(2, P, POOL, S, MAXP)
    rows = {(l, s): [] for l in range(2) for s in range(S)}
    for step in range(40):
        seqs = list(range(S))
        n = [int(v) for v in rng.integers(1, 6, size=S)]
        for layer in range(2):
            room = [min(ni, (MAXP - int(m.first[layer, s])) * P - int(m.len[layer, s])) for s, ni in zip(seqs, n)]
            n = [max(0, r) for r in room]
        if sum(n) and sum(-(-(int(m.len[0, s]) + ni) // P) - int(m.pages[0, s]) for s, ni in zip(seqs, n)) <= len(m.free[0]):
            for layer in range(2):
                kk = rng.normal(size=(sum(n), KVH, D)).astype(np.float32)
                t = torch.from_numpy(kk).to(gpu)
                c.Append(layer, t, t, seq_ids=seqs, n_tok=n, layout="SHD")
                m.append(layer, seqs, n)
                off = 0
                for s, ni in zip(seqs, n):
                    rows[(layer, s)].extend(oracle.bf16_from_f32(kk[off:off + ni]))
                    off += ni
        for s in range(S):
            r = int(rng.integers(0, 5))
            r = min(r, int(m.len[0, s]))
            c.Rollback(s, r)
            m.rollback(-1, s, r)
            for layer in range(2):
                if r:
                    del rows[(layer, s)][len(rows[(layer, s)]) - r:]
        if step % 10 == 9:
            for s in range(S):
                e = (int(m.len[0, s]) // P) // 4
                c.Evict(s, e)
                m.evict(-1, s, e)
                for layer in range(2):
                    del rows[(layer, s)][: e * P]
            if step % 20 == 19:
                c.Compact()
                m.compact(-1)
        for layer in range(2):
            assert c.FreeList(layer) == m.free[layer]
            for s in range(S):
                assert c.SeqState(layer, s) == m.state(layer, s)
                assert c.PageTable(layer, s) == list(m.table[layer][s])
    for layer in range(2):
        for s in range(S):
            ck, cv = c.View(layer, s)
            if not rows[(layer, s)]:
                assert ck is None
                continue
            want = np.stack(rows[(layer, s)]).transpose(1, 0, 2)
            assert np.array_equal(ck.view(torch.int16).cpu().numpy().view(np.uint16)[0], want)
    c.Release(0)
    m.release(-1, 0)
    assert c.FreeList(0) == m.free[0] and c.PageTable(1, 0) == list(m.table[1][0])


def test_mla_append_gather_bit_exact(gpu):
    rng = np.random.default_rng(13)
    P, S = 64, 3
    c = _mla(gpu, num_layers=1, max_len=1024, page_tokens=P, max_seqs=S, pool_pages=40)
    m = PagedModel(1, P, 40, S, 16)
    rows = {s: [] for s in range(S)}
    for step in range(5):
        n = [int(v) for v in rng.integers(0, 130, size=S)]
        cc = rng.normal(size=(sum(n), 512)).astype(np.float32)
        kr = rng.normal(size=(sum(n), 64)).astype(np.float32)
        c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu),
                 seq_ids=list(range(S)), n_tok=n)
        m.append(0, list(range(S)), n)
        off = 0
        for s in range(S):
            rows[s].append((cc[off:off + n[s]], kr[off:off + n[s]]))
            off += n[s]
    assert c.FreeList(0) == m.free[0]
    for s in range(S):
        assert c.PageTable(0, s) == list(m.table[0][s])
        got_c, got_kr = c.View(0, s)
        want_c = oracle.bf16_from_f32(np.concatenate([r[0] for r in rows[s]]))
        want_kr = oracle.bf16_from_f32(np.concatenate([r[1] for r in rows[s]]))
        assert np.array_equal(got_c.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_c)
        assert np.array_equal(got_kr.view(torch.int16).cpu().numpy().view(np.uint16)[0], want_kr)


def test_paged_script_matches_golden(gpu):
    """Replay the committed append / rollback / evict / compact / release
    script (tests/golden/paged_script.npz, written from oracle/paged.py):
    page table, length, first entry, position offset and free stack after
    every operation, and the live bytes, all exact."""
    import os
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "paged_script.npz"))
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_fixtures", os.path.join(os.path.dirname(__file__), "golden", "make_fixtures.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    PAGED_SCRIPT, cfg = mk.PAGED_SCRIPT, mk.PAGED_CFG
    KVH, D = 2, 64
    c = _kv(gpu, num_layers=1, max_len=cfg["max_pages"] * cfg["P"], num_kv_heads=KVH, head_dim=D,
            page_tokens=cfg["P"], max_seqs=cfg["max_seqs"], pool_pages=cfg["pool_pages"])
    rng = np.random.default_rng(5)
    rows = [[] for _ in range(cfg["max_seqs"])]  # live bf16 K rows [KVH, D] per token
    for i, (op, seq, n) in enumerate(PAGED_SCRIPT):
        if op == "append":
            k = rng.standard_normal((n, KVH, D), dtype=np.float32)
            kt = torch.from_numpy(k).to(gpu)
            c.Append(0, kt, -kt, seq_ids=[seq], n_tok=[n], layout="SHD")
            rows[seq].extend(oracle.bf16_from_f32(k))
        elif op == "rollback":
            c.Rollback(seq, n)
            del rows[seq][len(rows[seq]) - n:]
        elif op == "evict":
            c.Evict(seq, n)
            del rows[seq][: n * cfg["P"]]
        elif op == "compact":
            c.Compact()
        elif op == "release":
            c.Release(seq)
            rows[seq] = []
        for s in range(cfg["max_seqs"]):
            st = c.SeqState(0, s)
            assert st["len"] == fx["lens"][i, s] and st["first"] == fx["firsts"][i, s], (i, op, s)
            assert st["pos_offset"] == fx["pos_offsets"][i, s], (i, op, s)
            assert c.PageTable(0, s) == fx["tables"][i, s].tolist(), (i, op, s)
            if st["len"]:
                kv, _ = c.View(0, s)
                got = kv[0].view(torch.int16).cpu().numpy().view(np.uint16)
                np.testing.assert_array_equal(got, np.stack(rows[s]).transpose(1, 0, 2))
        free = fx["free"][i]
        assert c.FreeList(0) == free[free >= 0].tolist(), (i, op)


# ---- host spill tier ---------------------------------------------------------

def _k_page(rows, KVH, D, P):
    """One layer's K page as stored in HBM: per kv head P x D in the
    k-step-major order (k_page_off)."""
    out = np.zeros((KVH, P * D), np.uint16)
    s_ = np.arange(P)[:, None]
    d = np.arange(D)[None, :]
    off = s_ * D + d if D <= 32 else ((s_ >> 4) * (D >> 5) + (d >> 5)) * 512 + (s_ & 15) * 32 + (d & 31)
    blk = np.stack(rows)  # [P][KVH][D]
    for h in range(KVH):
        out[h, off.ravel()] = blk[:, h, :].ravel()
    return out.ravel()


def _v_page(rows, KVH, D, P):
    """One layer's V page as stored in HBM: per kv head D x P (dim-major)."""
    return np.stack(rows).transpose(1, 2, 0).ravel()  # [KVH][D][P]


@pytest.mark.parametrize("tier", ["pinned", "file"])
def test_spill_restore_state_and_bytes(gpu, tier, tmp_path):
    """Spill / restore / evict / release against oracle/paged.py: free
    lists, table rows, sequence state, tier slots and the gathered bytes
    bit-exact at every step; with a file tier, every spilled slot of the
    file holds the page's K and V bytes as stored in HBM."""
    rng = np.random.default_rng(21)
    KVH, D, P, S, POOL, MAXP, SLOTS = 2, 64, 16, 3, 48, 16, 40
    c = _kv(gpu, num_layers=2, max_len=MAXP * P, num_kv_heads=KVH, head_dim=D, page_tokens=P,
            max_seqs=S, pool_pages=POOL)
    path = str(tmp_path / "spill.bin") if tier == "file" else None
    c.AttachSpill(SLOTS, path=path)
    slot_bytes = 2 * KVH * P * D * 2
    assert c.SpillInfo() == {"slots": SLOTS, "slot_bytes": slot_bytes, "free": SLOTS, "file": tier == "file"}
    m = PagedModel(2, P, POOL, S, MAXP, host_slots=SLOTS)
    seqs = list(range(S))

    def append(n):
        for layer in range(2):
            kk = rng.normal(size=(sum(n), KVH, D)).astype(np.float32)
            vv = rng.normal(size=(sum(n), KVH, D)).astype(np.float32)
            c.Append(layer, torch.from_numpy(kk).to(gpu), torch.from_numpy(vv).to(gpu), seq_ids=seqs,
                     n_tok=n, layout="SHD")
            kb, vb = oracle.bf16_from_f32(kk), oracle.bf16_from_f32(vv)
            pay, off = [], 0
            for ni in n:
                pay.append([(kb[off + t], vb[off + t]) for t in range(ni)])
                off += ni
            m.append(layer, seqs, n, payloads=pay)

    def check():
        for layer in range(2):
            assert c.FreeList(layer) == m.free[layer]
            for s in seqs:
                assert c.SeqState(layer, s) == m.state(layer, s)
                assert c.PageTable(layer, s) == list(m.table[layer][s])
                assert c.SpilledSlots(layer, s) == [slot for slot, _ in m.spilled[layer][s]]
                ck, cv = c.View(layer, s)
                rows = m.rows[layer][s]
                if not rows:
                    assert ck is None
                    continue
                got_k = ck.view(torch.int16).cpu().numpy().view(np.uint16)[0]
                got_v = cv.view(torch.int16).cpu().numpy().view(np.uint16)[0]
                assert np.array_equal(got_k, np.stack([r[0] for r in rows]).transpose(1, 0, 2))
                assert np.array_equal(got_v, np.stack([r[1] for r in rows]).transpose(1, 0, 2))
        assert c.SpillInfo()["free"] == len(m.host_free)
        if tier == "file":
            c.Sync()
            f = np.fromfile(path, dtype=np.uint16)
            assert f.size == SLOTS * slot_bytes // 2
            half = slot_bytes // 4
            for layer in range(2):
                for s in seqs:
                    for slot, prow in m.spilled[layer][s]:
                        got = f[slot * 2 * half:(slot + 1) * 2 * half]
                        assert np.array_equal(got[:half], _k_page([r[0] for r in prow], KVH, D, P))
                        assert np.array_equal(got[half:], _v_page([r[1] for r in prow], KVH, D, P))

    append([70, 100, 35]); check()
    c.Spill(seqs, [2, 3, 1]); m.spill(-1, seqs, [2, 3, 1]); check()
    append([20, 5, 40]); check()
    c.Restore(seqs, [1, 2, 1]); m.restore(-1, seqs, [1, 2, 1]); check()
    c.Spill([1], [2], layer=1); m.spill(1, [1], [2]); check()
    c.Compact(); m.compact(-1)
    c.Restore([0, 1], [1, 1]); m.restore(-1, [0, 1], [1, 1]); check()  # seq 0: live entries move right
    c.Restore([1], [2], layer=1); m.restore(1, [1], [2]); check()
    c.Spill(seqs, [1, 1, 1]); m.spill(-1, seqs, [1, 1, 1]); check()
    c.Evict([1], [1]); m.evict(-1, 1, 1); check()  # drops seq 1's spilled pages
    c.Release(0); m.release(-1, 0); check()
    from relux_amd import ReluxError
    with pytest.raises(ReluxError):
        c.Restore([2], [5])
    check()


def test_attention_after_restore_is_bit_exact(gpu):
    """Spilling leaves attention exactly as Evict does; restoring brings the
    pre-spill output back bit for bit (same bytes, same positions, other
    page ids)."""
    rng = np.random.default_rng(22)
    KVH, H, D, P = 2, 8, 128, 16
    c = _kv(gpu, num_layers=1, max_len=1024, num_kv_heads=KVH, head_dim=D, page_tokens=P, max_seqs=2,
            pool_pages=80)
    e = _kv(gpu, num_layers=1, max_len=1024, num_kv_heads=KVH, head_dim=D, page_tokens=P, max_seqs=2,
            pool_pages=80)
    c.AttachSpill(16)
    n = [300, 211]
    kk = torch.from_numpy(rng.normal(size=(sum(n), KVH, D)).astype(np.float32)).to(gpu)
    vv = torch.from_numpy(rng.normal(size=(sum(n), KVH, D)).astype(np.float32)).to(gpu)
    for cc in (c, e):
        cc.Append(0, kk, vv, seq_ids=[0, 1], n_tok=n, layout="SHD")
    q = torch.from_numpy(rng.normal(size=(2, H, D)).astype(np.float32)).to(gpu)
    before = c.Attend(0, q, H, seq_ids=[0, 1]).cpu()
    c.Spill([0, 1], [5, 3])
    e.Evict([0, 1], [5, 3])
    assert torch.equal(c.Attend(0, q, H, seq_ids=[0, 1]).cpu(), e.Attend(0, q, H, seq_ids=[0, 1]).cpu())
    c.Restore([0, 1], [5, 3])
    assert torch.equal(c.Attend(0, q, H, seq_ids=[0, 1]).cpu(), before)


def test_mla_spill_restore_roundtrip(gpu, tmp_path):
    """Latent pages through a file tier and back, bytes bit-exact."""
    rng = np.random.default_rng(23)
    P = 64
    c = _mla(gpu, num_layers=2, max_len=1024, page_tokens=P, max_seqs=2, pool_pages=24)
    c.AttachSpill(12, path=str(tmp_path / "mla.bin"))
    n = [200, 150]
    for layer in range(2):
        cc = torch.from_numpy(rng.normal(size=(sum(n), 512)).astype(np.float32)).to(gpu)
        kr = torch.from_numpy(rng.normal(size=(sum(n), 64)).astype(np.float32)).to(gpu)
        c.Append(layer, cc, kr, seq_ids=[0, 1], n_tok=n)
    views = [[t.clone() for t in c.View(l, s)] for l in range(2) for s in range(2)]
    c.Spill([0, 1], [3, 2])
    assert c.TotalLen(0, 0) == 200 - 3 * P and c.SeqState(1, 1)["pos_offset"] == 2 * P
    assert c.SpillInfo()["free"] == 12 - 2 * 5
    c.Restore([0, 1], [3, 2])
    after = [[t.clone() for t in c.View(l, s)] for l in range(2) for s in range(2)]
    for a, b in zip(views, after):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_reserve_keeps_calls_from_allocating(gpu):
    """rlx_cache_reserve / rlx_cache_memory: a trial handle runs an MLA
    prefill (expanded latents in the workspace), an 80-sequence GQA decode
    (its plan staged, past what the kernel arguments hold) and a head_dim-12
    decode (rows padded through the adapter buffer); a second handle
    reserves the peaks the first reported, and the same calls then grow
    neither its workspace, its staging slots nor its adapter buffer, with
    outputs bit-identical to the trial handle's."""
    rng = np.random.default_rng(404)
    H, D, lens = 16, 128, [700, 300]
    cc = rng.standard_normal((sum(lens), 512), dtype=np.float32)
    kr = rng.standard_normal((sum(lens), 64), dtype=np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    w_uk = t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D))).view(np.int16)).view(torch.bfloat16)
    w_uv = t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D))).view(np.int16)).view(torch.bfloat16)
    qn = t(rng.standard_normal((sum(lens), H, D), dtype=np.float32))
    qr = t(rng.standard_normal((sum(lens), H, 64), dtype=np.float32))
    B, KVH = 80, 8
    glens = rng.integers(20, 200, B).tolist()
    gk = t(rng.standard_normal((sum(glens), KVH, D), dtype=np.float32))
    gv = t(rng.standard_normal((sum(glens), KVH, D), dtype=np.float32))
    gq = t(rng.standard_normal((B, 32, D), dtype=np.float32))
    D12, B12 = 12, 40
    olens = rng.integers(5, 60, B12).tolist()
    ok = t(rng.standard_normal((sum(olens), 2, D12), dtype=np.float32))
    oq = t(rng.standard_normal((B12, 4, D12), dtype=np.float32))

    def run(reserve=None):
        m = _mla(gpu, num_layers=1, max_len=1024, page_tokens=64, max_seqs=2)
        g = _kv(gpu, num_layers=1, max_len=256, num_kv_heads=KVH, head_dim=D, page_tokens=16,
                max_seqs=B)
        o = _kv(gpu, num_layers=1, max_len=64, num_kv_heads=2, head_dim=D12, max_seqs=B12)
        hs = (m, g, o)
        if reserve:
            for h, r in zip(hs, reserve):
                h.Reserve(*r)
        before = [h.MemoryStats() for h in hs]
        m.Append(0, t(cc), t(kr), seq_ids=[0, 1], n_tok=lens)
        mo = m.Attend(0, qn, qr, w_uk, w_uv, H, D, seq_ids=[0, 1], n_q=lens)
        g.Append(0, gk, gv, seq_ids=list(range(B)), n_tok=glens, layout="SHD")
        go = g.Attend(0, gq, 32, seq_ids=list(range(B)))
        o.Append(0, ok, ok, seq_ids=list(range(B12)), n_tok=olens, layout="SHD")
        oo = o.Attend(0, oq, 4, seq_ids=list(range(B12)))
        after = [h.MemoryStats() for h in hs]
        out = (mo.cpu(), go.cpu(), oo.cpu())
        for h in hs:
            h.close()
        return before, after, out

    _, stats, ref = run()
    ms, gs, os_ = stats
    assert ms["workspace_peak"] > 0 and gs["workspace_peak"] > 0 and gs["staging_peak"] > 0
    assert os_["adapter_peak"] > 0 and ms["adapter_peak"] == 0 and gs["adapter_peak"] == 0
    assert ms["workspace"] >= ms["workspace_peak"]  # (staging: slots unused so far stay empty)
    want = [(x["workspace_peak"], x["staging_peak"], x["adapter_peak"]) for x in stats]
    before, after, got = run(want)
    for b, a, (wsb, stb, adb) in zip(before, after, want):
        assert b["workspace"] >= wsb and b["staging"] >= stb and b["adapter"] >= adb
        for k in ("workspace", "staging", "adapter"):
            assert a[k] == b[k], (k, b, a)
    for x, y in zip(got, ref):
        assert torch.equal(x, y)


@pytest.mark.parametrize("D", [2, 4, 12, 100])
def test_odd_head_dims_append_and_gather_bit_exact(gpu, D):
    """head_dim not a multiple of 8 (the reference tests' 2 and 4, and wider):
    appended rows cross the C boundary padded with zero dims, the gather
    narrows them back; f32 and bf16 sources, both layouts, bit-exact against
    BF16FromF32.  The no-allocation attention refuses such head dims (its
    rows would need adapter memory)."""
    from relux_amd import _lib
    rng = np.random.default_rng(500 + D)
    KVH, lens = 2, [5, 40, 17]
    c = _kv(gpu, num_layers=1, max_len=64, num_kv_heads=KVH, head_dim=D, max_seqs=3)
    want = [[] for _ in lens]
    for step, (dt, layout) in enumerate([(torch.float32, "SHD"), (torch.bfloat16, "HSD")]):
        n = [L // 2 if step == 0 else L - L // 2 for L in lens]
        rows = [rng.standard_normal((KVH, m, D), dtype=np.float32) for m in n]  # logical [KVH][n][D]
        if layout == "SHD":
            src = np.concatenate([r.transpose(1, 0, 2) for r in rows])
        else:
            src = np.concatenate([r.reshape(-1, D) for r in rows])
        t = torch.from_numpy(np.ascontiguousarray(src)).to(gpu).to(dt)
        c.Append(0, t, t * 2, seq_ids=[0, 1, 2], n_tok=n, layout=layout)
        for i, r in enumerate(rows):
            want[i].append(oracle.round_bf16(torch.from_numpy(r).to(dt).float().numpy()))
    for i in range(len(lens)):
        k, v = c.View(0, i)
        w = np.concatenate(want[i], axis=1)[None]
        assert np.array_equal(k.float().cpu().numpy(), w), (D, i)
        assert np.array_equal(v.float().cpu().numpy(), oracle.round_bf16(w * 2)), (D, i)
    q = torch.zeros((3, 4, D), device=gpu)
    out = torch.empty_like(q)
    if D % 8:
        with pytest.raises(_lib.ReluxError) as e:
            c.AttendNoAlloc(0, q, 4, out, seq_ids=[0, 1, 2])
        assert e.value.code == _lib.RLX_ERR_UNSUPPORTED
