"""GPU parity of decode / verify attention over the paged cache.

Two references per case:
  * the oracle's restatement of the reference loops (fastexp32 softmax,
    mha.go:291-348 / mla.go:316-377): max-abs 2e-2, mean-abs 2e-3 at the
    context lengths of the benchmark configs;
  * an exact-softmax f64 attention (numpy, independent): max-abs 1e-2,
    mean-abs 1e-3, which bounds the kernel's own bf16 operand rounding.
At the full benchmark shapes a torch f32 attention over the gathered cache
is the reference (same exact-softmax tolerance).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import tiny_decoder as td

pytestmark = pytest.mark.gpu

TOL_ORACLE = (2e-2, 2e-3)
TOL_EXACT = (1e-2, 1e-3)
TOL_MLA_EXACT = (5e-3, 5e-4)


def _check(got, want, tol, what):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    assert err.max() <= tol[0] and err.mean() <= tol[1], (
        f"{what}: max-abs {err.max():.3e} mean-abs {err.mean():.3e} (tol {tol})")


def _limits(mask, nq, T):
    if mask == "causal":
        return [T - nq + i for i in range(nq)]
    if mask == "ref":
        return [i if nq == T else T - 1 for i in range(nq)]
    return [T - 1] * nq


def _fill_gqa(c, rng, gpu, lens, KVH, D, chunks=2):
    """Append lens[i] tokens to sequence i in `chunks` multi-sequence calls;
    returns the logical bf16 K/V per sequence as floats [KVH, T, D]."""
    S = len(lens)
    ks = [[] for _ in range(S)]
    vs = [[] for _ in range(S)]
    done = [0] * S
    for ci in range(chunks):
        n = [(L * (ci + 1)) // chunks - done[i] for i, L in enumerate(lens)]
        k = rng.standard_normal((sum(n), KVH, D), dtype=np.float32)
        v = rng.standard_normal((sum(n), KVH, D), dtype=np.float32)
        c.Append(0, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu),
                 seq_ids=list(range(S)), n_tok=n, layout="SHD")
        off = 0
        for i in range(S):
            ks[i].append(k[off:off + n[i]])
            vs[i].append(v[off:off + n[i]])
            off += n[i]
            done[i] += n[i]
    K = [oracle.round_bf16(np.concatenate(x)).transpose(1, 0, 2) for x in ks]
    V = [oracle.round_bf16(np.concatenate(x)).transpose(1, 0, 2) for x in vs]
    return K, V


@pytest.mark.parametrize("H,KVH,D,lens,nq,mask", [
    (32, 8, 128, [1, 2, 15, 16, 17, 64, 65, 300], 1, "causal"),     # ragged, page edges
    (32, 8, 128, [600, 1, 257], 4, "causal"),                        # verify, 4 drafts x 4 heads
    (64, 8, 128, [700, 33, 96], 4, "causal"),                        # 32 query rows per kv head
    (8, 8, 64, [5, 129, 1000], 2, "none"),
    (16, 4, 64, [7, 7, 40], 7, "ref"),                               # reference mask rule
    (16, 4, 128, [3, 12], 3, "ref"),
    (4, 2, 16, [8, 23, 300], 1, "causal"),                           # config-1 head_dim 16
    (4, 2, 16, [8, 9], 8, "ref"),
    (8, 2, 32, [17, 500], 4, "causal"),                              # head_dim 32
    (16, 4, 80, [300, 17, 1], 1, "causal"),                          # 80: stored as 96
    (32, 8, 96, [600, 33], 4, "causal"),                             # 96
    (16, 2, 256, [400, 65], 2, "causal"),                            # 256: 16-row tiles
    (4, 2, 8, [8, 23, 300], 1, "causal"),                            # 8: stored as 16
    (8, 2, 48, [260, 9], 3, "ref"),                                  # 48: stored as 64
    # head dims that are not multiples of 8 (rows padded at the C boundary):
    # the reference tests' own shapes, then wider ones on every path
    (2, 1, 2, [3, 40, 300], 1, "causal"),                            # mha_test.go:86 (dModel 4, 2 heads)
    (4, 2, 2, [9, 300], 4, "causal"),                                # NewMHA(8, 4, 2): head_dim 2
    (1, 1, 4, [5, 260], 1, "causal"),                                # NewMHA(4, 1, 1): head_dim 4
    (4, 1, 20, [70, 300], 40, "causal"),                             # 160 rows per kv head: query chunks
    (8, 2, 100, [300, 77], 50, "causal"),                            # 100 (stored 128): FA2 prefill
    (16, 4, 250, [290], 2, "causal"),                                # 250 (stored 256)
])
def test_gqa_attend_matches_oracle(gpu, H, KVH, D, lens, nq, mask):
    from relux_amd import KVCache
    rng = np.random.default_rng(H * 1000 + KVH * 100 + D + nq * 7 + len(lens))
    P = 16
    c = KVCache(num_layers=1, max_len=max(lens) + 32, num_kv_heads=KVH, head_dim=D,
                page_tokens=P, max_seqs=len(lens), device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    nqs = [min(nq, L) for L in lens]
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(len(lens))), n_q=nqs,
                   mask=mask).cpu().numpy()
    off = 0
    for i, L in enumerate(lens):
        qs = q[off:off + nqs[i]].transpose(1, 0, 2)            # [H, nq, D]
        got = out[off:off + nqs[i]].transpose(1, 0, 2)
        g = H // KVH
        exact = oracle.exact_attention_f64(qs, np.repeat(K[i], g, 0), np.repeat(V[i], g, 0),
                                           _limits(mask, nqs[i], L))
        _check(got, exact, TOL_EXACT, f"seq {i} len {L} vs exact")
        if L >= 256:
            ref = oracle.gqa_attend(qs, K[i], V[i], mask)
            _check(got, ref, TOL_ORACLE, f"seq {i} len {L} vs oracle")
        off += nqs[i]


def test_gqa_layouts_dtypes_and_bf16_output(gpu):
    from relux_amd import KVCache
    rng = np.random.default_rng(21)
    H, KVH, D, lens = 16, 4, 128, [100, 333]
    c = KVCache(num_layers=1, max_len=400, num_kv_heads=KVH, head_dim=D, max_seqs=2,
                device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    q = torch.from_numpy(rng.standard_normal((2, H, D), dtype=np.float32)).to(gpu)
    base = c.Attend(0, q, H, seq_ids=[0, 1]).cpu()
    # HSD layout = per sequence [H][nq][D] (identical when nq == 1)
    hsd = c.Attend(0, q, H, seq_ids=[0, 1], layout="HSD").cpu()
    assert torch.equal(base, hsd)
    b16 = c.Attend(0, q.bfloat16(), H, seq_ids=[0, 1], out_dtype=torch.bfloat16).float().cpu()
    _check(b16.numpy(), base.numpy(), (1.5e-2, 1.5e-3), "bf16 q/out")
    # reordered sequence list gives the same per-sequence rows
    rev = c.Attend(0, torch.flip(q, [0]).contiguous(), H, seq_ids=[1, 0]).cpu()
    assert torch.equal(rev[0], base[1]) and torch.equal(rev[1], base[0])


def test_gqa_attention_after_evict_equals_dense_survivors(gpu):
    """Attention over an evicted+compacted cache == exact attention over the
    surviving tokens (row A17 of the parity contract)."""
    from relux_amd import KVCache
    rng = np.random.default_rng(22)
    H, KVH, D, P = 32, 8, 128, 16
    lens = [500, 260]
    c = KVCache(num_layers=1, max_len=1024, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=2, device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    ev = [(L // P) // 4 for L in lens]
    for s, e in enumerate(ev):
        c.Evict(s, e)
    q = torch.from_numpy(rng.standard_normal((2, H, D), dtype=np.float32)).to(gpu)
    before = c.Attend(0, q, H, seq_ids=[0, 1]).cpu().numpy()
    c.Compact()
    after = c.Attend(0, q, H, seq_ids=[0, 1]).cpu().numpy()
    assert np.array_equal(before, after)
    for s in range(2):
        Ks, Vs = K[s][:, ev[s] * P:], V[s][:, ev[s] * P:]
        T = Ks.shape[1]
        exact = oracle.exact_attention_f64(q[s:s + 1].cpu().numpy().transpose(1, 0, 2),
                                           np.repeat(Ks, H // KVH, 0), np.repeat(Vs, H // KVH, 0),
                                           [T - 1])
        _check(after[s:s + 1].transpose(1, 0, 2), exact, TOL_EXACT, f"seq {s} survivors")


@pytest.mark.parametrize("D", [128, 64])
def test_gqa_prefill_after_evict_equals_survivors(gpu, D):
    """A chunked GQA prefill (the FA2 kernel, pages through the table from
    the first live entry) over sequences whose oldest pages were evicted ==
    exact attention over the surviving tokens, before and after compaction."""
    from relux_amd import KVCache
    rng = np.random.default_rng(23 + D)
    H, KVH, P = 16, 4, 16
    lens, ev, nqs = [520, 300], [5, 3], [96, 64]
    c = KVCache(num_layers=1, max_len=1024, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=2, device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    for s, e in enumerate(ev):
        c.Evict(s, e)
    q = torch.from_numpy(rng.standard_normal((sum(nqs), H, D), dtype=np.float32)).to(gpu)
    before = c.Attend(0, q, H, seq_ids=[0, 1], n_q=nqs).cpu().numpy()
    c.Compact()
    after = c.Attend(0, q, H, seq_ids=[0, 1], n_q=nqs).cpu().numpy()
    assert np.array_equal(before, after)
    off = 0
    for s in range(2):
        Ks, Vs = K[s][:, ev[s] * P:], V[s][:, ev[s] * P:]
        T = Ks.shape[1]
        exact = oracle.exact_attention_f64(q[off:off + nqs[s]].cpu().numpy().transpose(1, 0, 2),
                                           np.repeat(Ks, H // KVH, 0), np.repeat(Vs, H // KVH, 0),
                                           _limits("causal", nqs[s], T))
        _check(after[off:off + nqs[s]].transpose(1, 0, 2), exact, TOL_EXACT, f"seq {s} survivors")
        off += nqs[s]


def _torch_gqa_ref(k_list, v_list, q, H, KVH):
    """f32 exact attention in torch over dense K/V (full-size property check)."""
    outs = []
    g = H // KVH
    for i, (k, v) in enumerate(zip(k_list, v_list)):
        kf = k[0].float().repeat_interleave(g, 0)          # [H, T, D]
        vf = v[0].float().repeat_interleave(g, 0)
        s = torch.einsum("hd,htd->ht", q[i].float(), kf) / math.sqrt(kf.shape[-1])
        w = torch.softmax(s, dim=-1)
        outs.append(torch.einsum("ht,htd->hd", w, vf))
    return torch.stack(outs)


@pytest.mark.parametrize("n_rows,H,KVH,nq", [
    (40, 32, 8, 1),   # rows and ranges both in the kernel arguments
    (60, 32, 8, 1),   # rows in the arguments, ranges recomputed per work-group
    (60, 64, 8, 4),   # the same with 32 query rows per kv head
    (50, 8, 2, 2),    # 128 ranges: many cuts, rows shorter than a range
    (80, 32, 8, 1),   # rows and ranges staged to the device
])
def test_gqa_balanced_ranges_many_rows(gpu, n_rows, H, KVH, nq):
    """The decode work split cuts the batch's tokens into equal ranges that
    straddle rows: ragged lengths (a few tokens to ~1.5k, some next to the
    64-token pad boundaries where cuts snap), every plan route."""
    from relux_amd import KVCache
    rng = np.random.default_rng(n_rows * 10 + KVH + nq)
    D, P = 128, 16
    lens = rng.integers(1, 1500, size=n_rows)
    lens[::7] = rng.integers(1, 30, size=len(lens[::7]))
    lens[3::11] = 64 * rng.integers(1, 20, size=len(lens[3::11])) + rng.integers(-3, 4, size=len(lens[3::11]))
    lens = [int(max(L, nq)) for L in lens]
    c = KVCache(num_layers=1, max_len=max(lens) + 32, num_kv_heads=KVH, head_dim=D,
                page_tokens=P, max_seqs=n_rows, device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    nqs = [nq] * n_rows
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(n_rows)), n_q=nqs,
                   mask="causal").cpu().numpy()
    g = H // KVH
    off = 0
    for i, L in enumerate(lens):
        qs = q[off:off + nq].transpose(1, 0, 2)
        got = out[off:off + nq].transpose(1, 0, 2)
        exact = oracle.exact_attention_f64(qs, np.repeat(K[i], g, 0), np.repeat(V[i], g, 0),
                                           _limits("causal", nq, L))
        _check(got, exact, TOL_EXACT, f"row {i} len {L} vs exact")
        off += nq


def test_gqa_long_call_ranges(gpu):
    """A decode call of at least 4096 tokens per range (16 x ~6 200 tokens,
    8 kv heads: 99k tokens) takes three quarters of the ranges, rounded to
    the XCDs (24 per kv head on 256 CUs), as the 8k and 32k headlines do;
    every row against exact attention."""
    from relux_amd import KVCache
    rng = np.random.default_rng(61)
    H, KVH, D, P, B = 32, 8, 128, 16, 16
    lens = [int(L) for L in rng.integers(6100, 6300, size=B)]
    c = KVCache(num_layers=1, max_len=max(lens) + 32, num_kv_heads=KVH, head_dim=D,
                page_tokens=P, max_seqs=B, device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D, chunks=3)
    q = rng.standard_normal((B, H, D), dtype=np.float32)
    out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(B))).cpu().numpy()
    g = H // KVH
    for i, L in enumerate(lens):
        exact = oracle.exact_attention_f64(q[i:i + 1].transpose(1, 0, 2), np.repeat(K[i], g, 0),
                                           np.repeat(V[i], g, 0), _limits("causal", 1, L))
        _check(out[i:i + 1].transpose(1, 0, 2), exact, TOL_EXACT, f"row {i} len {L} vs exact")


def test_gqa_config2_full_shape(gpu):
    """B 16, H 32, KVH 8, D 128, T ~ U[512, 4096], 16-token
    pages randomly permuted in a shared pool, one append then one query."""
    from relux_amd import KVCache
    rng = np.random.default_rng(2)
    B, H, KVH, D, P = 16, 32, 8, 128, 16
    lens = rng.integers(512, 4097, size=B).tolist()
    c = KVCache(num_layers=1, max_len=4096 + 16, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=B, pool_pages=sum(-(-(L + 1) // P) for L in lens) + 64, device=gpu.index)
    # permute the pool: interleave sequences page by page in random order
    left = list(lens)
    while any(left):
        order = [i for i in rng.permutation(B) if left[i] > 0]
        n = [min(P, left[i]) for i in order]
        k = torch.randn(sum(n), KVH, D, device=gpu)
        c.Append(0, k, torch.randn_like(k), seq_ids=order, n_tok=n, layout="SHD")
        for i, ni in zip(order, n):
            left[i] -= ni
    k1 = torch.randn(B, KVH, D, device=gpu)
    c.Append(0, k1, torch.randn_like(k1), seq_ids=list(range(B)), n_tok=[1] * B, layout="SHD")
    q = torch.randn(B, H, D, device=gpu)
    out = c.Attend(0, q, H, seq_ids=list(range(B)))
    views = [c.View(0, i) for i in range(B)]
    ref = _torch_gqa_ref([v[0] for v in views], [v[1] for v in views], q, H, KVH)
    _check(out.cpu().numpy(), ref.cpu().numpy(), TOL_EXACT, "config 2 vs torch f32")
    for i in (0, 7):  # the reference loops themselves on two sequences
        kk = views[i][0][0].float().cpu().numpy()
        vv = views[i][1][0].float().cpu().numpy()
        ref_o = oracle.gqa_attend(q[i:i + 1].cpu().numpy().transpose(1, 0, 2), kk, vv, "causal")
        _check(out[i:i + 1].cpu().numpy().transpose(1, 0, 2), ref_o, TOL_ORACLE, f"seq {i} vs oracle")


# ---- MLA -------------------------------------------------------------------

def _mla_exact(qc, qr, c, kr, w_uk, w_uv, limits):
    """Absorbed MLA in f64 with exact softmax; qc [H,nq,D], qr [H,nq,dR]."""
    H, nq, D = qc.shape
    dC = c.shape[1]
    Wk = oracle.f32_from_bf16(w_uk).astype(np.float64).reshape(dC, H, D)
    Wv = oracle.f32_from_bf16(w_uv).astype(np.float64).reshape(dC, H, D)
    qlat = np.einsum("chd,hid->hic", Wk, qc.astype(np.float64))
    s = (np.einsum("hic,tc->hit", qlat, c.astype(np.float64)) +
         np.einsum("hir,tr->hit", qr.astype(np.float64), kr.astype(np.float64))) / math.sqrt(D + qr.shape[2])
    T = c.shape[0]
    s = np.where(np.arange(T)[None, None, :] <= np.asarray(limits)[None, :, None], s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    return np.einsum("hic,chd->hid", np.einsum("hit,tc->hic", w, c.astype(np.float64)), Wv)


@pytest.mark.parametrize("H,lens,nq,mask", [
    (16, [1, 15, 64, 65, 200, 300], 1, "causal"),
    # many ragged rows, each split into its own near-equal splits (rows in
    # the kernel arguments, work items found by search) ...
    (16, [int(x) for x in np.random.default_rng(5).integers(1, 400, 40)], 1, "causal"),
    # ... and more rows than the arguments hold (rows and work list staged)
    (8, [int(x) for x in np.random.default_rng(6).integers(2, 300, 70)], 2, "causal"),
    (16, [260, 7], 2, "causal"),
    (8, [90, 3], 3, "ref"),
    (16, [128], 1, "none"),
])
def test_mla_attend_matches_oracle(gpu, H, lens, nq, mask):
    _mla_attend_case(gpu, H, lens, nq, mask, 64)


@pytest.mark.parametrize("P,nq", [(16, 1), (48, 1), (16, 150), (48, 150)])
def test_mla_pages_16_and_48(gpu, P, nq):
    """The latent cache on 16-token pages (every 16-token tile of the decode
    ring on its own page) and on 48-token pages (not a power of two, the
    prefill's division route), decode and FA2 prefill, against exact
    attention."""
    _mla_attend_case(gpu, 16, [300, 170, 40], nq, "causal", P)


def _mla_attend_case(gpu, H, lens, nq, mask, P):
    from relux_amd import MLACache
    rng = np.random.default_rng(31 + H + nq + P)
    D = 128
    c = MLACache(num_layers=1, max_len=max(lens) + P, page_tokens=P, max_seqs=len(lens),
                 device=gpu.index)
    cc = rng.standard_normal((sum(lens), 512), dtype=np.float32)
    kr = rng.standard_normal((sum(lens), 64), dtype=np.float32)
    c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu),
             seq_ids=list(range(len(lens))), n_tok=lens)
    w_uk = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    w_uv = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    nqs = [min(nq, L) for L in lens]
    qn = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    qr = rng.standard_normal((sum(nqs), H, 64), dtype=np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    wuk = t(w_uk.view(np.int16)).view(torch.bfloat16)
    wuv = t(w_uv.view(np.int16)).view(torch.bfloat16)
    out = c.Attend(0, t(qn), t(qr), wuk, wuv, H, D, seq_ids=list(range(len(lens))), n_q=nqs,
                   mask=mask).cpu().numpy()
    off = 0
    toff = 0
    for i, L in enumerate(lens):
        cs = oracle.round_bf16(cc[toff:toff + L])
        ks = oracle.round_bf16(kr[toff:toff + L])
        qci = qn[off:off + nqs[i]].transpose(1, 0, 2)
        qri = qr[off:off + nqs[i]].transpose(1, 0, 2)
        got = out[off:off + nqs[i]].transpose(1, 0, 2)
        exact = _mla_exact(qci, qri, cs, ks, w_uk, w_uv, _limits(mask, nqs[i], L))
        # Outputs are ~0.05-0.5 (W_UV N(0,0.02) over 512 channels); short
        # contexts see the bf16 rounding of P and q_lat at ~2e-3 absolute.
        _check(got, exact, TOL_MLA_EXACT, f"seq {i} len {L} vs exact")
        if L >= 200:
            ref = oracle.mla_attend(qci, qri, cs, ks, w_uk, w_uv, mask)
            _check(got, ref, TOL_ORACLE, f"seq {i} len {L} vs oracle")
        off += nqs[i]
        toff += L


def test_mla_decode_many_splits(gpu):
    """Decode rows cut into more than 16 context splits (the merge reloads
    the split partials in batches of 16) and more than 64 (merge weights
    past split 64 in a second pass): a 12 000-token row alone takes 94
    splits, 2 100 tokens 17.  f32 outputs against exact attention; bf16
    outputs equal the f32 outputs rounded to nearest even, bit for bit."""
    from relux_amd import MLACache
    rng = np.random.default_rng(97)
    H, D, P = 16, 128, 64
    for lens in ([12000], [12000, 2100, 300, 40]):
        c = MLACache(num_layers=1, max_len=max(lens) + P, page_tokens=P, max_seqs=len(lens),
                     device=gpu.index)
        cc = rng.standard_normal((sum(lens), 512), dtype=np.float32)
        kr = rng.standard_normal((sum(lens), 64), dtype=np.float32)
        c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu),
                 seq_ids=list(range(len(lens))), n_tok=lens)
        w_uk = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
        w_uv = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
        qn = rng.standard_normal((len(lens), H, D), dtype=np.float32)
        qr = rng.standard_normal((len(lens), H, 64), dtype=np.float32)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
        args = (t(qn), t(qr), t(w_uk.view(np.int16)).view(torch.bfloat16),
                t(w_uv.view(np.int16)).view(torch.bfloat16), H, D)
        ids = list(range(len(lens)))
        out = c.Attend(0, *args, seq_ids=ids).cpu().numpy()
        out16 = c.Attend(0, *args, seq_ids=ids, out_dtype=torch.bfloat16).cpu()
        assert np.array_equal(out16.view(torch.int16).numpy().view(np.uint16),
                              oracle.bf16_from_f32(out)), lens
        toff = 0
        for i, L in enumerate(lens):
            cs = oracle.round_bf16(cc[toff:toff + L])
            ks = oracle.round_bf16(kr[toff:toff + L])
            exact = _mla_exact(qn[i:i + 1].transpose(1, 0, 2), qr[i:i + 1].transpose(1, 0, 2), cs, ks,
                               w_uk, w_uv, [L - 1])
            _check(out[i:i + 1].transpose(1, 0, 2), exact, TOL_MLA_EXACT, f"len {L} of {lens} vs exact")
            toff += L
        c.close()


@pytest.mark.parametrize("H,D,dC,dR,lens,nq,mask", [
    (4, 8, 32, 4, [8, 23, 300], 1, "causal"),      # TestTransformer_MLA's dims (transformer_test.go:1012-1027)
    (4, 16, 64, 8, [9, 100, 260], 4, "causal"),    # config-1-sized layer, 4-query verify
    (8, 64, 256, 32, [300, 17], 2, "causal"),
    (4, 32, 128, 16, [290, 64], 40, "causal"),     # 160 query rows: 5 head groups
    (4, 16, 64, 8, [70, 40], 40, "none"),          # unmasked, 160 rows
    (2, 8, 32, 4, [50], 50, "ref"),                # reference rule with n_q == len: causal
    (16, 128, 512, 64, [300, 65], 1, "causal"),    # default DeepSeek dims, generic absorb / out
    (8, 128, 256, 32, [2100, 70], 1, "causal"),    # head_dim 128 with d_c < 512: latent channels past d_c
    (16, 96, 384, 48, [260], 2, "causal"),
    # head dims that are not multiples of 8 (q_nope, W_UK, W_UV and the
    # output padded at the boundary): mla_test.go's dims (dModel 8, 2 heads:
    # headDim 4, dC 16, dHR 2), decode and FA2 prefill, and head_dim 20
    (2, 4, 16, 2, [9, 70], 1, "causal"),
    (2, 4, 16, 2, [60, 30], 40, "causal"),
    (3, 20, 80, 10, [300, 20], 2, "causal"),
    (8, 128, 512, 64, [280, 40], 30, "causal"),    # head_dim 128, 240 rows (8 head groups / FA2)
    # the reference's default dims (FA2: K_c / V^T expanded with zero rows to
    # a 128-dim pitch, W_UK / W_UV columns past d_c zero): 64 heads at
    # headDim 32 (dC 128, dR 16), and 40 heads decoding one query each
    (64, 32, 128, 16, [300, 90], 3, "causal"),
    (40, 64, 256, 32, [280, 50], 1, "causal"),
    # head_dim 160 (FA2: 256-dim pitch, two launches of 128 value dims)
    (48, 160, 512, 64, [270], 2, "causal"),
    # DeepSeek-V3 decode and verify shapes: 128 heads (4 head groups), and
    # 4-query verify at 64 heads (8 groups)
    (128, 128, 512, 64, [700, 33, 260], 1, "causal"),
    (64, 128, 512, 64, [500, 90], 4, "causal"),
])
@pytest.mark.parametrize("path", ["default", "fa2"])
def test_mla_other_dims_match_oracle(gpu, monkeypatch, path, H, D, dC, dR, lens, nq, mask):
    """MLA at the reference's default dims (dC = 4 headDim, dHR = headDim/2,
    transformer.go:223-233) and others: latent rows stored zero padded,
    absorb and W_UV projection at head_dims that are multiples of 8 (other
    widths padded to one at the C boundary), and calls of more than 32
    query rows per sequence.  Each case runs on the
    default path (up to 1024 query rows per sequence: the absorbed decode
    kernel in head groups of 32 rows) and with the FA2 expansion forced past
    32 rows (RLX_MLA_FA2_ROWS)."""
    from relux_amd import MLACache
    if path == "fa2":
        monkeypatch.setenv("RLX_MLA_FA2_ROWS", "32")
    rng = np.random.default_rng(61 + H + D + nq)
    P = 64 if D >= 64 else 16
    c = MLACache(num_layers=1, max_len=max(lens) + P, d_c=dC, d_r=dR, page_tokens=P,
                 max_seqs=len(lens), device=gpu.index)
    cc = rng.standard_normal((sum(lens), dC), dtype=np.float32)
    kr = rng.standard_normal((sum(lens), dR), dtype=np.float32)
    c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu),
             seq_ids=list(range(len(lens))), n_tok=lens)
    # weights ~ N(0, 0.5 / sqrt(dC)): scores and outputs of like size at every dC
    w_uk = oracle.bf16_from_f32(rng.normal(0, 0.5 / math.sqrt(dC), size=(dC, H * D)))
    w_uv = oracle.bf16_from_f32(rng.normal(0, 0.5 / math.sqrt(dC), size=(dC, H * D)))
    nqs = [min(nq, L) for L in lens]
    qn = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    qr = rng.standard_normal((sum(nqs), H, dR), dtype=np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    out = c.Attend(0, t(qn), t(qr), t(w_uk.view(np.int16)).view(torch.bfloat16),
                   t(w_uv.view(np.int16)).view(torch.bfloat16), H, D,
                   seq_ids=list(range(len(lens))), n_q=nqs, mask=mask).cpu().numpy()
    off = toff = 0
    for i, L in enumerate(lens):
        cs = oracle.round_bf16(cc[toff:toff + L])
        ks = oracle.round_bf16(kr[toff:toff + L])
        qci = qn[off:off + nqs[i]].transpose(1, 0, 2)
        qri = qr[off:off + nqs[i]].transpose(1, 0, 2)
        got = out[off:off + nqs[i]].transpose(1, 0, 2)
        exact = _mla_exact(qci, qri, cs, ks, w_uk, w_uv, _limits(mask, nqs[i], L))
        # bf16 q_lat and weights P (and, through FA2, bf16 K_c / V) against
        # exact f64 on outputs of size ~0.1-0.5
        tol = (2e-2, 2e-3) if nqs[i] * H > 32 else TOL_EXACT
        _check(got, exact, tol, f"seq {i} len {L} nq {nqs[i]} vs exact")
        # The oracle's softmax is the reference's fastexp32 (mha.go:823-833,
        # ~3% per weight): over a few keys its outputs sit ~3e-3 from exact,
        # so it is compared where many keys average that out.
        if L >= 200:
            ref = oracle.mla_attend(qci, qri, cs, ks, w_uk, w_uv, mask)
            _check(got, ref, TOL_ORACLE, f"seq {i} len {L} nq {nqs[i]} vs oracle")
        off += nqs[i]
        toff += L
    c.close()


# ---- chunked prefill (more than 32 query rows per kv head / sequence) -------

@pytest.mark.parametrize("H,KVH,D,lens,nqs,mask", [
    (16, 4, 128, [300, 65, 40], [100, 65, 33], "causal"),   # chunk on a cache, full prefill
    (16, 4, 128, [900, 600], [300, 64], "causal"),          # long rows for the oracle check
    (32, 4, 64, [257, 129], [200, 129], "causal"),          # G = 8, D = 64
    (8, 8, 128, [90, 70], [90, 30], "ref"),                 # reference mask rule both ways
    (16, 16, 128, [150], [150], "none"),
    # group sizes that do not divide 256: FA2 tiles of floor(256 / G) tokens
    (12, 4, 64, [290, 50], [60, 50], "causal"),            # G = 3: 85 tokens, 255 rows
    (6, 2, 128, [260], [260], "none"),
    (20, 4, 128, [300, 70], [120, 70], "causal"),          # G = 5: 51 tokens
    # shapes the FA2 kernel does not take: query tiles through the decode kernel
    (4, 2, 16, [300, 40], [70, 40], "causal"),             # head_dim 16
    (8, 2, 32, [280, 100], [120, 100], "ref"),             # head_dim 32
    (16, 4, 80, [300, 40], [70, 40], "causal"),            # padded head_dim: query tiles
    (8, 8, 96, [270], [40], "ref"),
    # FA2 at head_dim 256: two launches of 128 value dims each
    (8, 2, 256, [290, 50], [60, 50], "causal"),
    (32, 8, 256, [400, 100], [150, 100], "causal"),
    (16, 2, 256, [300], [300], "none"),
    # FA2 at a head_dim below the stored one (120 in 128-dim pages)
    (16, 4, 120, [300, 70], [100, 70], "causal"),
])
def test_gqa_prefill_matches_oracle(gpu, H, KVH, D, lens, nqs, mask):
    from relux_amd import KVCache
    rng = np.random.default_rng(41 + H + D)
    c = KVCache(num_layers=1, max_len=max(lens) + 32, num_kv_heads=KVH, head_dim=D,
                max_seqs=len(lens), device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D, chunks=3)
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(len(lens))), n_q=nqs,
                   mask=mask).cpu().numpy()
    off = 0
    g = H // KVH
    for i, L in enumerate(lens):
        qs = q[off:off + nqs[i]].transpose(1, 0, 2)
        got = out[off:off + nqs[i]].transpose(1, 0, 2)
        exact = oracle.exact_attention_f64(qs, np.repeat(K[i], g, 0), np.repeat(V[i], g, 0),
                                           _limits(mask, nqs[i], L))
        _check(got, exact, TOL_EXACT, f"seq {i} len {L} nq {nqs[i]} vs exact")
        ref = oracle.gqa_attend(qs, K[i], V[i], mask)
        # fastexp32 weights are off by up to ~3.5% each; the reference's own
        # error vs exact softmax averages below 2e-2 only for rows that attend
        # >= 256 keys, so those rows are judged against the oracle (all rows
        # are judged against exact softmax above).
        lim = np.array(_limits(mask, nqs[i], L))
        rows = np.nonzero(lim >= 255)[0]
        if len(rows):
            _check(got[:, rows], ref[:, rows], TOL_ORACLE, f"seq {i} vs oracle (rows >= 256 keys)")
        off += nqs[i]


@pytest.mark.parametrize("P", [48, 80])
def test_gqa_pages_not_power_of_two(gpu, P):
    """Pages of 48 / 80 tokens (multiples of 16, not powers of two): the
    prefill takes its division route for page and slot, the decode and the
    appends their generic ones; a 16-token half-block never straddles two
    pages.  Chunked prefill, full prefill and single-query decode against
    exact attention."""
    from relux_amd import KVCache
    rng = np.random.default_rng(P)
    H, KVH, D = 16, 4, 128
    lens, nqs = [301, 97, 160], [120, 97, 1]
    c = KVCache(num_layers=1, max_len=max(lens) + P, num_kv_heads=KVH, head_dim=D,
                page_tokens=P, max_seqs=len(lens), device=gpu.index)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D, chunks=3)
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(len(lens))), n_q=nqs,
                   mask="causal").cpu().numpy()
    g = H // KVH
    off = 0
    for i, L in enumerate(lens):
        qs = q[off:off + nqs[i]].transpose(1, 0, 2)
        exact = oracle.exact_attention_f64(qs, np.repeat(K[i], g, 0), np.repeat(V[i], g, 0),
                                           _limits("causal", nqs[i], L))
        _check(out[off:off + nqs[i]].transpose(1, 0, 2), exact, TOL_EXACT, f"P {P} seq {i} len {L}")
        off += nqs[i]
    # decode of every sequence in one call
    q1 = rng.standard_normal((len(lens), H, D), dtype=np.float32)
    o1 = c.Attend(0, torch.from_numpy(q1).to(gpu), H, seq_ids=list(range(len(lens)))).cpu().numpy()
    for i, L in enumerate(lens):
        exact = oracle.exact_attention_f64(q1[i:i + 1].transpose(1, 0, 2), np.repeat(K[i], g, 0),
                                           np.repeat(V[i], g, 0), _limits("causal", 1, L))
        _check(o1[i:i + 1].transpose(1, 0, 2), exact, TOL_EXACT, f"P {P} decode seq {i}")


def test_gqa_query_tiles_layouts(gpu):
    """Query-tiled attention (head_dim 16, 40 queries x 2 heads per kv head)
    gives the same rows in both q/out layouts."""
    from relux_amd import KVCache
    rng = np.random.default_rng(47)
    H, KVH, D, lens, nqs = 4, 2, 16, [60, 45], [40, 45]
    c = KVCache(num_layers=1, max_len=64, num_kv_heads=KVH, head_dim=D, max_seqs=2,
                device=gpu.index)
    _fill_gqa(c, rng, gpu, lens, KVH, D)
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    shd = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=[0, 1], n_q=nqs).cpu().numpy()
    qh = np.concatenate([q[:40].transpose(1, 0, 2).reshape(-1), q[40:].transpose(1, 0, 2).reshape(-1)])
    hsd = c.Attend(0, torch.from_numpy(qh).to(gpu), H, seq_ids=[0, 1], n_q=nqs,
                   layout="HSD").cpu().numpy()
    back = np.concatenate([hsd[:40 * H * D].reshape(H, 40, D).transpose(1, 0, 2),
                           hsd[40 * H * D:].reshape(H, 45, D).transpose(1, 0, 2)])
    np.testing.assert_array_equal(back, shd)


def test_gqa_prefill_rows_equal_decode_after_rollback(gpu):
    """Row i of a causal prefill over n_q queries == decode of query i on the
    cache rolled back to T - n_q + i + 1 tokens (prefill kernel vs decode
    kernel, linked by the paged rollback)."""
    from relux_amd import KVCache
    rng = np.random.default_rng(43)
    H, KVH, D, T, nq = 32, 8, 128, 400, 48
    c = KVCache(num_layers=1, max_len=512, num_kv_heads=KVH, head_dim=D, device=gpu.index)
    _fill_gqa(c, rng, gpu, [T], KVH, D)
    q = torch.from_numpy(rng.standard_normal((nq, H, D), dtype=np.float32)).to(gpu)
    full = c.Attend(0, q, H, n_q=[nq]).cpu().numpy()
    for i in (nq - 1, 30, 7, 0):
        c.Rollback(0, c.TotalLen(0) - (T - nq + i + 1))
        one = c.Attend(0, q[i:i + 1].contiguous(), H).cpu().numpy()
        _check(full[i:i + 1], one, (4e-3, 4e-4), f"row {i}")


@pytest.mark.parametrize("H,lens,nqs,mask", [
    (16, [200, 130], [64, 130], "causal"),
    (8, [300], [300], "ref"),
    (32, [96, 160], [40, 100], "causal"),
])
def test_mla_prefill_matches_oracle(gpu, H, lens, nqs, mask):
    from relux_amd import MLACache
    rng = np.random.default_rng(51 + H)
    D, P = 128, 64
    c = MLACache(num_layers=1, max_len=max(lens) + 64, page_tokens=P, max_seqs=len(lens),
                 device=gpu.index)
    cc = rng.standard_normal((sum(lens), 512), dtype=np.float32)
    kr = rng.standard_normal((sum(lens), 64), dtype=np.float32)
    c.Append(0, torch.from_numpy(cc).to(gpu), torch.from_numpy(kr).to(gpu),
             seq_ids=list(range(len(lens))), n_tok=lens)
    w_uk = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    w_uv = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    qn = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    qr = rng.standard_normal((sum(nqs), H, 64), dtype=np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    out = c.Attend(0, t(qn), t(qr), t(w_uk.view(np.int16)).view(torch.bfloat16),
                   t(w_uv.view(np.int16)).view(torch.bfloat16), H, D,
                   seq_ids=list(range(len(lens))), n_q=nqs, mask=mask).cpu().numpy()
    off = toff = 0
    for i, L in enumerate(lens):
        cs = oracle.round_bf16(cc[toff:toff + L])
        ks = oracle.round_bf16(kr[toff:toff + L])
        qci = qn[off:off + nqs[i]].transpose(1, 0, 2)
        qri = qr[off:off + nqs[i]].transpose(1, 0, 2)
        got = out[off:off + nqs[i]].transpose(1, 0, 2)
        exact = _mla_exact(qci, qri, cs, ks, w_uk, w_uv, _limits(mask, nqs[i], L))
        # decompressed K_c / V are rounded to bf16 before attention
        _check(got, exact, (1e-2, 1e-3), f"seq {i} len {L} nq {nqs[i]} vs exact")
        ref = oracle.mla_attend(qci, qri, cs, ks, w_uk, w_uv, mask)
        lim = np.array(_limits(mask, nqs[i], L))
        rows = np.nonzero(lim >= 255)[0]
        if len(rows):
            _check(got[:, rows], ref[:, rows], TOL_ORACLE, f"seq {i} vs oracle (rows >= 256 keys)")
        off += nqs[i]
        toff += L


def test_mla_prefill_after_evict_equals_survivors(gpu):
    """A chunked MLA prefill (the expansion path: the call's rope keys
    gathered through the page table from the first live entry) over
    sequences whose oldest pages were evicted == exact attention over the
    surviving tokens, before and after compaction (row A17)."""
    from relux_amd import MLACache
    rng = np.random.default_rng(61)
    H, D, P = 16, 128, 16
    lens, ev, nqs = [300, 200], [3, 2], [64, 40]
    c = MLACache(num_layers=1, max_len=max(lens) + P, page_tokens=P, max_seqs=2, device=gpu.index)
    cc = rng.standard_normal((sum(lens), 512), dtype=np.float32)
    kr = rng.standard_normal((sum(lens), 64), dtype=np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    c.Append(0, t(cc), t(kr), seq_ids=[0, 1], n_tok=lens)
    c.Evict([0, 1], ev)
    w_uk = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    w_uv = oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D)))
    qn = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    qr = rng.standard_normal((sum(nqs), H, 64), dtype=np.float32)
    args = (t(qn), t(qr), t(w_uk.view(np.int16)).view(torch.bfloat16),
            t(w_uv.view(np.int16)).view(torch.bfloat16), H, D)
    before = c.Attend(0, *args, seq_ids=[0, 1], n_q=nqs).cpu().numpy()
    c.Compact()
    after = c.Attend(0, *args, seq_ids=[0, 1], n_q=nqs).cpu().numpy()
    assert np.array_equal(before, after)
    off = toff = 0
    for i, L in enumerate(lens):
        s0 = toff + ev[i] * P  # first surviving token
        T = L - ev[i] * P
        cs = oracle.round_bf16(cc[s0:toff + L])
        ks = oracle.round_bf16(kr[s0:toff + L])
        exact = _mla_exact(qn[off:off + nqs[i]].transpose(1, 0, 2), qr[off:off + nqs[i]].transpose(1, 0, 2),
                           cs, ks, w_uk, w_uv, _limits("causal", nqs[i], T))
        _check(after[off:off + nqs[i]].transpose(1, 0, 2), exact, (1e-2, 1e-3), f"seq {i} survivors")
        off += nqs[i]
        toff += L


@pytest.mark.parametrize("H,budget_mb", [(24, 2), (16, 3)])
def test_mla_prefill_head_groups_identical(gpu, monkeypatch, H, budget_mb):
    """A chunked-prefill call whose expanded K_c / V^T exceed the expansion
    budget runs head group by head group; each head's attention is the same
    computation, so the output equals the one-group call bit for bit (here
    the budget is shrunk to force 8 and 4 groups of 3 / 5 + a smaller last
    group)."""
    from relux_amd import MLACache
    rng = np.random.default_rng(77 + H)
    D, P, lens, nqs = 128, 64, [700, 300], [200, 120]
    c = MLACache(num_layers=1, max_len=max(lens) + 64, page_tokens=P, max_seqs=2, device=gpu.index)
    c.Append(0, torch.from_numpy(rng.standard_normal((sum(lens), 512), dtype=np.float32)).to(gpu),
             torch.from_numpy(rng.standard_normal((sum(lens), 64), dtype=np.float32)).to(gpu),
             seq_ids=[0, 1], n_tok=lens)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    w = [t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D))).view(np.int16)).view(torch.bfloat16)
         for _ in range(2)]
    qn = t(rng.standard_normal((sum(nqs), H, D), dtype=np.float32))
    qr = t(rng.standard_normal((sum(nqs), H, 64), dtype=np.float32))
    args = (0, qn, qr, w[0], w[1], H, D)
    one = c.Attend(*args, seq_ids=[0, 1], n_q=nqs).cpu()
    # expanded bytes per head: 2 x (768 + 384 padded tokens) x 128 x 2 B = 0.56 MB
    monkeypatch.setenv("RLX_MLA_EXPAND_MB", str(budget_mb))
    grouped = c.Attend(*args, seq_ids=[0, 1], n_q=nqs).cpu()
    assert torch.equal(one, grouped)
    c.close()


@pytest.mark.parametrize("case", ["decode_f32_shd", "decode_bf16_hsd_d64", "multi4_p32", "d80_two",
                                  "d256", "nqt2", "pending_freed", "compacted", "big_plan", "fa2",
                                  "d12_padded", "d100_padded_fa2"])
def test_gqa_append_attend_equals_append_then_attend(gpu, case):
    """rlx_gqa_append_attend against rlx_kv_append followed by
    rlx_gqa_attend on a twin cache: outputs, K/V bytes, page tables, free
    lists and sequence states identical, bit for bit, over two steps -- for
    both source layouts and dtypes, stored head dims 64-256, one and two
    query tiles, table writes pending from a rollback or a compaction, a
    call too large for the kernel-argument plan and the FA2 prefill path."""
    from relux_amd import KVCache
    cfg = {  # H, KVH, D, P, n_tok, B, src dtype, kv layout
        "decode_f32_shd": (8, 2, 128, 16, 1, 6, torch.float32, "SHD"),
        "decode_bf16_hsd_d64": (16, 4, 64, 16, 1, 5, torch.bfloat16, "HSD"),
        "multi4_p32": (8, 2, 128, 32, 4, 7, torch.bfloat16, "SHD"),
        "d80_two": (8, 2, 80, 16, 2, 4, torch.float32, "HSD"),
        "d256": (8, 2, 256, 16, 1, 3, torch.bfloat16, "SHD"),
        "nqt2": (16, 2, 128, 16, 4, 5, torch.bfloat16, "SHD"),
        "pending_freed": (8, 2, 128, 16, 1, 6, torch.bfloat16, "SHD"),
        "compacted": (8, 2, 128, 16, 1, 6, torch.bfloat16, "SHD"),
        "big_plan": (8, 8, 64, 16, 1, 100, torch.bfloat16, "SHD"),
        "fa2": (8, 2, 128, 16, 40, 2, torch.bfloat16, "SHD"),
        # head dims padded to a multiple of 8 at the boundary (K, V, q, out)
        "d12_padded": (4, 2, 12, 16, 2, 4, torch.float32, "HSD"),
        "d100_padded_fa2": (8, 2, 100, 16, 40, 2, torch.bfloat16, "SHD"),
    }[case]
    H, KVH, D, P, ntok, B, dt, kvl = cfg
    rng = np.random.default_rng(sum(map(ord, case)))
    lens = [int(x) for x in rng.integers(20, 400, size=B)]
    seqs = list(range(B))
    caches = [KVCache(num_layers=2, max_len=max(lens) + 4 * P + ntok, num_kv_heads=KVH, head_dim=D,
                      page_tokens=P, max_seqs=B, device=gpu.index) for _ in range(2)]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    k0 = t(rng.standard_normal((sum(lens), KVH, D), dtype=np.float32))
    v0 = t(rng.standard_normal((sum(lens), KVH, D), dtype=np.float32))
    for c in caches:
        c.Append(1, k0, v0, seq_ids=seqs, n_tok=lens, layout="SHD")
        if case == "pending_freed":
            for i in seqs:  # frees pages: their table writes stay pending
                c.Rollback(i, P + 3, layer=1)
        if case == "compacted":
            for i in seqs:  # compaction rewrites live table entries
                c.Evict(i, 1, layer=1)
            c.Compact(layer=1)
    rows = B * ntok
    shape = (rows, KVH, D) if kvl == "SHD" else (rows * KVH, D)  # HSD: per sequence [KVH][n][D]
    k1 = t(rng.standard_normal(shape, dtype=np.float32)).to(dt)
    v1 = t(rng.standard_normal(shape, dtype=np.float32)).to(dt)
    q = t(rng.standard_normal((rows, H, D), dtype=np.float32)).to(dt)
    n_tok = [ntok] * B
    a, f = caches
    a.Append(1, k1, v1, seq_ids=seqs, n_tok=n_tok, layout=kvl)
    want = a.Attend(1, q, H, seq_ids=seqs, n_q=n_tok).cpu()
    got = f.AppendAttend(1, k1, v1, q, H, seq_ids=seqs, n_tok=n_tok, kv_layout=kvl).cpu()
    assert torch.equal(got, want)
    for i in seqs[:6] + seqs[-2:]:
        assert a.SeqState(1, i) == f.SeqState(1, i)
        assert a.PageTable(1, i) == f.PageTable(1, i)
        for x, y in zip(a.View(1, i), f.View(1, i)):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert a.FreeList(1) == f.FreeList(1)
    # a second step reads the first one's new pages through the device table
    a.Append(1, v1, k1, seq_ids=seqs, n_tok=n_tok, layout=kvl)
    want = a.Attend(1, q, H, seq_ids=seqs, n_q=n_tok).cpu()
    got = f.AppendAttend(1, v1, k1, q, H, seq_ids=seqs, n_tok=n_tok, kv_layout=kvl).cpu()
    assert torch.equal(got, want)
    for c in caches:
        c.close()


@pytest.mark.parametrize("case", ["decode_f32", "chunked_bf16", "fa2_bf16", "staged_plans", "groups_h128"])
def test_mla_append_attend_equals_append_then_attend(gpu, case):
    """rlx_mla_append_attend (the append inside the absorb launch on the
    decode path; before the FA2 kernels on the prefill path) against
    rlx_mla_append followed by rlx_mla_attend on a twin cache: outputs,
    latent rows, page tables, free lists and sequence states identical, bit
    for bit.  The twins go through a rollback that frees pages first, so the
    fused call also carries pending page-table writes.  A call with a bad
    argument appends nothing."""
    from relux_amd import MLACache
    rng = np.random.default_rng({"decode_f32": 1, "chunked_bf16": 2, "fa2_bf16": 3, "staged_plans": 4,
                                 "groups_h128": 5}[case])
    P = 64
    # chunked_bf16: 48 query rows per sequence at head_dim 64 take the
    # decode kernels in two head groups; fa2_bf16: 1120 rows at head_dim 128
    # take the expansion + FA2 path; staged_plans: 140 sequences, so the
    # append and the row plans no longer fit the kernel arguments;
    # groups_h128: a 128-head decode step, 4 head groups per sequence.
    H, D, ntok, B = {"decode_f32": (16, 128, 1, 6), "chunked_bf16": (4, 64, 12, 3),
                     "fa2_bf16": (16, 128, 70, 2), "staged_plans": (8, 128, 1, 140),
                     "groups_h128": (128, 128, 1, 5)}[case]
    dt = torch.float32 if case == "decode_f32" else torch.bfloat16
    lens = [int(x) for x in rng.integers(100, 700, size=B)]
    seqs = list(range(B))
    caches = [MLACache(num_layers=2, max_len=max(lens) + 3 * P, page_tokens=P, max_seqs=B,
                       device=gpu.index) for _ in range(2)]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    cc = t(rng.standard_normal((sum(lens), 512), dtype=np.float32))
    kr = t(rng.standard_normal((sum(lens), 64), dtype=np.float32))
    back = [int(x) for x in rng.integers(1, 90, size=B)]  # some cross a page boundary
    for c in caches:
        c.Append(1, cc, kr, seq_ids=seqs, n_tok=lens)
        for i in seqs:
            c.Rollback(i, back[i], layer=1)
    w = [t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D))).view(np.int16)).view(torch.bfloat16)
         for _ in range(2)]
    rows = B * ntok
    c1 = t(rng.standard_normal((rows, 512), dtype=np.float32)).to(dt)
    k1 = t(rng.standard_normal((rows, 64), dtype=np.float32)).to(dt)
    qn = t(rng.standard_normal((rows, H, D), dtype=np.float32)).to(dt)
    qr = t(rng.standard_normal((rows, H, 64), dtype=np.float32)).to(dt)
    n_tok = [ntok] * B
    a, f = caches
    a.Append(1, c1, k1, seq_ids=seqs, n_tok=n_tok)
    want = a.Attend(1, qn, qr, w[0], w[1], H, D, seq_ids=seqs, n_q=n_tok).cpu()
    from relux_amd import _lib
    bad = f._lib.rlx_mla_append_attend(  # head_dim past 256
        f._h, 1, B, _lib.i32_array(seqs), _lib.i32_array(n_tok), c1.data_ptr(), k1.data_ptr(),
        _lib.RLX_F32 if dt == torch.float32 else _lib.RLX_BF16, H, 300, qn.data_ptr(), qr.data_ptr(),
        _lib.RLX_F32 if dt == torch.float32 else _lib.RLX_BF16, w[0].data_ptr(), w[1].data_ptr(), 0.0,
        _lib.RLX_MASK_CAUSAL, torch.empty(rows, H, D, device=gpu).data_ptr(), _lib.RLX_F32)
    assert bad == _lib.RLX_ERR_UNSUPPORTED
    assert [f.TotalLen(1, i) for i in seqs] == [lens[i] - back[i] for i in seqs]
    got = f.AppendAttend(1, c1, k1, qn, qr, w[0], w[1], H, D, seq_ids=seqs, n_tok=n_tok).cpu()
    assert torch.equal(got, want)
    for i in seqs[:8] + seqs[-2:]:
        assert a.TotalLen(1, i) == f.TotalLen(1, i)
        assert a.SeqState(1, i) == f.SeqState(1, i)
        assert a.PageTable(1, i) == f.PageTable(1, i)
        for x, y in zip(a.View(1, i), f.View(1, i)):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert a.FreeList(1) == f.FreeList(1)
    for c in caches:
        c.close()


def test_mla_append_attend_failures_keep_host_and_device_in_step(gpu, monkeypatch):
    """rlx_mla_append_attend on the decode path carries the append in the
    attention's first launch.  When the call fails after the host has
    committed the append (here the workspace, capped by RLX_WS_MAX_KB), the
    tokens and their page-table writes still reach the device: the gather
    through the device table returns the appended rows, the host table and
    state equal a twin's that ran Append alone, and the next attention
    equals the twin's bit for bit.  A prefill refused for its expansion size
    (RLX_MLA_EXPAND_MB below one head) appends nothing."""
    from relux_amd import MLACache, ReluxError, _lib
    rng = np.random.default_rng(17)
    H, D, B, P = 16, 128, 5, 64
    lens = [130, 64, 200, 1, 77]
    seqs = list(range(B))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    a, f = [MLACache(num_layers=1, max_len=2304, page_tokens=P, max_seqs=B, device=gpu.index)
            for _ in range(2)]
    cc = t(rng.standard_normal((sum(lens), 512), dtype=np.float32))
    kr = t(rng.standard_normal((sum(lens), 64), dtype=np.float32))
    for c in (a, f):
        c.Append(0, cc, kr, seq_ids=seqs, n_tok=lens)
    w = [t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, H * D))).view(np.int16)).view(torch.bfloat16)
         for _ in range(2)]
    c1 = t(rng.standard_normal((B, 512), dtype=np.float32))
    k1 = t(rng.standard_normal((B, 64), dtype=np.float32))
    qn = t(rng.standard_normal((B, H, D), dtype=np.float32))
    qr = t(rng.standard_normal((B, H, 64), dtype=np.float32))
    a.Append(0, c1, k1, seq_ids=seqs, n_tok=[1] * B)  # sequence 1 opens a new page
    monkeypatch.setenv("RLX_WS_MAX_KB", "1")
    with pytest.raises(ReluxError):
        f.AppendAttend(0, c1, k1, qn, qr, w[0], w[1], H, D, seq_ids=seqs, n_tok=[1] * B)
    monkeypatch.delenv("RLX_WS_MAX_KB")
    for i in seqs:
        assert a.SeqState(0, i) == f.SeqState(0, i)
        assert a.PageTable(0, i) == f.PageTable(0, i)
        for x, y in zip(a.View(0, i), f.View(0, i)):  # through the device table
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert a.FreeList(0) == f.FreeList(0)
    want = a.Attend(0, qn, qr, w[0], w[1], H, D, seq_ids=seqs).cpu()
    got = f.Attend(0, qn, qr, w[0], w[1], H, D, seq_ids=seqs).cpu()
    assert torch.equal(got, want)
    # prefill (80 query rows per sequence, the expansion + FA2 path forced
    # past 32 rows) whose single head would expand past a 1 MB budget:
    # refused before the append
    monkeypatch.setenv("RLX_MLA_FA2_ROWS", "32")
    monkeypatch.setenv("RLX_MLA_EXPAND_MB", "1")
    n5 = [5] * B
    c5 = t(rng.standard_normal((5 * B, 512), dtype=np.float32))
    k5 = t(rng.standard_normal((5 * B, 64), dtype=np.float32))
    q5 = t(rng.standard_normal((5 * B, H, D), dtype=np.float32))
    r5 = t(rng.standard_normal((5 * B, H, 64), dtype=np.float32))
    f.Append(0, t(rng.standard_normal((2000, 512), dtype=np.float32)),
             t(rng.standard_normal((2000, 64), dtype=np.float32)), seq_ids=[2], n_tok=[2000])
    before = [f.SeqState(0, i) for i in seqs]
    with pytest.raises(ReluxError) as e:
        f.AppendAttend(0, c5, k5, q5, r5, w[0], w[1], H, D, seq_ids=seqs, n_tok=n5)
    assert e.value.code == _lib.RLX_ERR_UNSUPPORTED
    assert [f.SeqState(0, i) for i in seqs] == before
    monkeypatch.delenv("RLX_MLA_EXPAND_MB")
    for c in (a, f):
        c.close()


@pytest.mark.parametrize("KVH,D,chunks,nq,mask", [
    (4, 64, [[5, 1, 3, 7, 1, 16, 2], [9, 1, 1, 30]], 1, "ref"),
    (2, 128, [[40, 1, 1, 1], [17, 5]], 3, "causal"),
    (8, 16, [[20], [3, 3, 3]], 20, "ref"),   # prefill row: n_q == len on sequence 0
])
def test_reference_byte_image_attention(gpu, KVH, D, chunks, nq, mask):
    """rlx_gqa_attend_ref_image reads head h at token t from the D-row at
    flat index h*T + t of the reference KVCache buffer, whose rows each
    Append filled with its raw [KVH, S, D] block: exact f64 attention over
    the byte image the oracle rebuilds from the same appends."""
    from relux_amd import KVCache, ReluxError
    rng = np.random.default_rng(KVH * 100 + D + nq)
    H = 2 * KVH
    S = len(chunks)
    lens = [sum(ch) for ch in chunks]
    c = KVCache(num_layers=1, max_len=max(lens) + 16, num_kv_heads=KVH, head_dim=D, page_tokens=16,
                max_seqs=S, device=gpu.index)
    logical = [[np.zeros((KVH, 0, D), np.float32)] * 2 for _ in range(S)]
    for step in range(max(len(ch) for ch in chunks)):
        ids = [i for i in range(S) if step < len(chunks[i])]
        n = [chunks[i][step] for i in ids]
        k = rng.standard_normal((sum(n), KVH, D), dtype=np.float32)
        v = rng.standard_normal((sum(n), KVH, D), dtype=np.float32)
        c.Append(0, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), seq_ids=ids, n_tok=n,
                 layout="SHD")
        off = 0
        for i, ni in zip(ids, n):
            kb = oracle.round_bf16(k[off:off + ni]).transpose(1, 0, 2)
            vb = oracle.round_bf16(v[off:off + ni]).transpose(1, 0, 2)
            logical[i] = [np.concatenate([logical[i][0], kb], 1), np.concatenate([logical[i][1], vb], 1)]
            off += ni
    nqs = [min(nq, L) for L in lens]
    q = rng.standard_normal((sum(nqs), H, D), dtype=np.float32)
    out = c.AttendRefImage(0, torch.from_numpy(q).to(gpu), H, seq_ids=list(range(S)), n_q=nqs,
                           mask=mask).cpu().numpy()
    off = 0
    for i, L in enumerate(lens):
        img_k = td.ref_byte_image(logical[i][0], chunks[i], L).reshape(KVH, L, D)
        img_v = td.ref_byte_image(logical[i][1], chunks[i], L).reshape(KVH, L, D)
        G = H // KVH
        qi = q[off:off + nqs[i]].transpose(1, 0, 2)
        want = oracle.exact_attention_f64(qi, np.repeat(img_k, G, 0), np.repeat(img_v, G, 0),
                                          _limits(mask, nqs[i], L))
        _check(out[off:off + nqs[i]].transpose(1, 0, 2), want, TOL_EXACT, f"seq {i}")
        off += nqs[i]
    # a rollback of whole appends keeps the image; one that cuts an append does not
    if len(chunks[0]) < 2:
        c.close()
        return
    last = chunks[0][-1]
    c.Rollback(0, last)
    q1 = torch.from_numpy(q[:1].copy()).to(gpu)
    got = c.AttendRefImage(0, q1, H, seq_ids=[0], n_q=[1], mask=mask).cpu().numpy()
    L0 = lens[0] - last
    img_k = td.ref_byte_image(logical[0][0][:, :L0], chunks[0][:-1], L0).reshape(KVH, L0, D)
    img_v = td.ref_byte_image(logical[0][1][:, :L0], chunks[0][:-1], L0).reshape(KVH, L0, D)
    want = oracle.exact_attention_f64(q[:1].transpose(1, 0, 2), np.repeat(img_k, H // KVH, 0),
                                      np.repeat(img_v, H // KVH, 0), [L0 - 1])
    _check(got.transpose(1, 0, 2), want, TOL_EXACT, "after rollback of the last append")
    if chunks[0][-2] > 1:
        c.Rollback(0, 1)
        with pytest.raises(ReluxError):
            c.AttendRefImage(0, q1, H, seq_ids=[0], n_q=[1])
    c.close()


def test_spec_verify_stress_small(gpu):
    """Config 5 at small scale: every step appends 4 drafts per sequence,
    verifies them (4 drafts x 8 heads = 32 rows per kv head), rolls back a
    random suffix; every 8 steps the oldest 25% of full pages are evicted
    and the table compacted.  Attention is checked each step against exact
    f64 attention over the logical surviving tokens, and the integer state
    against the page-table model."""
    from relux_amd import KVCache
    from oracle.paged import PagedModel
    rng = np.random.default_rng(55)
    B, H, KVH, D, P, nd = 6, 64, 8, 128, 16, 4
    lens = [int(x) for x in np.exp(rng.uniform(np.log(40), np.log(700), size=B))]
    maxp = 80
    c = KVCache(num_layers=1, max_len=maxp * P, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=B, pool_pages=B * maxp, device=gpu.index)
    m = PagedModel(1, P, B * maxp, B, maxp)
    K, V = _fill_gqa(c, rng, gpu, lens, KVH, D)
    for ci in range(2):  # the same two multi-sequence Append calls _fill_gqa made
        m.append(0, list(range(B)), [(L * (ci + 1)) // 2 - (L * ci) // 2 for L in lens])
    Kl = [list(K[i].transpose(1, 0, 2)) for i in range(B)]  # per-token [KVH, D]
    Vl = [list(V[i].transpose(1, 0, 2)) for i in range(B)]
    seqs = list(range(B))
    g = H // KVH
    for step in range(24):
        kd = rng.standard_normal((B * nd, KVH, D), dtype=np.float32)
        vd = rng.standard_normal((B * nd, KVH, D), dtype=np.float32)
        c.Append(0, torch.from_numpy(kd).to(gpu), torch.from_numpy(vd).to(gpu), seq_ids=seqs,
                 n_tok=[nd] * B, layout="SHD")
        m.append(0, seqs, [nd] * B)
        for i in range(B):
            Kl[i].extend(oracle.round_bf16(kd[i * nd:(i + 1) * nd]))
            Vl[i].extend(oracle.round_bf16(vd[i * nd:(i + 1) * nd]))
        q = rng.standard_normal((B * nd, H, D), dtype=np.float32)
        out = c.Attend(0, torch.from_numpy(q).to(gpu), H, seq_ids=seqs, n_q=[nd] * B).cpu().numpy()
        for i in (step % B, (step + 3) % B):
            Ki = np.repeat(np.stack(Kl[i], axis=1), g, 0)
            Vi = np.repeat(np.stack(Vl[i], axis=1), g, 0)
            T = Ki.shape[1]
            exact = oracle.exact_attention_f64(q[i * nd:(i + 1) * nd].transpose(1, 0, 2), Ki, Vi,
                                               [T - nd + j for j in range(nd)])
            _check(out[i * nd:(i + 1) * nd].transpose(1, 0, 2), exact, TOL_EXACT,
                   f"step {step} seq {i} T {T}")
        r = [int(x) for x in rng.integers(0, nd + 1, size=B)]
        c.Rollback(seqs, r)
        for i in range(B):
            m.rollback(0, i, r[i])
            if r[i]:
                del Kl[i][len(Kl[i]) - r[i]:]
                del Vl[i][len(Vl[i]) - r[i]:]
        if step % 8 == 7:
            ev = [int(m.len[0, i] // P) // 4 for i in range(B)]
            c.Evict(seqs, ev)
            c.Compact()
            for i in range(B):
                m.evict(0, i, ev[i])
                del Kl[i][: ev[i] * P]
                del Vl[i][: ev[i] * P]
            m.compact(0)
        for i in range(B):
            assert c.SeqState(0, i) == m.state(0, i)
            assert c.PageTable(0, i) == list(m.table[0][i])
        assert c.FreeList(0) == m.free[0]


def test_kernel_timing_counts_and_leaves_results_unchanged(gpu):
    """The timing events bench.py reads: one event pair per attention launch
    (GQA decode, MLA decode, FA2 prefill), positive durations that add up,
    and outputs bit-identical to untimed calls."""
    from relux_amd import KVCache, MLACache
    rng = np.random.default_rng(404)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    g = KVCache(num_layers=1, max_len=1024, num_kv_heads=2, head_dim=128, page_tokens=16, max_seqs=2,
                device=gpu.index)
    lens = [300, 700]
    k = t(rng.standard_normal((sum(lens), 2, 128), dtype=np.float32))
    g.Append(0, k, k * 0.5, seq_ids=[0, 1], n_tok=lens, layout="SHD")
    q1 = t(rng.standard_normal((2, 8, 128), dtype=np.float32))
    qp = t(rng.standard_normal((sum(lens), 8, 128), dtype=np.float32))
    m = MLACache(num_layers=1, max_len=1024, page_tokens=64, max_seqs=2, device=gpu.index)
    m.Append(0, t(rng.standard_normal((sum(lens), 512), dtype=np.float32)),
             t(rng.standard_normal((sum(lens), 64), dtype=np.float32)), seq_ids=[0, 1], n_tok=lens)
    w = [t(oracle.bf16_from_f32(rng.normal(0, 0.02, size=(512, 16 * 128))).view(np.int16)).view(torch.bfloat16)
         for _ in range(2)]
    mq = (t(rng.standard_normal((2, 16, 128), dtype=np.float32)), t(rng.standard_normal((2, 16, 64), dtype=np.float32)))

    def calls():
        return [g.Attend(0, q1, 8, seq_ids=[0, 1]).cpu(),
                g.Attend(0, qp, 8, seq_ids=[0, 1], n_q=lens).cpu(),  # FA2 prefill
                m.Attend(0, mq[0], mq[1], w[0], w[1], 16, 128, seq_ids=[0, 1]).cpu()]

    plain = calls()
    for c in (g, m):
        c.Timing(True)
    timed = calls()
    (gms, gn), (mms, mn) = g.KernelTime(), m.KernelTime()
    assert (gn, mn) == (2, 1)
    assert 0.0 < gms < 100.0 and 0.0 < mms < 100.0
    for a, b in zip(plain, timed):
        assert torch.equal(a, b)
    for c in (g, m):
        c.Timing(False)
    calls()
    assert g.KernelTime() == (0.0, 0) and m.KernelTime() == (0.0, 0)
    g.close()
    m.close()
