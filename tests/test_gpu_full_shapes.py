"""GPU parity at the exact BASELINE shapes of configs 3, 4 and 5, with the
dtypes the bench runs them in (bf16 queries and outputs, bf16 cache).

  * config 3 -- MLA latent decode, B 32, H 16, d_c 512, d_r 64, T 8192,
    64-token pages scattered over the pool, one appended latent row per
    sequence before attention (mla.go:316-377, absorbed);
  * config 4 -- MLA chunked prefill, 4 sequences x (6144 cached + 2048 new),
    128 heads, causal with the cache offset (mla.go:316-377, decompressed);
  * config 5 -- GQA speculative verify stress, B 64, H 64, KVH 8, D 128,
    T log-uniform in [1k, 32k], 16-token pages: each step appends 4 drafts
    per sequence, verifies them causally, rolls back U{0..4} tokens; at step
    256 the oldest 25% of every sequence's full pages are evicted and the
    table compacted (speculative.go:89-163 loop shape).

References are computed from the logical inputs the test generated (never
from the cache's own gather): torch f32 exact-softmax attention on the GPU
for every checked row, and the oracle's restatement of the Go loops
(fastexp32 softmax) on sampled rows at the north-star tolerance.
"""
import math
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TOL_ORACLE = (2e-2, 2e-3)
TOL_EXACT = (1e-2, 1e-3)
TOL_MLA_EXACT = (5e-3, 5e-4)


def _check(got, want, tol, what):
    got = got.double() if torch.is_tensor(got) else torch.from_numpy(np.asarray(got, np.float64))
    want = want.double() if torch.is_tensor(want) else torch.from_numpy(np.asarray(want, np.float64))
    err = (got.cpu() - want.cpu()).abs()
    assert err.max().item() <= tol[0] and err.mean().item() <= tol[1], (
        f"{what}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e} (tol {tol})")


def _fill_interleaved(append_fn, lens, P, rng):
    """Append every sequence's tokens one page at a time, sequences in a fresh
    random order each round (pages of a sequence scattered over the pool)."""
    left = list(lens)
    while any(left):
        order = [int(i) for i in rng.permutation(len(lens)) if left[i] > 0]
        n = [min(P, left[i]) for i in order]
        append_fn(order, n)
        for i, ni in zip(order, n):
            left[i] -= ni


def _np(t):
    return t.float().cpu().numpy()


# ---- config 3 ----------------------------------------------------------------

def test_mla_config3_full_shape(gpu):
    from relux_amd import MLACache
    torch.manual_seed(3)
    rng = np.random.default_rng(3)
    B, H, D, dC, dR, T, P = 32, 16, 128, 512, 64, 8192, 64
    c = MLACache(num_layers=1, max_len=T + P, page_tokens=P, max_seqs=B,
                 pool_pages=B * (T // P) + 8, device=gpu.index)
    lat = torch.randn(B, T, dC, device=gpu).bfloat16()     # logical latent rows
    rope = torch.randn(B, T, dR, device=gpu).bfloat16()
    done = [0] * B

    def app(order, n):
        cc = torch.cat([lat[s, done[s]:done[s] + k] for s, k in zip(order, n)])
        kr = torch.cat([rope[s, done[s]:done[s] + k] for s, k in zip(order, n)])
        c.Append(0, cc, kr, seq_ids=order, n_tok=n)
        for s, k in zip(order, n):
            done[s] += k
    _fill_interleaved(app, [T - 1] * B, P, rng)
    # the decode step's own append: one latent row per sequence
    c.Append(0, lat[:, T - 1].contiguous(), rope[:, T - 1].contiguous(), seq_ids=list(range(B)),
             n_tok=[1] * B)
    w_uk = (torch.randn(dC, H * D, device=gpu) * 0.02).bfloat16()
    w_uv = (torch.randn(dC, H * D, device=gpu) * 0.02).bfloat16()
    qn = torch.randn(B, H, D, device=gpu).bfloat16()
    qr = torch.randn(B, H, dR, device=gpu).bfloat16()
    out = torch.empty(B, H, D, device=gpu, dtype=torch.bfloat16)
    c.Attend(0, qn, qr, w_uk, w_uv, H, D, seq_ids=list(range(B)), out=out)
    torch.cuda.synchronize()
    for s in range(B):
        assert c.TotalLen(0, s) == T
    Wk = w_uk.float().view(dC, H, D)
    Wv = w_uv.float().view(dC, H, D)
    for s in range(B):
        cc, kk = lat[s].float(), rope[s].float()
        qlat = torch.einsum("chd,hd->hc", Wk, qn[s].float())
        sc = (qlat @ cc.T + qr[s].float() @ kk.T) / math.sqrt(D + dR)
        ref = torch.einsum("hc,chd->hd", torch.softmax(sc, dim=-1) @ cc, Wv)
        _check(out[s].float(), ref, TOL_MLA_EXACT, f"config 3 row {s} vs torch f32")
    # the reference loops themselves (decompress-all, fastexp32) on two rows
    wuk_u16 = w_uk.view(torch.int16).cpu().numpy().view(np.uint16)
    wuv_u16 = w_uv.view(torch.int16).cpu().numpy().view(np.uint16)

    def ref_row(s):
        return oracle.mla_attend(_np(qn[s])[:, None, :], _np(qr[s])[:, None, :], _np(lat[s]),
                                 _np(rope[s]), wuk_u16, wuv_u16, "causal")[:, 0, :]
    rows = (5, 27)
    with ThreadPoolExecutor(len(rows)) as ex:
        refs = list(ex.map(ref_row, rows))
    for s, ref in zip(rows, refs):
        _check(out[s].float(), ref, TOL_ORACLE, f"config 3 row {s} vs oracle")
    c.close()


# ---- config 4 ----------------------------------------------------------------

def test_mla_config4_full_shape(gpu):
    from relux_amd import MLACache
    torch.manual_seed(4)
    rng = np.random.default_rng(4)
    B, H, D, dC, dR, T0, n, P = 4, 128, 128, 512, 64, 6144, 2048, 64
    T = T0 + n
    c = MLACache(num_layers=1, max_len=T + P, page_tokens=P, max_seqs=B,
                 pool_pages=B * (T // P) + 8, device=gpu.index)
    lat = torch.randn(B, T, dC, device=gpu).bfloat16()
    rope = torch.randn(B, T, dR, device=gpu).bfloat16()
    done = [0] * B

    def app(order, cnt):
        cc = torch.cat([lat[s, done[s]:done[s] + k] for s, k in zip(order, cnt)])
        kr = torch.cat([rope[s, done[s]:done[s] + k] for s, k in zip(order, cnt)])
        c.Append(0, cc, kr, seq_ids=order, n_tok=cnt)
        for s, k in zip(order, cnt):
            done[s] += k
    _fill_interleaved(app, [T0] * B, P, rng)
    seqs = list(range(B))
    # the chunk: 2048 new latent rows per sequence in one multi-sequence call
    c.Append(0, lat[:, T0:].reshape(B * n, dC).contiguous(), rope[:, T0:].reshape(B * n, dR).contiguous(),
             seq_ids=seqs, n_tok=[n] * B)
    w_uk = (torch.randn(dC, H * D, device=gpu) * 0.02).bfloat16()
    w_uv = (torch.randn(dC, H * D, device=gpu) * 0.02).bfloat16()
    qn = torch.randn(B * n, H, D, device=gpu).bfloat16()
    qr = torch.randn(B * n, H, dR, device=gpu).bfloat16()
    out = torch.empty(B * n, H, D, device=gpu, dtype=torch.bfloat16)
    c.Attend(0, qn, qr, w_uk, w_uv, H, D, seq_ids=seqs, n_q=[n] * B, out=out)
    torch.cuda.synchronize()
    mask = torch.arange(T, device=gpu)[None, :] <= (T0 + torch.arange(n, device=gpu))[:, None]
    heads = {0: (0, 77, 101, 127), 1: (3, 45, 64, 90), 2: (17, 33, 111, 126), 3: (1, 58, 96, 120)}
    for s in seqs:
        cc, kk = lat[s].float(), rope[s].float()
        for h in heads[s]:
            kc = cc @ w_uk.float()[:, h * D:(h + 1) * D]        # decompressed K^C, f32
            v = cc @ w_uv.float()[:, h * D:(h + 1) * D]
            sc = (qn[s * n:(s + 1) * n, h].float() @ kc.T + qr[s * n:(s + 1) * n, h].float() @ kk.T)
            sc = (sc / math.sqrt(D + dR)).masked_fill(~mask, float("-inf"))
            ref = torch.softmax(sc, dim=-1) @ v
            _check(out[s * n:(s + 1) * n, h].float(), ref, TOL_EXACT, f"config 4 seq {s} head {h}")
    # one head of one sequence through the reference loops (every row here
    # attends >= 6145 keys, where fastexp32's weight error averages out)
    s, h = 2, 111
    want = oracle.mla_attend(
        _np(qn[s * n:(s + 1) * n, h])[None], _np(qr[s * n:(s + 1) * n, h])[None], _np(lat[s]),
        _np(rope[s]), w_uk[:, h * D:(h + 1) * D].contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
        w_uv[:, h * D:(h + 1) * D].contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
        "causal")[0]
    _check(out[s * n:(s + 1) * n, h].float(), want, TOL_ORACLE, f"config 4 seq {s} head {h} vs oracle")
    c.close()


# ---- config 5 ----------------------------------------------------------------

class _Mirror:
    """Logical K/V of every sequence, kept apart from the cache: a device
    buffer per sequence with a live window [start, end)."""

    def __init__(self, lens, cap, KVH, D, dev):
        self.k = [torch.empty(L + cap, KVH, D, device=dev, dtype=torch.bfloat16) for L in lens]
        self.v = [torch.empty_like(x) for x in self.k]
        self.start = [0] * len(lens)
        self.end = [0] * len(lens)

    def append(self, s, k, v):
        e = self.end[s]
        self.k[s][e:e + k.shape[0]] = k
        self.v[s][e:e + k.shape[0]] = v
        self.end[s] += k.shape[0]

    def live(self, s):
        return self.k[s][self.start[s]:self.end[s]], self.v[s][self.start[s]:self.end[s]]


def test_spec_stress_config5_full_shape(gpu):
    from oracle.paged import PagedModel
    from relux_amd import KVCache
    torch.manual_seed(5)
    rng = np.random.default_rng(5)
    B, H, KVH, D, P, nd, evict_every = 64, 64, 8, 128, 16, 4, 256
    steps = evict_every + 4                    # one evict + compact at step 256
    lens = [int(x) for x in np.exp(rng.uniform(np.log(1024), np.log(32768), size=B))]
    grow = nd * steps
    max_pages = -(-(max(lens) + grow) // P)
    pool = sum(-(-(T + grow) // P) for T in lens) + 8
    c = KVCache(num_layers=1, max_len=max_pages * P, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=B, pool_pages=pool, device=gpu.index)
    m = PagedModel(1, P, pool, B, max_pages)
    mir = _Mirror(lens, grow, KVH, D, gpu)

    def app(order, n):
        k = torch.randn(sum(n), KVH, D, device=gpu).bfloat16()
        v = torch.randn_like(k)
        c.Append(0, k, v, seq_ids=order, n_tok=n, layout="SHD")
        m.append(0, order, n)
        off = 0
        for s, ni in zip(order, n):
            mir.append(s, k[off:off + ni], v[off:off + ni])
            off += ni
    # fill 1024 tokens per sequence per call, sequences in random order
    left = list(lens)
    while any(left):
        order = [int(i) for i in rng.permutation(B) if left[i] > 0]
        n = [min(1024, left[i]) for i in order]
        app(order, n)
        for s, ni in zip(order, n):
            left[s] -= ni
    seqs = list(range(B))
    g = H // KVH

    def check_state(step):
        for s in seqs:
            assert c.SeqState(0, s) == m.state(0, s), (step, s)
            assert c.PageTable(0, s) == list(m.table[0][s]), (step, s)
        assert c.FreeList(0) == m.free[0], step

    def check_rows(q, out, rows, step):
        for s in rows:
            k, v = mir.live(s)
            T = k.shape[0]
            kf = k.float().permute(1, 0, 2).contiguous()                   # [KVH, T, D]
            vf = v.float().permute(1, 0, 2).contiguous()
            # query head h = kv * g + j; rows of kv head kv are (j, i)
            qs = q[s * nd:(s + 1) * nd].float().permute(1, 0, 2).reshape(KVH, g * nd, D)
            sc = torch.bmm(qs, kf.transpose(1, 2).contiguous()) / math.sqrt(D)
            lim = T - nd + torch.arange(g * nd, device=gpu) % nd
            sc = sc.masked_fill(torch.arange(T, device=gpu)[None, None, :] > lim[None, :, None],
                                float("-inf"))
            ref = torch.bmm(torch.softmax(sc, dim=-1), vf).reshape(H, nd, D)
            _check(out[s * nd:(s + 1) * nd].float().permute(1, 0, 2), ref, TOL_EXACT,
                   f"step {step} seq {s} T {T}")

    check_state(-1)
    evictions = 0
    out = torch.empty(B * nd, H, D, device=gpu, dtype=torch.bfloat16)
    for step in range(steps):
        kd = torch.randn(B * nd, KVH, D, device=gpu).bfloat16()
        vd = torch.randn_like(kd)
        c.Append(0, kd, vd, seq_ids=seqs, n_tok=[nd] * B, layout="SHD")
        m.append(0, seqs, [nd] * B)
        for s in seqs:
            mir.append(s, kd[s * nd:(s + 1) * nd], vd[s * nd:(s + 1) * nd])
        q = torch.randn(B * nd, H, D, device=gpu).bfloat16()
        c.Attend(0, q, H, seq_ids=seqs, n_q=[nd] * B, out=out)
        # every row on the first step and on the steps either side of the
        # eviction, four rotating rows on the others
        if step in (0, evict_every - 1, evict_every, steps - 1):
            rows = seqs
        else:
            rows = [(step * 4 + j) % B for j in range(4)]
        check_rows(q, out, rows, step)
        r = [int(x) for x in rng.integers(0, nd + 1, size=B)]
        c.Rollback(seqs, r)
        for s in seqs:
            m.rollback(0, s, r[s])
            mir.end[s] -= r[s]
        if (step + 1) % evict_every == 0:
            ev = [int(m.len[0, s] // P) // 4 for s in seqs]
            c.Evict(seqs, ev)
            c.Compact()
            for s in seqs:
                m.evict(0, s, ev[s])
                mir.start[s] += ev[s] * P
            m.compact(0)
            evictions += 1
        check_state(step)
    assert evictions == 1
    c.close()
