"""Token selection on the device (rlx_greedy, rlx_sample, rlx_spec_accept)
against the oracle's restatement of sampler.go / speculative.go on the same
logits and draws, and the speculative decoder end to end on the paged GPU
caches.

Bar: token ids equal.  The device sums the vocabulary block-parallel, the
reference sequentially, so a draw that lies within a few ulp of a
cumulative boundary may land on the neighbouring token; a case counts only
when the oracle's own answer is unchanged with the draws moved by +-1e-5
(the test reports how many were excluded; with a 50k vocabulary a few
rows per 24 are, as token boundaries sit closer together).
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import sampling as S
from oracle import tiny_decoder as td

pytestmark = pytest.mark.gpu

DELTA = 1e-5


@pytest.fixture(scope="module")
def handle(gpu):
    from relux_amd import KVCache
    return KVCache(num_layers=1, max_len=64, num_kv_heads=1, head_dim=64, page_tokens=16,
                   device=gpu.index)


def dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu)


def make_sampler(p, draws=None):
    from relux_amd import Sampler
    return Sampler(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                   repeat_penalty=p.repeat_penalty, frequency_penalty=p.frequency_penalty,
                   presence_penalty=p.presence_penalty, repeat_window=p.repeat_window, rand=draws)


def test_greedy(gpu, handle):
    from relux_amd import Sampler
    rng = np.random.default_rng(11)
    for V in (7, 1000, 32000):
        x = rng.normal(0, 1, (9, V)).astype(np.float32)
        x[1, [3, V - 1]] = 50.0  # tie: first index wins
        x[2, :] = 0.0
        got = Sampler().Greedy(dev(x, gpu), handle)
        assert got == [S.greedy(r) for r in x], V


PARAMS = {
    "plain": S.SamplerParams(),
    "temp0.7": S.SamplerParams(temperature=0.7),
    "temp0": S.SamplerParams(temperature=0.0),
    "topk5": S.SamplerParams(top_k=5),
    "topk50_t1.3": S.SamplerParams(top_k=50, temperature=1.3),
    "topp0.9": S.SamplerParams(top_p=0.9),
    "minp0.05": S.SamplerParams(min_p=0.05),
    "all": S.SamplerParams(temperature=0.8, top_k=40, top_p=0.95, min_p=0.02),
    # top-k chunks select before the division by the temperature
    "topk5_t0": S.SamplerParams(top_k=5, temperature=0.0),
    "topk40_t25": S.SamplerParams(top_k=40, temperature=25.0, top_p=0.9),
    "penalties": S.SamplerParams(repeat_penalty=1.3, frequency_penalty=0.2, presence_penalty=0.3,
                                 repeat_window=16),
}


# V 50000 is past the LDS row (32768 entries): the whole-row path's
# memory-read form, with the penalised tokens in the LDS bitmap.  With top-k
# on and V past 8192 the vocabulary is split over work-groups (V 32000: 4
# chunks of 8000; V 50000: 7), each keeping its own candidates; V 50257 and
# 32003 put every row but the first off 16-byte alignment (the chunks' loads
# fall back to single floats).
CASES = [(n, V) for V in (100, 4096) for n in sorted(PARAMS)] + \
    [(n, 32000) for n in ("topk5", "topk50_t1.3", "all", "topk5_t0", "topk40_t25")] + \
    [(n, 50000) for n in ("plain", "temp0.7", "topk5", "all", "penalties")] + \
    [("all", 50257), ("topk50_t1.3", 32003)]


@pytest.mark.parametrize("name,V", CASES)
def test_sample(gpu, handle, name, V):
    p = PARAMS[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()) + V)
    rows = 24
    x = rng.normal(0, 2.5, (rows, V)).astype(np.float32)
    u = rng.random(rows, dtype=np.float32)
    prev = [list(rng.integers(0, V, rng.integers(0, 40))) for _ in range(rows)]
    got = make_sampler(p, S.Draws(u)).Sample(dev(x, gpu), prev, handle)
    kept = 0
    for i in range(rows):
        want = S.sample(x[i], p, u[i], prev=prev[i])
        if S.sample(x[i], p, u[i] - DELTA, prev=prev[i]) != want or \
                S.sample(x[i], p, u[i] + DELTA, prev=prev[i]) != want:
            continue
        kept += 1
        assert got[i] == want, (name, V, i, got[i], want)
    print(f"sample {name} V{V}: {kept}/{rows} robust rows compared")
    assert kept >= rows // 2


def test_sample_split_ties(gpu, handle):
    """Ties at a chunk's k-th largest value: a chunk list past its slots (or a
    merge past the candidate capacity) sends the row down the whole-row
    path, smaller ties stay on the split path; every row agrees with the
    oracle, which keeps all entries tied with the k-th largest."""
    rng = np.random.default_rng(77)
    V, rows = 32000, 8
    x = rng.normal(0, 2.5, (rows, V)).astype(np.float32)
    x[0, :] = 0.0                    # ties at every chunk's k-th largest: all lists overflow;
    x[0, [5, 17000, 31000]] = 12.0   # three entries hold most of the mass (a flat row's
    #                                  sequential f32 sums drift by 1e-4 over 32000 entries)
    x[1, 100:400] = 12.0             # 300 tied maxima in one chunk (past its slots)
    x[2, ::500] = 12.0               # 64 tied maxima spread over the 4 chunks
    x[3, 7990:8010] = 12.0           # ties across a chunk boundary (chunks of 8000)
    x[4, :] = np.round(x[4, :])      # a few thousand entries on each integer
    x[5, 31990:] = 12.0              # ties in the last chunk
    x[6, :60] = np.float32(-np.inf)  # masked entries in the first chunk
    u = rng.random(rows, dtype=np.float32)
    for p in (S.SamplerParams(top_k=50, temperature=0.9), S.SamplerParams(top_k=5, min_p=0.05)):
        got = make_sampler(p, S.Draws(u)).Sample(dev(x, gpu), None, handle)
        kept = 0
        for i in range(rows):
            want = S.sample(x[i], p, u[i])
            if S.sample(x[i], p, u[i] - DELTA) != want or S.sample(x[i], p, u[i] + DELTA) != want:
                continue
            kept += 1
            assert got[i] == want, (p, i, got[i], want)
        assert kept >= rows // 2


# Split-path boundaries: the smallest split (V 8193: two chunks), top-k at
# both ends of the split path (1 and 256, the largest it takes), many
# chunks (V 65537: nine), and top-p / min-p filtering after the merge.
SPLIT_EDGES = [
    (8193, S.SamplerParams(top_k=1)),
    (8193, S.SamplerParams(top_k=256, temperature=1.1)),
    (65537, S.SamplerParams(top_k=256, top_p=0.8, min_p=0.01)),
    (65537, S.SamplerParams(top_k=7, temperature=0.5)),
    (20000, S.SamplerParams(top_k=100, top_p=0.5, min_p=0.1, temperature=1.7)),
]


@pytest.mark.parametrize("V,p", SPLIT_EDGES)
def test_sample_split_edges(gpu, handle, V, p):
    rng = np.random.default_rng(V + p.top_k)
    rows = 16
    x = rng.normal(0, 2.5, (rows, V)).astype(np.float32)
    u = rng.random(rows, dtype=np.float32)
    got = make_sampler(p, S.Draws(u)).Sample(dev(x, gpu), None, handle)
    kept = 0
    for i in range(rows):
        want = S.sample(x[i], p, u[i])
        if S.sample(x[i], p, u[i] - DELTA) != want or S.sample(x[i], p, u[i] + DELTA) != want:
            continue
        kept += 1
        assert got[i] == want, (V, p, i, got[i], want)
    print(f"split edge V{V} k{p.top_k}: {kept}/{rows} robust rows compared")
    assert kept >= rows // 2


WINDOW_CASES = [
    # (V, history stride, repeat_window, id range): ragged histories, ids
    # outside [0, V) mixed in, windows shorter than, equal to and (0) all of
    # the history, heavy duplicates from a small id range
    (100, 40, 16, 100),
    (4096, 300, 64, 60),
    (4096, 300, 0, 4096),
    (32000, 4096, 0, 700),        # whole history at the 4096-entry limit
    (32000, 5000, 4096, 32000),   # window at the limit inside a longer history
    (50000, 200, 32, 50000),      # memory-read path (past the LDS row)
]


@pytest.mark.parametrize("V,S_,W,idr", WINDOW_CASES)
def test_sample_async_equals_host_windows(gpu, handle, V, S_, W, idr):
    """rlx_sample_async counts each row's window on the device from a device
    token history; with the same windows and draws it picks the same tokens
    as rlx_sample, whose windows the host counts."""
    rng = np.random.default_rng(V + S_ + W)
    rows = 24
    p = S.SamplerParams(temperature=0.9, top_k=40, top_p=0.95, repeat_penalty=1.4,
                        frequency_penalty=0.3, presence_penalty=0.5, repeat_window=W)
    x = rng.normal(0, 2.5, (rows, V)).astype(np.float32)
    # make the penalised ids matter: raise the logits of the window ids
    hist = rng.integers(0, idr, (rows, S_)).astype(np.int32)
    hist[:, ::7] = -1
    hist[:, 3::11] = V + 3
    lens = rng.integers(0, S_ + 1, rows).astype(np.int32)
    lens[0], lens[1] = 0, S_
    for b in range(rows):
        x[b, hist[b, :lens[b]][(hist[b, :lens[b]] >= 0) & (hist[b, :lens[b]] < V)]] += 3.0
    u = rng.random(rows, dtype=np.float32)
    smp = make_sampler(p, S.Draws(u))
    want = smp.Sample(dev(x, gpu), [list(hist[b, :lens[b]]) for b in range(rows)], handle)
    xd = dev(x, gpu)
    got = smp.SampleAsync(xd, torch.from_numpy(hist).to(gpu), torch.from_numpy(lens).to(gpu),
                          torch.from_numpy(u).to(gpu), handle)
    assert got.cpu().tolist() == list(want)
    # a strided history (rows of a wider buffer) and an out tensor given
    wide = torch.zeros(rows, S_ + 9, dtype=torch.int32, device=gpu)
    wide[:, :S_] = torch.from_numpy(hist).to(gpu)
    out = torch.full((rows,), -7, dtype=torch.int32, device=gpu)
    if W == 0 and S_ + 9 > 4096:
        return
    smp.SampleAsync(xd, wide[:, :S_], torch.from_numpy(lens).to(gpu), torch.from_numpy(u).to(gpu),
                    handle, out=out)
    assert out.cpu().tolist() == list(want)


def test_sample_async_no_history_and_limits(gpu, handle):
    from relux_amd import ReluxError
    rng = np.random.default_rng(5)
    V, rows = 1000, 8
    x = dev(rng.normal(0, 2, (rows, V)), gpu)
    u = rng.random(rows, dtype=np.float32)
    p = S.SamplerParams(top_k=20, repeat_penalty=1.3, repeat_window=0)
    smp = make_sampler(p, S.Draws(u))
    want = smp.Sample(x, None, handle)
    got = smp.SampleAsync(x, None, None, torch.from_numpy(u).to(gpu), handle)
    assert got.cpu().tolist() == list(want)
    lens = torch.zeros(rows, dtype=torch.int32, device=gpu)
    ud = torch.from_numpy(u).to(gpu)
    # longest possible window past 4096 entries: refused before any launch
    with pytest.raises(ReluxError):
        smp.SampleAsync(x, torch.zeros(rows, 4097, dtype=torch.int32, device=gpu), lens, ud, handle)
    smp4097 = make_sampler(S.SamplerParams(repeat_penalty=1.3, repeat_window=4097), S.Draws(u))
    with pytest.raises(ReluxError):
        smp4097.SampleAsync(x, torch.zeros(rows, 5000, dtype=torch.int32, device=gpu), lens, ud, handle)
    # host tensors are refused, not passed to the kernel
    with pytest.raises(TypeError):
        smp.SampleAsync(x, None, None, torch.from_numpy(u), handle)


# V 32000 and 50000: the next-row Sample of all-accepted rows runs split
# (top-k 30); every V reduces its softmax statistics over 4096-entry chunks;
# V 32003 leaves every row but the first off 16-byte alignment.
@pytest.mark.parametrize("V", [100, 4096, 32000, 50000, 32003])
def test_spec_accept(gpu, handle, V):
    from relux_amd import spec_accept
    rng = np.random.default_rng(V)
    B, K = 16, 4
    d = rng.normal(0, 1.5, (B, K, V)).astype(np.float32)
    t = np.concatenate([d + rng.normal(0, 0.7, (B, K, V)).astype(np.float32),
                        rng.normal(0, 1.5, (B, 1, V)).astype(np.float32)], axis=1)
    nd = np.array([K] * 10 + [2, 3, 1, 0, K, K], np.int32)
    tok = np.zeros((B, K), np.int32)
    for b in range(B):  # drafts drawn from the draft distribution
        for i in range(K):
            tok[b, i] = S.sample(d[b, i], S.SamplerParams(), float(rng.random()))
    u = rng.random((B, K + 1), dtype=np.float32)
    params = S.SamplerParams(temperature=0.9, top_k=30)
    acc, nxt = spec_accept(handle, dev(d, gpu), dev(t, gpu), tok, nd, u, make_sampler(params))
    kept = 0
    outcomes = set()
    for b in range(B):
        k = nd[b]
        want = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1], params)
        lo = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1] - DELTA, params)
        hi = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1] + DELTA, params)
        if lo != want or hi != want:
            continue
        kept += 1
        outcomes.add(want[0] == k)
        assert (acc[b], nxt[b]) == want, (V, b, acc[b], nxt[b], want)
    print(f"spec_accept V{V}: {kept}/{B} robust rows compared")
    assert kept >= B // 2
    assert outcomes == {True, False}  # both the rejection and the all-accepted paths ran


@pytest.mark.parametrize("K,V", [(1, 32000), (8, 32000), (8, 4096)])
def test_spec_accept_draft_counts(gpu, handle, K, V):
    """One and eight drafts per row (the statistics launch holds 2K row
    sides per row), counts from 0 to K."""
    from relux_amd import spec_accept
    rng = np.random.default_rng(1000 * K + V)
    B = 12
    d = rng.normal(0, 1.5, (B, K, V)).astype(np.float32)
    t = np.concatenate([d + rng.normal(0, 0.6, (B, K, V)).astype(np.float32),
                        rng.normal(0, 1.5, (B, 1, V)).astype(np.float32)], axis=1)
    nd = rng.integers(0, K + 1, B).astype(np.int32)
    nd[:4] = K
    tok = np.zeros((B, K), np.int32)
    for b in range(B):
        for i in range(K):
            tok[b, i] = S.sample(d[b, i], S.SamplerParams(), float(rng.random()))
    u = rng.random((B, K + 1), dtype=np.float32)
    params = S.SamplerParams(temperature=0.8, top_k=40, top_p=0.9)
    acc, nxt = spec_accept(handle, dev(d, gpu), dev(t, gpu), tok, nd, u, make_sampler(params))
    kept = 0
    for b in range(B):
        k = nd[b]
        want = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1], params)
        lo = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1] - DELTA, params)
        hi = S.spec_accept(d[b, :k], t[b, :k + 1], tok[b, :k], u[b, :k + 1] + DELTA, params)
        if lo != want or hi != want:
            continue
        kept += 1
        assert (acc[b], nxt[b]) == want, (K, V, b, acc[b], nxt[b], want)
    print(f"spec_accept K{K} V{V}: {kept}/{B} robust rows compared")
    assert kept >= B // 2


@pytest.mark.parametrize("V", [4096, 50000])
def test_spec_accept_async_equals_sync(gpu, handle, V):
    """rlx_spec_accept_async (draft ids, counts and draws on the device)
    gives rlx_spec_accept's results on valid inputs; a count past max_k is
    clamped and an id outside [0, V) is a rejection at its position."""
    from relux_amd import spec_accept, spec_accept_async
    rng = np.random.default_rng(V + 3)
    B, K = 12, 4
    d = rng.normal(0, 1.5, (B, K, V)).astype(np.float32)
    t = np.concatenate([d + rng.normal(0, 0.7, (B, K, V)).astype(np.float32),
                        rng.normal(0, 1.5, (B, 1, V)).astype(np.float32)], axis=1)
    nd = np.array([K, K, 3, 2, 1, 0, K, K, K, 2, K, K], np.int32)
    tok = rng.integers(0, V, (B, K)).astype(np.int32)
    for b in range(B):  # mostly draws from the draft rows, so both outcomes occur
        for i in range(K):
            tok[b, i] = S.sample(d[b, i], S.SamplerParams(), float(rng.random()))
    u = rng.random((B, K + 1), dtype=np.float32)
    params = S.SamplerParams(temperature=0.9, top_k=30)
    smp = make_sampler(params)
    acc, nxt = spec_accept(handle, dev(d, gpu), dev(t, gpu), tok, nd, u, smp)
    it = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    acc_d, nxt_d = spec_accept_async(handle, dev(d, gpu), dev(t, gpu), it(tok), it(nd), dev(u, gpu), smp)
    assert acc_d.cpu().tolist() == list(acc) and nxt_d.cpu().tolist() == list(nxt)
    # counts past max_k are clamped; ids outside [0, V) are rejections there
    nd2 = nd.copy()
    nd2[0] = K + 5
    nd2[1] = -3
    tok2 = tok.copy()
    tok2[6, 0] = V
    tok2[7, 2] = -1
    u2 = u.copy()
    u2[7, :2] = 0.0  # the first two drafts of row 7 are accepted
    acc2, nxt2 = spec_accept_async(handle, dev(d, gpu), dev(t, gpu), it(tok2), it(nd2), dev(u2, gpu), smp)
    acc2, nxt2 = acc2.cpu().tolist(), nxt2.cpu().tolist()
    ref_acc, ref_nxt = spec_accept(handle, dev(d, gpu), dev(t, gpu), tok, np.clip(nd2, 0, K), u2, smp)
    for b in range(B):
        if b in (6, 7):
            continue
        assert (acc2[b], nxt2[b]) == (ref_acc[b], ref_nxt[b]), b
    assert acc2[6] == 0 and 0 <= nxt2[6] < V
    assert acc2[7] == 2 and 0 <= nxt2[7] < V


def test_spec_accept_rejects_bad_tokens(gpu, handle):
    from relux_amd import ReluxError, spec_accept
    d = torch.zeros(1, 2, 10, device=gpu)
    t = torch.zeros(1, 3, 10, device=gpu)
    with pytest.raises(ReluxError):
        spec_accept(handle, d, t, [[1, 10]], [2], np.full(3, 0.5), make_sampler(S.SamplerParams()))
    with pytest.raises(ReluxError):
        spec_accept(handle, d, t, [[1, 2]], [3], np.full(3, 0.5), make_sampler(S.SamplerParams()))


# ---- speculative decoding end to end on the GPU caches -----------------------

class GpuLM:
    """A config-1 decoder (CPU math for the non-attention modules, as in
    test_gpu_tiny_decoder) whose attention cache is the paged GPU cache;
    records every forward / rollback with the logits it returned."""

    def __init__(self, model, gpu):
        from relux_amd import KVCache
        self.m, self.gpu = model, gpu
        cfg = model.cfg
        self.cache = KVCache(num_layers=cfg["layers"], max_len=cfg["max_seq"], num_kv_heads=cfg["kv_heads"],
                             head_dim=cfg["d_model"] // cfg["heads"], page_tokens=16, device=gpu.index)
        self.H = cfg["heads"]
        self.calls = []

    # the three cache calls TinyDecoder makes
    def total_len(self, layer):
        return self.cache.TotalLen(layer)

    def append(self, layer, k, v):
        self.cache.Append(layer, torch.from_numpy(k).to(self.gpu), torch.from_numpy(v).to(self.gpu), layout="HSD")

    def attend(self, layer, q):
        S_ = q.shape[1]
        out = self.cache.Attend(layer, torch.from_numpy(np.ascontiguousarray(q)).to(self.gpu),
                                num_heads=self.H, n_q=[S_], layout="HSD", mask="causal")
        return out.cpu().numpy()

    # the model interface SpeculativeDecoder drives
    def forward(self, ids):
        lg = self.m.forward(list(ids), self)
        self.calls.append(("f", list(ids), lg))
        return torch.from_numpy(lg).to(self.gpu)

    def rollback(self, n):
        self.calls.append(("r", n, None))
        if n:
            self.cache.Rollback(0, n)

    def reset(self):
        self.cache.Reset()


class ReplayLM:
    """Returns the logits a GpuLM produced, in call order, checking that the
    oracle loop makes the same calls."""

    def __init__(self, calls):
        self.calls = list(calls)

    def forward(self, ids):
        kind, want_ids, lg = self.calls.pop(0)
        assert kind == "f" and want_ids == list(ids), (kind, want_ids, ids)
        return lg

    def rollback(self, n):
        kind, want_n, _ = self.calls.pop(0)
        assert kind == "r" and want_n == n, (kind, want_n, n)


def test_speculative_same_model_is_greedy(gpu):
    from relux_amd import Draws, Sampler, SpeculativeDecoder
    m = td.TinyDecoder(td.CFG1, seed=0, rope_rule="offset")
    prompt = td.prompt_ids(td.CFG1)
    lm = GpuLM(m, gpu)
    want, _, _ = m.generate(prompt, 12, lm)
    sd = SpeculativeDecoder(GpuLM(m, gpu), GpuLM(m, gpu), 4, Sampler(temperature=0.0, rand=Draws(seed=1)))
    gen, rate = sd.Generate(prompt, 12)
    assert gen == want[len(prompt):] and rate == 1.0


def test_speculative_decoder_replays_on_oracle(gpu):
    from relux_amd import Draws, SpeculativeDecoder
    target = GpuLM(td.TinyDecoder(td.CFG1, seed=0, rope_rule="offset"), gpu)
    draft = GpuLM(td.TinyDecoder(td.CFG1, seed=1, rope_rule="offset"), gpu)
    prompt = td.prompt_ids(td.CFG1)
    draws = np.random.default_rng(5).random(600, dtype=np.float32)
    params = S.SamplerParams(temperature=0.9, top_k=40, repeat_penalty=1.1, repeat_window=8)
    sd = SpeculativeDecoder(draft, target, 3, make_sampler(params, Draws(values=draws)))
    gen, rate = sd.Generate(prompt, 20)
    assert len(gen) == 20
    # 1. Decisions: the oracle loop over the same logits and draws makes the
    #    same calls (ids, rollback counts) and commits the same tokens.
    og, orate = S.speculative_generate(ReplayLM(draft.calls), ReplayLM(target.calls), prompt, 20, 3,
                                       params, S.Draws(draws))
    assert og == gen and orate == rate
    rolled = [c[1] for c in target.calls if c[0] == "r"]
    print(f"acceptance {rate:.2f}; target rollbacks {rolled}")
    assert any(rolled)  # some drafts were rejected and rolled back
    # 2. Cache semantics: the oracle model on a logical cache, driven by the
    #    same call sequence, gives the same logits at every call.
    for lm in (draft, target):
        logical = td.LogicalCache(td.CFG1)
        for kind, arg, lg in lm.calls:
            if kind == "r":
                for layer in range(td.CFG1["layers"]):
                    logical.rollback(layer, arg)
                continue
            want = lm.m.forward(arg, logical)
            d = np.abs(lg - want)
            assert d.max() < 2e-2 and d.mean() < 2e-3, (d.max(), d.mean())
        # 3. The paged cache holds exactly the committed prefix: layer 0 K/V
        #    (position-only inputs) bit-exact against the logical cache.
        T = logical.total_len(0)
        assert lm.cache.TotalLen(0) == T
        k_dev, v_dev = lm.cache.View(0)
        np.testing.assert_array_equal(k_dev.cpu().float().numpy()[0], logical.k[0])
        np.testing.assert_array_equal(v_dev.cpu().float().numpy()[0], logical.v[0])
