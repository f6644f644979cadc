"""The oracle's restatement of the reference's token selection
(oracle/sampling.c, oracle/sampling.py), pinned without the Go build:

* the reference's own sampler_test.go cases;
* for every stage, the distribution the draw is taken from, computed here
  independently in f64 from the stage's definition (softmax of fastexp32
  weights, the k largest logits, the smallest top-probability prefix
  reaching p, the min-p floor, hand-applied penalties), against the
  frequencies of a sweep of r over [0, 1) -- a dropped stage, a wrong
  comparison or a mis-indexed token moves the frequencies;
* acceptPhase: the accepted fraction over a sweep of the test draw equals
  min(1, p_t/p_d) and the resample frequencies equal norm(max(0, p_t-p_d));
* the speculative loop: with draft == target and temperature 0 it
  reproduces greedy generation with every draft accepted, and whatever the
  draft, the target cache ends holding exactly the committed tokens.
"""
import numpy as np
import pytest

import oracle
from oracle import sampling as S
from oracle import tiny_decoder as td

N_SWEEP = 20000


def fe_probs(x):
    """f64 softmax of fastexp32 weights (fastexp32 itself is pinned in
    test_oracle.py), -inf entries weight 0."""
    x = np.asarray(x, np.float32)
    m = np.max(x)
    w = np.where(np.isneginf(x), 0.0, oracle.fastexp32(np.where(np.isneginf(x), 0, x - m)).astype(np.float64))
    return w / w.sum()


def sweep(logits, params, prev=None):
    r = (np.arange(N_SWEEP) + 0.5) / N_SWEEP
    toks = np.array([S.sample(logits, params, float(ri), prev=prev) for ri in r])
    return np.bincount(toks, minlength=len(logits)) / N_SWEEP


def renorm(p, keep):
    q = np.where(keep, p, 0.0)
    return q / q.sum()


# ---- sampler_test.go ------------------------------------------------------

def test_reference_greedy_cases():
    assert S.greedy([1, 5, 3, 2, 4]) == 1
    assert S.greedy([5, 5, 3]) == 0  # first argmax on ties


def test_reference_temperature_zero_is_argmax():
    p = S.SamplerParams(temperature=1e-10)
    assert all(S.sample([1, 5, 3], p, r) == 1 for r in np.linspace(0, 0.9999, 100))


def test_reference_top2():
    p = S.SamplerParams(top_k=2)
    got = {S.sample([1, 5, 3, 2, 4], p, r) for r in np.random.default_rng(42).random(100)}
    assert got <= {1, 4} and got == {1, 4}


def test_reference_distribution_sums_to_one():
    _, probs = S.sample([0.0, 0.0, 0.0, 0.0], S.SamplerParams(), 0.5, want_probs=True)
    assert abs(float(probs.sum()) - 1.0) < 1e-5


# ---- each stage against its stated distribution ----------------------------

@pytest.fixture(scope="module")
def logits():
    return np.random.default_rng(7).normal(0, 2, 40).astype(np.float32)


def test_plain_and_temperature(logits):
    for T in (1.0, 0.7, 2.5):
        want = fe_probs(logits / np.float32(T)) if T != 1.0 else fe_probs(logits)
        got = sweep(logits, S.SamplerParams(temperature=T))
        assert np.abs(got - want).max() < 3.0 / N_SWEEP, T


def test_top_k(logits):
    for k in (1, 3, 10):
        top = np.argsort(-logits)[:k]
        keep = np.zeros(len(logits), bool)
        keep[top] = True
        want = renorm(fe_probs(np.where(keep, logits, -np.inf)), keep)
        got = sweep(logits, S.SamplerParams(top_k=k))
        assert np.abs(got - want).max() < 3.0 / N_SWEEP, k
        assert set(np.nonzero(got)[0]) <= set(top)


def test_top_p(logits):
    p = fe_probs(logits)
    for top_p in (0.3, 0.75, 0.95):
        order = np.argsort(-p)
        cum = np.cumsum(p[order])
        cut = int(np.argmax(cum >= top_p)) + 1
        keep = np.zeros(len(p), bool)
        keep[order[:cut]] = True
        got = sweep(logits, S.SamplerParams(top_p=top_p))
        assert np.abs(got - renorm(p, keep)).max() < 3.0 / N_SWEEP, top_p


def test_min_p(logits):
    p = fe_probs(logits)
    for mp in (0.05, 0.3):
        keep = p >= p.max() * mp
        got = sweep(logits, S.SamplerParams(min_p=mp))
        assert np.abs(got - renorm(p, keep)).max() < 3.0 / N_SWEEP, mp


def test_penalties_by_hand():
    x = np.array([2.0, -1.0, 0.5, 3.0, -2.0, 1.0], np.float32)
    prev = [3, 1, 3, 5, 0, 3, 9]  # 9 is outside the vocabulary: ignored
    rp, fp, pp = 1.5, 0.25, 0.4
    want_x = x.copy()
    counts = {3: 3, 1: 1, 5: 1, 0: 1}
    for t, c in counts.items():
        v = want_x[t]
        v = v / np.float32(rp) if v > 0 else v * np.float32(rp)
        v = v - np.float32(fp) * np.float32(c)
        want_x[t] = v - np.float32(pp)
    params = S.SamplerParams(repeat_penalty=rp, frequency_penalty=fp, presence_penalty=pp)
    got = sweep(x, params, prev=prev)
    assert np.abs(got - fe_probs(want_x)).max() < 3.0 / N_SWEEP
    # A window of 2 sees only the last two tokens, 3 (once) and 9.
    w2 = x.copy()
    v = w2[3] / np.float32(rp)
    w2[3] = (v - np.float32(fp)) - np.float32(pp)
    params.repeat_window = 2
    got = sweep(x, params, prev=prev)
    assert np.abs(got - fe_probs(w2)).max() < 3.0 / N_SWEEP


# ---- acceptPhase -----------------------------------------------------------

def test_accept_rate_and_resample_distribution():
    rng = np.random.default_rng(3)
    V = 30
    d = rng.normal(0, 1, (1, V)).astype(np.float32)
    t = np.concatenate([d + rng.normal(0, 0.8, (1, V)).astype(np.float32),
                        rng.normal(0, 1, (1, V)).astype(np.float32)])
    pd, pt = fe_probs(d[0]), fe_probs(t[0])
    params = S.SamplerParams()
    for tok in range(V):
        a = min(1.0, pt[tok] / max(pd[tok], 1e-10))
        grid = (np.arange(2000) + 0.5) / 2000
        acc = np.mean([S.spec_accept(d, t, [tok], [u0, 0.5], params)[0] == 1 for u0 in grid])
        assert abs(acc - a) < 2e-3, tok
    tok = int(np.argmax(pd / pt))  # most over-proposed token: rejected often
    res = np.maximum(pt - pd, 0)
    res /= res.sum()
    grid = (np.arange(N_SWEEP) + 0.5) / N_SWEEP
    nxt = [S.spec_accept(d, t, [tok], [0.99999, r], params) for r in grid]
    assert all(n == 0 for n, _ in nxt)
    got = np.bincount([x for _, x in nxt], minlength=V) / N_SWEEP
    assert np.abs(got - res).max() < 3.0 / N_SWEEP


def test_all_accepted_samples_next_target_row():
    rng = np.random.default_rng(4)
    d = rng.normal(0, 1, (2, 20)).astype(np.float32)
    t = np.concatenate([d, rng.normal(0, 1, (1, 20)).astype(np.float32)])  # p_t == p_d: always accept
    params = S.SamplerParams(temperature=0.8, top_k=5)
    for r in np.linspace(0.01, 0.99, 25):
        n, nxt = S.spec_accept(d, t, [3, 7], [0.9999, 0.9999, r], params)
        assert n == 2 and nxt == S.sample(t[2], params, r)
    assert S.spec_draws_used(2, 2) == 3 and S.spec_draws_used(0, 4) == 2


# ---- the speculative loop ---------------------------------------------------

class OracleLM:
    def __init__(self, model):
        self.m = model
        self.cache = td.LogicalCache(model.cfg)

    def forward(self, ids):
        return self.m.forward(ids, self.cache)

    def rollback(self, n):
        for layer in range(self.m.cfg["layers"]):
            self.cache.rollback(layer, n)


def test_speculative_same_model_is_greedy():
    m = td.TinyDecoder(td.CFG1, seed=0, rope_rule="offset")
    prompt = td.prompt_ids(td.CFG1)
    want, _, _ = m.generate(prompt, 12, td.LogicalCache(m.cfg))
    gen, rate = S.speculative_generate(OracleLM(m), OracleLM(m), prompt, 12, 4,
                                       S.SamplerParams(temperature=0.0), S.Draws(np.full(200, 0.5)))
    assert gen == want[len(prompt):] and rate == 1.0


def test_speculative_caches_hold_committed_prefix():
    target = OracleLM(td.TinyDecoder(td.CFG1, seed=0, rope_rule="offset"))
    draft = OracleLM(td.TinyDecoder(td.CFG1, seed=1, rope_rule="offset"))
    prompt = td.prompt_ids(td.CFG1)
    draws = S.Draws(np.random.default_rng(5).random(400, dtype=np.float32))
    gen, rate = S.speculative_generate(draft, target, prompt, 14, 3, S.SamplerParams(temperature=0.9), draws)
    assert len(gen) == 14 and 0.0 <= rate <= 1.0
    # The last round may commit one token past max_new (the output is cut
    # to max_new as speculative.go:160 does): the cache then holds all of seq.
    seq = prompt + gen
    T = target.cache.total_len(0)
    assert T in (len(seq) - 1, len(seq))
    fresh = td.LogicalCache(td.CFG1)
    target.m.forward(seq[:T], fresh)
    for layer in range(td.CFG1["layers"]):
        assert target.cache.total_len(layer) == T
        np.testing.assert_array_equal(target.cache.k[0], fresh.k[0])
        np.testing.assert_allclose(target.cache.k[layer], fresh.k[layer], atol=1e-5)
        np.testing.assert_allclose(target.cache.v[layer], fresh.v[layer], atol=1e-5)
