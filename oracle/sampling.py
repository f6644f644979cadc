"""Token selection of the reference, restated -- TEST INFRASTRUCTURE ONLY.

Front end of oracle/sampling.c (Sampler.Greedy / Sampler.Sample,
sampler.go:56-210; SpeculativeDecoder.acceptPhase / resampleRejected,
speculative.go:203-290) plus the speculative generation loop with the
corrected cache semantics the device build implements (the reference feeds
the last committed token twice and never rolls its caches back,
speculative.go:124-157, 171-198; see speculative_generate).

Each rng.Float32() draw of the reference is an argument here, so the device
path can be checked on the same numbers.
"""
import ctypes

import numpy as np

from . import lib


class SamplerParams:
    """Sampler (sampler.go:33-43) without Rand; the defaults of NewSampler."""

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=0.0,
                 frequency_penalty=0.0, presence_penalty=0.0, repeat_window=0):
        self.temperature, self.top_k, self.top_p, self.min_p = temperature, top_k, top_p, min_p
        self.repeat_penalty, self.frequency_penalty = repeat_penalty, frequency_penalty
        self.presence_penalty, self.repeat_window = presence_penalty, repeat_window

    def f(self):
        return np.array([self.temperature, self.top_p, self.min_p, self.repeat_penalty,
                         self.frequency_penalty, self.presence_penalty], np.float32)

    def i(self):
        return np.array([self.top_k, self.repeat_window], np.int32)


def greedy(logits):
    x = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_greedy(x, x.size))


def sample(logits, params, r, prev=None, want_probs=False):
    """Sampler.Sample(logits, prev) with the draw r; optionally the final
    distribution the draw is taken from."""
    x = np.ascontiguousarray(logits, np.float32)
    pv = None if prev is None or len(prev) == 0 else np.ascontiguousarray(prev, np.int32)
    probs = np.empty(x.size, np.float32) if want_probs else None
    t = lib().orc_sample(x, x.size, params.f(), params.i(),
                         None if pv is None else pv.ctypes.data, 0 if pv is None else pv.size,
                         float(r), None if probs is None else probs.ctypes.data)
    return (int(t), probs) if want_probs else int(t)


def spec_accept(d_logits, t_logits, d_tok, u, params):
    """acceptPhase over k drafts: d_logits [k, V], t_logits [k+1, V], draws
    u [k+1] in draw order.  Returns (accepted, next token)."""
    d = np.ascontiguousarray(d_logits, np.float32)
    t = np.ascontiguousarray(t_logits, np.float32)
    k, V = d.shape
    assert t.shape == (k + 1, V)
    nxt = ctypes.c_int(0)
    n = lib().orc_spec_accept(d.reshape(-1), t.reshape(-1), np.ascontiguousarray(d_tok, np.int32),
                              k, V, np.ascontiguousarray(u, np.float32), params.f(), params.i(),
                              ctypes.byref(nxt))
    return int(n), int(nxt.value)


class Draws:
    """The reference's single rng stream as a list of f32 draws: take(n)
    consumes n, peek(n) looks ahead without consuming."""

    def __init__(self, values):
        self.v = np.asarray(values, np.float32)
        self.i = 0

    def peek(self, n):
        assert self.i + n <= self.v.size, "draw stream exhausted"
        return self.v[self.i:self.i + n]

    def take(self, n):
        out = self.peek(n)
        self.i += n
        return out


def spec_draws_used(n_acc, k):
    """Draws acceptPhase consumes: one test per draft up to the first
    rejection, then one for the resample or the final Sample."""
    return n_acc + 2 if n_acc < k else k + 1


def speculative_generate(draft, target, prompt, max_new, K, params, draws):
    """Speculative decoding with caches that hold exactly the committed
    tokens but the last (the pending one).

    draft / target: objects with forward(ids) -> logits [len(ids), V] (f32)
    that append to their own cache, and rollback(n) that drops the newest n
    cached tokens.  draws: a Draws stream (the one rng the reference shares
    between Sample and acceptPhase).  Per round (speculative.go:124-157,
    corrected):
      draft: feed the pending suffix, sample k drafts one at a time
        (Sample(logits, prev) with prev = committed + drafts so far);
      target: verify [pending] + drafts in one call (k+1 causal rows);
      accept (acceptPhase); commit the accepted drafts and the new token;
      roll both caches back to the committed prefix.
    Returns (generated tokens, acceptance rate)."""
    gen = []
    seq = list(prompt)
    if len(seq) > 1:
        draft.forward(seq[:-1])
        target.forward(seq[:-1])
    d_pending = [seq[-1]]  # committed tokens not yet in the draft cache
    drafted = accepted = 0
    while len(gen) < max_new:
        k = min(K, max_new - len(gen))
        d_tok, d_rows = [], []
        feed = d_pending
        for _ in range(k):
            lg = draft.forward(feed)[-1]
            d_rows.append(lg)
            t = sample(lg, params, draws.take(1)[0], prev=seq + d_tok)
            d_tok.append(t)
            feed = [t]
        t_rows = target.forward([seq[-1]] + d_tok)
        n_acc, nxt = spec_accept(np.stack(d_rows), t_rows, d_tok, draws.peek(k + 1), params)
        draws.take(spec_draws_used(n_acc, k))
        # Target cache: +k+1 (pending + drafts); keep pending + accepted.
        target.rollback(k - n_acc)
        # Draft cache: +len(d_pending) + k - 1 (the last draft was never
        # fed); keep the committed prefix up to the accepted drafts.
        if n_acc < k:
            draft.rollback(k - 1 - n_acc)
            d_pending = [nxt]
        else:
            d_pending = [d_tok[-1], nxt]
        seq += d_tok[:n_acc] + [nxt]
        gen += d_tok[:n_acc] + [nxt]
        drafted += k
        accepted += n_acc
    return gen[:max_new], (accepted / drafted if drafted else 0.0)
