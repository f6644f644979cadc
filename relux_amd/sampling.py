"""Token selection and speculative decoding over the device caches.

Mirrors of the reference's Sampler (internal/transformer/sampler.go:33-301)
and SpeculativeDecoder (speculative.go:47-375).  Greedy, Sample and the
speculative acceptance test run on the device (rlx_greedy, rlx_sample,
rlx_spec_accept) on logits that stay in device memory; only token ids come
back.  Random draws: the reference draws rng.Float32() inside Sample and
acceptPhase from one shared *rand.Rand; here the draws come from a Draws
stream the caller owns (a seeded generator, or a fixed list), passed to
the device in the reference's order.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import SamplerParams, check


class Draws:
    """One stream of f32 draws in [0, 1): take(n) consumes, peek(n) looks
    ahead.  Backed by a numpy Generator (seed) or a fixed list (values)."""

    def __init__(self, seed=None, values=None):
        self._gen = None if values is not None else np.random.default_rng(seed)
        self._buf = np.asarray(values if values is not None else [], np.float32)
        self._i = 0

    def peek(self, n):
        while self._i + n > self._buf.size:
            if self._gen is None:
                raise IndexError("draw stream exhausted")
            more = self._gen.random(max(n, 256), dtype=np.float32)
            self._buf = np.concatenate([self._buf[self._i:], more])
            self._i = 0
        return self._buf[self._i:self._i + n]

    def take(self, n):
        out = self.peek(n).copy()
        self._i += n
        return out


class Sampler:
    """transformer.Sampler: penalties -> temperature -> top-k -> top-p ->
    min-p -> draw (sampler.go:33-43; NewSampler defaults)."""

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=0.0,
                 frequency_penalty=0.0, presence_penalty=0.0, repeat_window=0, rand=None):
        self.Temperature, self.TopK, self.TopP, self.MinP = temperature, top_k, top_p, min_p
        self.RepeatPenalty, self.FrequencyPenalty = repeat_penalty, frequency_penalty
        self.PresencePenalty, self.RepeatWindow = presence_penalty, repeat_window
        self.Rand = rand if rand is not None else Draws()

    def params(self):
        return SamplerParams(self.Temperature, self.TopK, self.TopP, self.MinP, self.RepeatPenalty,
                             self.FrequencyPenalty, self.PresencePenalty, self.RepeatWindow)

    @staticmethod
    def _rows(logits):
        if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32):
            raise TypeError("logits must be a float32 device tensor")
        x = logits if logits.dim() == 2 else logits.reshape(1, -1)
        if x.stride(1) != 1:
            x = x.contiguous()
        return x

    def Greedy(self, logits, cache):
        """sampler.go:56-68 per row; one int for a 1-D row, else a list."""
        x = self._rows(logits)
        out = (ctypes.c_int32 * x.shape[0])()
        check(_lib.load().rlx_greedy(cache._h, x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), out))
        return out[0] if logits.dim() == 1 else list(out)

    def Sample(self, logits, previous_tokens, cache, draws=None):
        """sampler.go:73-210 per row.  previous_tokens: a list of ids (1-D
        logits) or a list of lists (one per row), or None."""
        x = self._rows(logits)
        n = x.shape[0]
        prev = previous_tokens
        if prev is not None and logits.dim() == 1:
            prev = [prev]
        off = tok = None
        if prev is not None:
            offs = np.zeros(n + 1, np.int32)
            for i, p in enumerate(prev):
                offs[i + 1] = offs[i] + len(p)
            flat = np.concatenate([np.asarray(p, np.int32) for p in prev]) if offs[-1] else np.zeros(1, np.int32)
            off = offs.ctypes.data_as(_lib._pi32)
            tok = flat.ctypes.data_as(_lib._pi32)
        u = (draws or self.Rand).take(n).astype(np.float32)
        out = (ctypes.c_int32 * n)()
        p = self.params()
        check(_lib.load().rlx_sample(cache._h, x.data_ptr(), n, x.shape[1], x.stride(0), ctypes.byref(p),
                                     tok, off, u.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out))
        return out[0] if logits.dim() == 1 else list(out)


    def SampleAsync(self, logits, history, hist_len, uniforms, cache, out=None):
        """Sample over device state (rlx_sample_async): logits [n, V] f32,
        history [n, S] int32 (each row's previous tokens, hist_len[n] int32
        of them; None: no penalties), uniforms [n] f32 draws, all device
        tensors.  Returns (or fills) out [n] int32 on the device; enqueued on
        the cache's stream without waiting."""
        x = self._rows(logits)
        n, V = x.shape[0], x.shape[1]
        if out is None:
            out = torch.empty(n, dtype=torch.int32, device=x.device)
        if out.dtype != torch.int32 or out.numel() != n or not out.is_contiguous():
            raise ValueError("out must be a contiguous int32 tensor of one entry per row")
        if uniforms.dtype != torch.float32 or uniforms.numel() != n or not uniforms.is_contiguous():
            raise ValueError("uniforms must be a contiguous f32 tensor of one draw per row")
        for name, t in (("out", out), ("uniforms", uniforms), ("history", history), ("hist_len", hist_len)):
            if t is not None and (not t.is_cuda or t.device != x.device):
                raise TypeError(f"{name} must be a tensor on the logits' device")
        hp = hl = None
        stride = 0
        if history is not None:
            if history.dtype != torch.int32 or history.dim() != 2 or history.shape[0] != n or \
                    history.stride(1) != 1:
                raise ValueError("history must be int32 [n_rows, S] with unit stride along S")
            if hist_len.dtype != torch.int32 or hist_len.numel() != n or not hist_len.is_contiguous():
                raise ValueError("hist_len must be a contiguous int32 tensor of one length per row")
            hp, hl, stride = history.data_ptr(), hist_len.data_ptr(), history.stride(0)
        p = self.params()
        check(_lib.load().rlx_sample_async(cache._h, x.data_ptr(), n, V, x.stride(0), ctypes.byref(p),
                                           hp, stride, hl, uniforms.data_ptr(), out.data_ptr()))
        return out


def spec_accept(cache, draft_logits, target_logits, draft_tokens, n_draft, uniforms, sampler):
    """Batched acceptPhase (speculative.go:203-290) on the device.
    draft_logits [B, K, V], target_logits [B, K+1, V] (f32 device tensors),
    draft_tokens [B, K] and n_draft [B] (host ints), uniforms [B, K+1].
    Returns (accepted per row, next token per row)."""
    B, Kp1, V = target_logits.shape
    K = Kp1 - 1
    d = draft_logits.contiguous() if K > 0 else target_logits
    t = target_logits.contiguous()
    dt = np.ascontiguousarray(np.asarray(draft_tokens, np.int32).reshape(B, K))
    nd = np.ascontiguousarray(np.asarray(n_draft, np.int32).reshape(B))
    u = np.ascontiguousarray(np.asarray(uniforms, np.float32).reshape(B, K + 1))
    acc = (ctypes.c_int32 * B)()
    nxt = (ctypes.c_int32 * B)()
    p = sampler.params()
    check(_lib.load().rlx_spec_accept(cache._h, d.data_ptr(), t.data_ptr(), dt.ctypes.data_as(_lib._pi32),
                                      nd.ctypes.data_as(_lib._pi32), B, K, V,
                                      u.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), ctypes.byref(p),
                                      acc, nxt))
    return list(acc), list(nxt)



def spec_accept_async(cache, draft_logits, target_logits, draft_tokens, n_draft, uniforms, sampler,
                      n_acc=None, next_tok=None):
    """Batched acceptPhase on device state (rlx_spec_accept_async):
    draft_logits [B, K, V], target_logits [B, K+1, V] f32, draft_tokens
    [B, K] int32, n_draft [B] int32, uniforms [B, K+1] f32 -- all tensors
    on the device.  Returns (or fills) (n_acc [B], next [B]) int32 device
    tensors; enqueued on the cache's stream without waiting."""
    B, Kp1, V = target_logits.shape
    K = Kp1 - 1
    dev = target_logits.device
    d = draft_logits.contiguous() if K > 0 else target_logits
    t = target_logits.contiguous()
    if n_acc is None:
        n_acc = torch.empty(B, dtype=torch.int32, device=dev)
    if next_tok is None:
        next_tok = torch.empty(B, dtype=torch.int32, device=dev)
    checks = (("draft_tokens", draft_tokens, torch.int32, B * K), ("n_draft", n_draft, torch.int32, B),
              ("uniforms", uniforms, torch.float32, B * (K + 1)), ("n_acc", n_acc, torch.int32, B),
              ("next_tok", next_tok, torch.int32, B))
    for name, x, dt, n in checks:
        if not isinstance(x, torch.Tensor) or x.device != dev or x.dtype != dt or x.numel() != n \
                or not x.is_contiguous():
            raise TypeError(f"{name} must be a contiguous {dt} tensor of {n} entries on the logits' device")
    if t.dtype != torch.float32 or d.dtype != torch.float32 or not t.is_cuda:
        raise TypeError("logits must be float32 device tensors")
    p = sampler.params()
    check(_lib.load().rlx_spec_accept_async(cache._h, d.data_ptr(), t.data_ptr(), draft_tokens.data_ptr(),
                                            n_draft.data_ptr(), B, K, V, uniforms.data_ptr(), ctypes.byref(p),
                                            n_acc.data_ptr(), next_tok.data_ptr()))
    return n_acc, next_tok

def spec_draws_used(n_acc, k):
    """Draws acceptPhase consumes: a test per draft up to the first
    rejection, then one for the resample or the final Sample."""
    return n_acc + 2 if n_acc < k else k + 1


class SpeculativeDecoder:
    """speculative.go:47-375 with the cache semantics corrected.

    draft / target: model objects with
      forward(ids) -> f32 device tensor [len(ids), vocab], appending to the
        model's own cache (a relux_amd cache, `model.cache`);
      rollback(n): drop the newest n tokens of that cache (rlx_rollback);
      reset(): empty the cache.
    The reference prefills both caches with the whole prompt and then feeds
    the last token again as the first draft / verify input, and it never
    truncates its caches (speculative.go:118-157, 171-198).  Here each cache
    holds exactly the committed tokens but the newest (the pending one), the
    verify call scores [pending] + drafts causally, and after acceptance both
    caches are rolled back to the committed prefix.  Draws follow the
    reference's order: one per draft sample, then acceptPhase's."""

    def __init__(self, draft, target, num_speculate=5, sampling=None):
        self.draft, self.target = draft, target
        self.K = num_speculate if num_speculate > 0 else 5
        self.sampling = sampling if sampling is not None else Sampler()

    def Generate(self, prompt, max_new):
        if not prompt:
            raise ValueError("speculative: empty prompt")
        d, t, smp = self.draft, self.target, self.sampling
        d.reset()
        t.reset()
        seq = list(prompt)
        if len(seq) > 1:
            d.forward(seq[:-1])
            t.forward(seq[:-1])
        pending = [seq[-1]]
        gen = []
        drafted = accepted = 0
        while len(gen) < max_new:
            k = min(self.K, max_new - len(gen))
            toks, rows = [], []
            feed = pending
            for _ in range(k):
                lg = d.forward(feed)[-1]
                rows.append(lg)
                nxt = smp.Sample(lg, seq + toks, d.cache)
                toks.append(nxt)
                feed = [nxt]
            t_rows = t.forward([seq[-1]] + toks)
            u = smp.Rand.peek(k + 1)
            acc, nx = spec_accept(t.cache, torch.stack(rows).unsqueeze(0), t_rows.unsqueeze(0),
                                  [toks], [k], u, smp)
            n_acc, nxt = acc[0], nx[0]
            smp.Rand.take(spec_draws_used(n_acc, k))
            t.rollback(k - n_acc)
            if n_acc < k:
                d.rollback(k - 1 - n_acc)
                pending = [nxt]
            else:
                pending = [toks[-1], nxt]
            seq += toks[:n_acc] + [nxt]
            gen += toks[:n_acc] + [nxt]
            drafted += k
            accepted += n_acc
        return gen[:max_new], (accepted / drafted if drafted else 0.0)
