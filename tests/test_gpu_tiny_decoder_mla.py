"""TestTransformer_MLA's decoder (transformer_test.go:1012-1027: d_model 32,
4 heads of 8 dims, d_c 32, d_r 4, 2 layers) generating greedily with its
latent cache on the GPU.

The projections, norms, MLP and head are the CPU restatement (outside the
device path); every latent Append and every absorbed attention call goes
through the HIP library.  Checked:
  * cache bytes: each layer's paged rows, gathered, equal BF16FromF32 of
    the c^KV / k^R rows the model appended (bit-exact);
  * logits: every step within max-abs 2e-2 / mean-abs 2e-3 of the oracle
    model (MLA.forwardCached restated, corrected semantics, bf16 rows) run
    over the same tokens;
  * tokens: each greedy token is the oracle's argmax unless the oracle's
    own top-2 gap at that step is within the observed logit difference.
A 12-token prompt puts 48 query rows (4 heads x 12) in the prefill call,
which the library cuts into causal query chunks.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import tiny_decoder as td

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3


class GpuMLACache:
    """The three latent-cache calls the MLA decoder makes, on the paged GPU
    cache (absorbed attention: q_lat = W_UK^T q_c, o = W_UV^T o_lat)."""

    def __init__(self, cfg, device):
        from relux_amd import MLACache
        self.H = cfg["heads"]
        self.D, dC, dR = td.mla_dims(cfg)
        self.c = MLACache(num_layers=cfg["layers"], max_len=cfg["max_seq"], d_c=dC, d_r=dR,
                          page_tokens=16, device=device.index)
        self.device = device
        self.appended = [[] for _ in range(cfg["layers"])]

    def total_len(self, layer):
        return self.c.TotalLen(layer)

    def append(self, layer, c, kr):
        self.appended[layer].append((c.copy(), kr.copy()))
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(self.device)
        self.c.Append(layer, t(c), t(kr))

    def attend(self, layer, qc, qr, w_uk, w_uv):
        S = qc.shape[1]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(self.device)
        w = lambda a: t(a.view(np.int16)).view(torch.bfloat16)
        out = self.c.Attend(layer, t(qc.transpose(1, 0, 2)), t(qr.transpose(1, 0, 2)), w(w_uk),
                            w(w_uv), self.H, self.D, n_q=[S], mask="causal")
        return out.cpu().numpy().transpose(1, 0, 2)  # [H, S, D]


@pytest.fixture(scope="module", params=[8, 12], ids=["prompt8", "prompt12"])
def run(request, gpu):
    m = td.MLATinyDecoder(td.CFG_MLA, seed=0)
    prompt = td.prompt_ids(m.cfg, n=request.param)
    new = m.cfg["max_seq"] - request.param - 4
    cache = GpuMLACache(m.cfg, gpu)
    toks, logits, _ = m.generate(prompt, new, cache)
    logical = td.MLALogicalCache(m.cfg)
    want = [m.forward(prompt, logical)[-1]]
    for t in toks[len(prompt):-1]:
        want.append(m.forward([t], logical)[-1])
    yield m, prompt, toks, logits, np.stack(want), cache
    cache.c.close()


def test_mla_decoder_logits_and_tokens(run):
    m, prompt, toks, logits, want, _ = run
    new = len(toks) - len(prompt)
    d = np.abs(logits - want)
    print(f"mla decoder logits max {d.max():.3e} mean {d.mean():.3e}")
    assert d.max() < TOL_MAX and d.mean() < TOL_MEAN
    for i in range(new):
        top2 = np.sort(want[i])[-2:]
        if top2[1] - top2[0] > 2 * d[i].max():
            assert toks[len(prompt) + i] == int(np.argmax(want[i])), i


def test_mla_decoder_cache_bytes(run):
    m, prompt, toks, logits, want, cache = run
    for layer in range(m.cfg["layers"]):
        ins = cache.appended[layer]
        c_log = np.concatenate([c for c, _ in ins])
        kr_log = np.concatenate([k for _, k in ins])
        assert c_log.shape[0] == len(toks) - 1 == cache.total_len(layer)
        gc, gk = cache.c.View(layer)
        np.testing.assert_array_equal(gc[0].view(torch.int16).cpu().numpy().view(np.uint16),
                                      oracle.bf16_from_f32(c_log))
        np.testing.assert_array_equal(gk[0].view(torch.int16).cpu().numpy().view(np.uint16),
                                      oracle.bf16_from_f32(kr_log))
