"""Config 1 end to end: the README tiny GQA decoder (head_dim 16, 2 KV heads)
generating 16 tokens greedily with its attention cache on the GPU.

The non-attention modules are the CPU restatement (they are outside the
device path); every Append / attention call goes through the HIP library.
Checked:
  * cache bytes: each layer's paged cache, gathered, equals BF16FromF32 of
    the K/V rows the model appended (bit-exact), and the reference's own
    byte image rebuilt from it by the raw-copy rule equals the image the
    reference KVCache (oracle RefCache) holds after the same appends;
  * logits: every step within max-abs 2e-2 / mean-abs 2e-3 of the oracle
    model run over the same tokens with the corrected cache semantics;
  * tokens: each greedy token is the oracle's argmax unless the oracle's
    own top-2 gap at that step is within the observed logit difference.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import tiny_decoder as td

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3


class GpuCache:
    """The three cache calls the model makes, on the paged GPU cache."""

    def __init__(self, cfg, device):
        from relux_amd import KVCache
        self.cfg = cfg
        self.H = cfg["heads"]
        self.c = KVCache(num_layers=cfg["layers"], max_len=cfg["max_seq"],
                         num_kv_heads=cfg["kv_heads"], head_dim=cfg["d_model"] // cfg["heads"],
                         page_tokens=16, device=device.index)
        self.device = device
        self.appended = [[] for _ in range(cfg["layers"])]  # f32 [KVH,S,D] inputs

    def total_len(self, layer):
        return self.c.TotalLen(layer)

    def append(self, layer, k, v):
        self.appended[layer].append((k.copy(), v.copy()))
        self.c.Append(layer, torch.from_numpy(k).to(self.device), torch.from_numpy(v).to(self.device),
                      layout="HSD")

    def attend(self, layer, q):
        S = q.shape[1]
        out = self.c.Attend(layer, torch.from_numpy(np.ascontiguousarray(q)).to(self.device),
                            num_heads=self.H, n_q=[S], layout="HSD", mask="causal")
        return out.cpu().numpy()


@pytest.fixture(scope="module")
def run(gpu):
    m = td.TinyDecoder(td.CFG1, seed=0)
    prompt = td.prompt_ids(td.CFG1)
    cache = GpuCache(m.cfg, gpu)
    toks, logits, _ = m.generate(prompt, 16, cache)
    # Oracle over the SAME tokens (teacher forcing), corrected semantics.
    logical = td.LogicalCache(m.cfg)
    ref = td.RefCache(m.cfg)
    want = [m.forward(prompt, logical)[-1]]
    for t in toks[len(prompt):-1]:
        want.append(m.forward([t], logical)[-1])
    return m, prompt, toks, logits, np.stack(want), cache, logical, ref


def test_cfg1_logits_and_tokens(run):
    m, prompt, toks, logits, want, *_ = run
    assert len(toks) == len(prompt) + 16
    d = np.abs(logits - want)
    print(f"cfg1 logits max {d.max():.3e} mean {d.mean():.3e}")
    assert d.max() < TOL_MAX and d.mean() < TOL_MEAN
    for i in range(16):
        top2 = np.sort(want[i])[-2:]
        if top2[1] - top2[0] > 2 * d[i].max():
            assert toks[len(prompt) + i] == int(np.argmax(want[i])), i


def test_cfg1_cache_bytes(run):
    m, prompt, toks, logits, want, cache, *_ = run
    cfg = m.cfg
    cap = cfg["max_seq"]
    for layer in range(cfg["layers"]):
        ins = cache.appended[layer]
        chunks = [k.shape[1] for k, _ in ins]
        k_log = np.concatenate([k for k, _ in ins], axis=1)
        v_log = np.concatenate([v for _, v in ins], axis=1)
        assert sum(chunks) == len(toks) - 1 == cache.total_len(layer)
        gk, gv = cache.c.View(layer)
        gk = gk[0].view(torch.int16).cpu().numpy().view(np.uint16)
        gv = gv[0].view(torch.int16).cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(gk, oracle.bf16_from_f32(k_log))
        np.testing.assert_array_equal(gv, oracle.bf16_from_f32(v_log))
        # Reference byte image after the same Append calls.
        ref = td.RefCache(cfg)
        for k, v in ins:
            ref.append(layer, k, v)
        np.testing.assert_array_equal(td.ref_byte_image(gk, chunks, cap), ref.k[layer])
        np.testing.assert_array_equal(td.ref_byte_image(gv, chunks, cap), ref.v[layer])


def test_cfg1_layer0_bytes_match_fixture(run):
    """Layer-0 K/V depend only on the token and its position, so over the
    fixture's own tokens the GPU cache must reproduce the fixture bytes."""
    import os
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_tiny_decoder.npz"))
    m, prompt, toks, *_ = run
    ftoks = fx["tokens"].tolist()
    assert ftoks[:8] == prompt
    cache = GpuCache(m.cfg, torch.device("cuda", 0))
    m.forward(ftoks[:8], cache)
    for t in ftoks[8:-1]:
        m.forward([t], cache)
    gk, gv = cache.c.View(0)
    np.testing.assert_array_equal(gk[0].view(torch.int16).cpu().numpy().view(np.uint16),
                                  fx["kv_bytes"][0, 0])
    np.testing.assert_array_equal(gv[0].view(torch.int16).cpu().numpy().view(np.uint16),
                                  fx["kv_bytes"][0, 1])


class GpuRefImageCache(GpuCache):
    """The paged GPU cache read as the reference KVCache holds its bytes
    (rlx_gqa_attend_ref_image, the reference's mask rule)."""

    def attend(self, layer, q):
        S = q.shape[1]
        out = self.c.AttendRefImage(layer, torch.from_numpy(np.ascontiguousarray(q)).to(self.device),
                                    num_heads=self.H, n_q=[S], layout="HSD", mask="ref")
        return out.cpu().numpy()


def test_cfg1_reference_byte_image_on_gpu(gpu):
    """KVH = 2: relux's own decode reads its cache rows scrambled (each
    Append's [KVH, S, D] block copied raw, rows read head-major with stride
    totalLen).  The device's ref-image attention reproduces the oracle
    model over the reference KVCache (RefCache): logits within tolerance,
    greedy tokens equal where the oracle's top-2 gap allows -- and they are
    not the corrected-semantics logits."""
    m = td.TinyDecoder(td.CFG1, seed=0)
    prompt = td.prompt_ids(td.CFG1)
    toks, logits, _ = m.generate(prompt, 16, GpuRefImageCache(m.cfg, gpu))
    ref = td.RefCache(m.cfg)
    want = [m.forward(prompt, ref)[-1]]
    for t in toks[len(prompt):-1]:
        want.append(m.forward([t], ref)[-1])
    want = np.stack(want)
    d = np.abs(logits - want)
    print(f"cfg1 reference byte image: logits max {d.max():.3e} mean {d.mean():.3e}")
    assert d.max() < TOL_MAX and d.mean() < TOL_MEAN
    for i in range(16):
        top2 = np.sort(want[i])[-2:]
        if top2[1] - top2[0] > 2 * d[i].max():
            assert toks[len(prompt) + i] == int(np.argmax(want[i])), i
    logical = td.LogicalCache(m.cfg)
    lw = [m.forward(prompt, logical)[-1]]
    for t in toks[len(prompt):-1]:
        lw.append(m.forward([t], logical)[-1])
    assert np.abs(np.stack(lw)[1:] - want[1:]).max() > 1e-2  # the decode rows differ
    # the committed reference-semantics generation (tests/golden/make_fixtures.py)
    import os
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_tiny_decoder.npz"))
    assert fx["prompt"].tolist() == prompt
    fd = np.abs(logits - fx["logits_ref"])
    assert fd.max() < TOL_MAX and fd.mean() < TOL_MEAN
    # free-running tokens agree step by step until a step the logit
    # difference cannot decide (the runs may part there)
    top2 = np.sort(fx["logits_ref"], axis=1)[:, -2:]
    agreed = 0
    for i in range(16):
        if top2[i, 1] - top2[i, 0] <= 2 * fd[i].max():
            break
        assert toks[len(prompt) + i] == int(fx["tokens_ref"][len(prompt) + i]), i
        agreed += 1
    print(f"cfg1 reference byte image: {agreed} of 16 tokens checked against the fixture")
