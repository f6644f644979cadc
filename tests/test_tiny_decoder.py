"""Config-1 tiny decoder on the CPU oracle: the reference cache semantics,
the corrected semantics and the uncached forward pinned against each other,
and the committed fixtures reproduced byte for byte."""
import os

import numpy as np
import pytest

import oracle
from oracle import tiny_decoder as td

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def model():
    return td.TinyDecoder(td.CFG1, seed=0)


def test_one_kv_head_compat_equals_corrected():
    """With one KV head a cache row is one head's D values, so the
    reference's head-major read (stride totalLen) is the logical order and
    its seqQ == totalLen mask is the causal mask: both caches must agree to
    the bit, tokens and logits."""
    cfg = dict(td.CFG1, kv_heads=1)
    m = td.TinyDecoder(cfg, seed=3)
    p = td.prompt_ids(cfg, seed=3)
    a, la, _ = m.generate(p, 12, td.RefCache(cfg))
    b, lb, _ = m.generate(p, 12, td.LogicalCache(cfg))
    assert a == b
    np.testing.assert_array_equal(la, lb)


def test_two_kv_heads_prefill_agrees_then_decode_scrambles(model):
    """KVH=2: the prefill block is copied raw [KVH,S,D] and read back with
    stride S, so prefill logits match; every decode row is written
    token-major and read head-major, so decode logits differ."""
    p = td.prompt_ids()
    _, la, _ = model.generate(p, 4, td.RefCache(model.cfg))
    _, lb, _ = model.generate(p, 4, td.LogicalCache(model.cfg))
    np.testing.assert_array_equal(la[0], lb[0])
    assert np.abs(la[1:] - lb[1:]).max() > 1e-2


def test_ref_image_permutation(model):
    """The reference byte image equals the logical rows placed by the raw
    copy rule (ref_byte_image), for K and V of both layers."""
    p = td.prompt_ids()
    ref, logical = td.RefCache(model.cfg), td.LogicalCache(model.cfg)
    toks, _, _ = model.generate(p, 6, logical)
    # Feed the same tokens through the reference cache (teacher forcing), so
    # both caches hold the same projected K/V inputs at layer 0.
    model.forward(toks[:len(p)], ref)
    for t in toks[len(p):-1]:
        model.forward([t], ref)
    chunks = [len(p)] + [1] * (len(toks) - 1 - len(p))
    kb = oracle.bf16_from_f32(logical.k[0])
    vb = oracle.bf16_from_f32(logical.v[0])
    np.testing.assert_array_equal(td.ref_byte_image(kb, chunks, model.cfg["max_seq"]), ref.k[0])
    np.testing.assert_array_equal(td.ref_byte_image(vb, chunks, model.cfg["max_seq"]), ref.v[0])


def test_cached_decode_matches_uncached_forward(model):
    """A12: the uncached forward over tokens[:t+1] (positions 0..t, causal,
    f32 K/V) is the exact decode of step t; the bf16 cached decode stays
    within the logits tolerance of it."""
    p = td.prompt_ids()
    toks, logits, _ = model.generate(p, 16, td.LogicalCache(model.cfg))
    for i in range(16):
        t = len(p) - 1 + i
        lu = model.forward_uncached(toks[:t + 1])[-1]
        d = np.abs(lu - logits[i])
        assert d.max() < 2e-3 and d.mean() < 5e-4, (i, d.max())


def test_rope_positions_of_prefill(model):
    """Prefill rotates rows at positions 0..S-1 (rope.go:157, startPos 0):
    rotating the keys again by position is the identity at position 0 and a
    norm-preserving map elsewhere."""
    c, s = model.rope
    x = np.random.default_rng(0).normal(size=(2, 5, model.D)).astype(np.float32)
    y = oracle.rope_apply(x, 0, model.rope, model.cfg["max_seq"])
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def _load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def test_cfg1_fixture_reproduced():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mkfx", os.path.join(GOLDEN, "make_fixtures.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    for name, fn in mk.FIXTURES.items():
        want = _load(name)
        got = fn()
        assert set(got) == set(want), name
        for k in want:
            np.testing.assert_array_equal(np.asarray(got[k]), want[k], err_msg=f"{name}:{k}")


def test_cfg1_fixture_contents():
    d = _load("cfg1_tiny_decoder.npz")
    assert len(d["tokens"]) == 8 + 16 and len(d["tokens_ref"]) == 8 + 16
    assert (d["tokens"] >= 0).all() and (d["tokens"] < 100).all()
    # 23 cached tokens per layer: 2 x 23 x 2 x 16 x 2 B = 2944 B of K+V.
    assert d["kv_bytes"].shape == (2, 2, 2, 23, 16)
    assert d["kv_ref_bytes"].nbytes == 2 * 2944
    # The prefill is computed identically in both semantics, so the first 8
    # rows of the reference image are the logical prefill rows copied raw.
    for layer in range(2):
        for kv in range(2):
            img = td.ref_byte_image(d["kv_bytes"][layer, kv][:, :8], [8], 8)
            np.testing.assert_array_equal(d["kv_ref_bytes"][layer, kv][:8 * 32], img)


def test_bf16_fixture_known_answers():
    """A few hand-derived BF16FromF32 results inside the fixture."""
    d = _load("bf16_fastexp.npz")
    m = dict(zip(d["bf16_in_bits"].tolist(), d["bf16_out"].tolist()))
    assert m[0x3F808000] == 0x3F80  # tie, even stays
    assert m[0x3F818000] == 0x3F82  # tie, odd rounds up
    assert m[0x3F807FFF] == 0x3F80 and m[0x3F808001] == 0x3F81
    assert m[0x7F7FFFFF] == 0x7F80  # overflows to +inf
    assert m[0x7F7F8000] == 0x7F80  # tie at the top, odd -> inf
    assert m[0x42C90000] == 0x42C9  # 100.5 exact
    assert m[0x80000000] == 0x8000 and m[0x00000001] == 0x0000
    assert m[0x7FFFFFFF] == 0x8000  # NaN payload carries into the sign


# ---- AttnType "mla" (TestTransformer_MLA's configuration) ------------------

def test_mla_default_dims():
    """Unset latent dims default to 4 head_dim and head_dim / 2
    (transformer.go:223-233); TestTransformer_MLA sets exactly those."""
    assert td.mla_dims(td.CFG_MLA) == (8, 32, 4)
    assert td.mla_dims(dict(td.CFG_MLA, d_c=0, d_r=0)) == (8, 32, 4)
    assert td.mla_dims(dict(td.CFG1, d_c=None, d_r=None)) == (16, 64, 8)


@pytest.fixture(scope="module")
def mla_model():
    return td.MLATinyDecoder(td.CFG_MLA, seed=0)


def test_mla_cached_decode_equals_uncached(mla_model):
    """Greedy decode over an f32 corrected cache: every step's logits equal
    the matching row of one uncached forward over the whole sequence
    (positions 0..S-1 in one call, causal), which pins the cached length,
    the RoPE offsets of q^R and k^R and the mask."""
    m = mla_model
    p = td.prompt_ids(m.cfg)
    toks, steps, gap = m.generate(p, 16, td.MLALogicalCache(m.cfg, store_bf16=False))
    full = m.forward_uncached(toks[:-1])
    np.testing.assert_allclose(steps, full[len(p) - 1:], rtol=0, atol=2e-6)
    assert gap > 0


def test_mla_one_head_compat_equals_corrected():
    """One head: the reference's head-major read of the decompressed rows is
    the logical order and its seqQ == totalLen mask is causal, so the
    reference cache and the corrected f32 cache agree to the bit."""
    cfg = dict(td.CFG_MLA, d_model=8, heads=1, kv_heads=1)
    m = td.MLATinyDecoder(cfg, seed=2)
    p = td.prompt_ids(cfg, seed=2)
    a, la, _ = m.generate(p, 10, td.MLARefCache(cfg))
    b, lb, _ = m.generate(p, 10, td.MLALogicalCache(cfg, store_bf16=False))
    assert a == b
    np.testing.assert_array_equal(la, lb)


def test_mla_four_heads_ref_read_differs(mla_model):
    """Four heads: forwardCached reads the token-major K_c / V rows
    head-major (mla.go:348-356), so already the prefill differs from the
    per-head slices."""
    m = mla_model
    p = td.prompt_ids(m.cfg)
    _, la, _ = m.generate(p, 2, td.MLARefCache(m.cfg))
    _, lb, _ = m.generate(p, 2, td.MLALogicalCache(m.cfg, store_bf16=False))
    assert np.abs(la[0] - lb[0]).max() > 1e-3


def test_mla_bf16_rows_stay_close(mla_model):
    """bf16 latent rows (the device cache) against f32 rows (the reference
    MLACache) over the same tokens: the logits move by the storage rounding
    only."""
    m = mla_model
    p = td.prompt_ids(m.cfg)
    toks, lf, _ = m.generate(p, 12, td.MLALogicalCache(m.cfg, store_bf16=False))
    c = td.MLALogicalCache(m.cfg)
    lb = [m.forward(p, c)[-1]]
    for t in toks[len(p):-1]:
        lb.append(m.forward([t], c)[-1])
    d = np.abs(np.stack(lb) - lf)
    assert 0 < d.max() < 2e-2 and d.mean() < 2e-3
