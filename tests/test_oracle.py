"""Pin the CPU oracle (oracle/relux_oracle.c) before trusting it.

Each check compares the oracle with something it does not restate: the
reference's own known-answer tests (dtype_test.go, kvcache_test.go,
rope_test.go), an independent formulation (float-comparison rounding, f64
exact softmax attention, absorbed MLA), or closed forms.
"""
import math
import struct

import numpy as np
import pytest

import oracle


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bits_f32(u):
    return struct.unpack("<f", struct.pack("<I", u))[0]


# ---- bf16 conversion (dtype_convert.go:15-35) ------------------------------

def test_bf16_known_answers_dtype_test():
    # dtype_test.go:10-36: typical values round-trip within 1% relative.
    for x in [1.0, -1.0, 0.5, -0.5, 0.001, 1e-6, 1234.5678, -9876.543]:
        got = oracle.round_bf16(np.array([x], np.float32))[0]
        assert abs(float(got) - x) / abs(x) <= 0.01
    # dtype_test.go:38-50: powers of two are exact.
    for p in range(-20, 21):
        x = np.float32(2.0 ** p)
        assert oracle.round_bf16(x) == x
    # dtype_test.go:52-70: +-Inf and +-0 preserved (sign of zero too).
    for x in [math.inf, -math.inf]:
        assert oracle.round_bf16(np.float32(x)) == x
    z = oracle.round_bf16(np.array([-0.0], np.float32))[0]
    assert z == 0 and math.copysign(1.0, float(z)) < 0
    # dtype_test.go:86-102: f64 -> f32 -> bf16 exact for these.
    for x in [1.0, -1.0, 0.5, 100.5]:
        assert oracle.round_bf16(np.float32(x)) == np.float32(x)
    # dtype_test.go:72-84 slice round trip within 1%.
    src = np.array([0.1, 0.2, 0.3, 1.5, -2.5, 100.25], np.float32)
    got = oracle.round_bf16(src)
    assert np.all(np.abs(got - src) <= 0.01 * np.abs(src))


def _rne_by_comparison(u):
    """Independent RNE: choose the nearer of the two bf16 neighbours by
    comparing real distances in f64, ties to the even mantissa."""
    x = np.asarray(u, np.uint32).view(np.float32).astype(np.float64)
    lo = (np.asarray(u, np.uint32) & np.uint32(0xFFFF0000))
    hi = lo + np.uint32(0x10000)
    lo_v = lo.view(np.float32).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        hi_v = hi.view(np.float32).astype(np.float64)
        dlo = np.abs(x - lo_v)
        dhi = np.abs(hi_v - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((lo >> 16) & 1) == 1))
    return np.where(pick_hi, hi >> 16, lo >> 16).astype(np.uint16)


def test_bf16_rne_matches_independent_rounding():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    # finite inputs whose rounding stays finite (|x| below the largest bf16)
    exp = (u >> 23) & 0xFF
    u = u[(exp < 0xFE)]
    got = oracle.bf16_from_f32(u.view(np.float32))
    want = _rne_by_comparison(u)
    assert np.array_equal(got, want)


def test_bf16_special_bit_patterns():
    # Closed-form consequences of the reference's integer formula
    # (dtype_convert.go:21-23), including its NaN behaviour.
    cases = {
        0x7FFFFFFF: 0x8000,  # NaN whose rounding carries into the sign: -0
        0x7F800001: 0x7F80,  # signalling NaN with tiny payload rounds to +Inf
        0x7FC00000: 0x7FC0,  # quiet NaN preserved
        0x7F7FFFFF: 0x7F80,  # f32 max rounds up to +Inf
        0x00000001: 0x0000,  # smallest denormal rounds to +0
        0x00008000: 0x0000,  # tie, even -> down
        0x00018000: 0x0002,  # tie, odd -> up
        0x80000000: 0x8000,
        0x3F800000: 0x3F80,
    }
    # Bit patterns go through numpy arrays: a Python float would quiet the
    # signalling NaN before the oracle sees it.
    u = np.array(list(cases), np.uint32)
    got = oracle.bf16_from_f32(u.view(np.float32))
    assert [hex(g) for g in got] == [hex(w) for w in cases.values()]


# ---- fastexp32 and softmaxRows (mha.go:823-861) ----------------------------

def test_fastexp32_constants_and_band():
    # Reference constants: factor = f32(2^23/ln2), bias = f32(127*2^23-405000).
    assert bits_f32(f32_bits(np.float32(2**23 / math.log(2)))) == np.float32(12102203.0)
    assert np.float32(127 * 2**23 - 405000) == np.float32(1064948224.0)
    assert oracle.fastexp32(np.float32(0.0)) == np.float32(bits_f32(1064948224))
    x = np.linspace(-20, 20, 200001, dtype=np.float32)
    y = oracle.fastexp32(x)
    r = y.astype(np.float64) / np.exp(x.astype(np.float64))
    # Schraudolph's linear-mantissa exp: ratio in [2^-0.0483, 1.0615*2^-0.0483]
    assert r.min() > 0.965 and r.max() < 1.028
    assert np.all(np.diff(y) >= 0)
    assert oracle.fastexp32(np.float32(-88.0)) == 0.0
    assert np.isinf(oracle.fastexp32(np.float32(88.0)))


def test_softmax_rows_properties():
    rng = np.random.default_rng(1)
    m = rng.normal(0, 4, size=(16, 300)).astype(np.float32)
    m[3, :] = -1e4
    m[3, 7] = 0.0  # only one entry survives the -20 cutoff
    s = oracle.softmax_rows(m)
    assert np.allclose(s.sum(axis=1), 1.0, atol=1e-5)
    assert np.array_equal(np.argmax(s, axis=1), np.argmax(m, axis=1))
    assert s[3, 7] == 1.0 and np.count_nonzero(s[3]) == 1
    diff = m - m.max(axis=1, keepdims=True)
    assert np.all(s[diff < -20] == 0.0)
    exact = np.exp(diff.astype(np.float64))
    exact /= exact.sum(axis=1, keepdims=True)
    big = exact > 1e-3
    assert np.all(np.abs(s[big] / exact[big] - 1) < 0.07)


def test_matmuls_against_f64():
    rng = np.random.default_rng(2)
    a = rng.normal(size=(7, 33)).astype(np.float32)
    b = rng.normal(size=(33, 5)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.allclose(oracle.matmul(a, b), ref, rtol=1e-5, atol=1e-5)
    assert np.allclose(oracle.matmul_transb(a, b.T.copy()), ref, rtol=1e-5, atol=1e-5)


# ---- RoPE (rope.go) --------------------------------------------------------

def test_rope_known_answers_rope_test():
    tabs = oracle.rope_tables(4, 10000.0, 4)
    c, s = tabs
    assert c[0] == 1.0 and s[0] == 0.0                     # rope_test.go:10-20
    x = np.array([1, 2, 3, 4], np.float32)
    assert np.allclose(oracle.rope_apply(x, 0, tabs, 4), x, atol=1e-5)  # :22-34
    y = oracle.rope_apply(np.array([1, 0, 0, 1], np.float32), 1, tabs, 4)
    want = [math.cos(1), math.sin(1), -math.sin(0.01), math.cos(0.01)]  # :36-63
    assert np.allclose(y, want, atol=1e-5)
    with pytest.raises(IndexError):                          # :84-95
        oracle.rope_apply(x, 4, tabs, 4)


def test_rope_preserves_pair_norms_and_offset_rule():
    tabs = oracle.rope_tables(64, 10000.0, 512)
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 3, 5, 64)).astype(np.float32)
    for start in (0, 17):
        y = oracle.rope_apply(x, start, tabs, 512)
        n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
        n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
        assert np.allclose(n0, n1, rtol=1e-5, atol=1e-5)
    # startPos > 0 rotates every row at the same position (rope.go:152-153):
    # rows with equal content at seq positions 0 and 4 rotate identically,
    # and equal a rank-1 rotation at that position.
    x2 = x.copy()
    x2[0, 0, 4] = x2[0, 0, 0]
    y = oracle.rope_apply(x2, 17, tabs, 512)
    assert np.array_equal(y[0, 0, 4], y[0, 0, 0])
    r0 = oracle.rope_apply(np.ascontiguousarray(x2[0, 0, 0]), 17, tabs, 512)
    assert np.array_equal(y[0, 0, 0], r0)
    y_zero = oracle.rope_apply(x2, 0, tabs, 512)
    assert not np.array_equal(y_zero[0, 0, 4], y_zero[0, 0, 0])
    # startPos == 0: row r is at position r % seq (rope.go:157)
    y0 = oracle.rope_apply(x, 0, tabs, 512)
    c, s = tabs
    half = 32
    pos = 3
    xr = x[1, 2, pos]
    exp0 = xr[0::2] * c[pos * half:(pos + 1) * half] - xr[1::2] * s[pos * half:(pos + 1) * half]
    assert np.allclose(y0[1, 2, pos, 0::2], exp0, atol=1e-6)


# ---- KVCache byte image (kvcache.go:407-438) ------------------------------

def test_kv_copy_into_known_answers_kvcache_test():
    # kvcache_test.go:16-40 (values exactly representable in bf16)
    dst = np.zeros(2 * 3 * 4, np.uint16)
    oracle.kv_copy_into(dst, np.arange(1, 7, dtype=np.float32), 0, 1, 6)
    assert np.array_equal(oracle.f32_from_bf16(dst[:6]), np.arange(1, 7))
    # kvcache_test.go:42-66: grows by 1 then 2 rows
    dst = np.zeros(3 * 4, np.uint16)
    oracle.kv_copy_into(dst, np.array([1, 2, 3, 4], np.float32), 0, 1, 4)
    oracle.kv_copy_into(dst, np.arange(9, 17, dtype=np.float32), 1, 2, 4)
    assert np.array_equal(oracle.f32_from_bf16(dst), [1, 2, 3, 4, 9, 10, 11, 12, 13, 14, 15, 16])


def test_kv_copy_into_reference_layout_quirk():
    # A [1,KVH=2,n=3,D] block is copied flat, so the rows the reference reads
    # head-major afterwards are a permutation of the logical (h,t) rows.
    KVH, n, D = 2, 3, 2
    src = np.arange(KVH * n * D, dtype=np.float32).reshape(KVH, n, D)
    dst = np.zeros(8 * KVH * D, np.uint16)
    oracle.kv_copy_into(dst, src, 0, n, KVH * D)
    image = oracle.f32_from_bf16(dst[: n * KVH * D])
    assert np.array_equal(image, src.reshape(-1))       # raw copy of [H,S,D]
    token_major = src.transpose(1, 0, 2).reshape(-1)     # what a token-major row store holds
    assert not np.array_equal(image, token_major)


# ---- attention restatements -----------------------------------------------

def _limits(mode, nq, T):
    if mode == "causal":
        return [T - nq + i for i in range(nq)]
    if mode == "ref":
        return [i if nq == T else T - 1 for i in range(nq)]
    return [T - 1] * nq


@pytest.mark.parametrize("mode,nq,T", [("causal", 1, 37), ("causal", 4, 50), ("ref", 5, 5),
                                       ("ref", 3, 9), ("none", 2, 20)])
def test_gqa_attend_against_exact_f64(mode, nq, T):
    rng = np.random.default_rng(4)
    H, KVH, D = 8, 2, 16
    q = rng.normal(size=(H, nq, D)).astype(np.float32)
    k = oracle.round_bf16(rng.normal(size=(KVH, T, D)))
    v = oracle.round_bf16(rng.normal(size=(KVH, T, D)))
    got = oracle.gqa_attend(q, k, v, mode)
    g = H // KVH
    ke, ve = np.repeat(k, g, axis=0), np.repeat(v, g, axis=0)
    want = oracle.exact_attention_f64(q, ke, ve, _limits(mode, nq, T))
    err = np.abs(got - want)
    # fastexp32's weights differ from exp by <= ~3.5%; the output moves by
    # at most that fraction of the spread of V.
    assert err.max() < 0.1 and err.mean() < 0.02
    # a planted head-mapping mistake (kv head h % KVH instead of h // g) fails
    ke_bad = np.stack([k[h % KVH] for h in range(H)])
    ve_bad = np.stack([v[h % KVH] for h in range(H)])
    bad = oracle.exact_attention_f64(q, ke_bad, ve_bad, _limits(mode, nq, T))
    assert np.abs(got - bad).max() > 0.1


def test_mla_decompress_equals_absorbed():
    rng = np.random.default_rng(5)
    H, D, dC, dR, nq, T = 4, 16, 32, 8, 2, 24
    qc = rng.normal(size=(H, nq, D)).astype(np.float32)
    qr = rng.normal(size=(H, nq, dR)).astype(np.float32)
    c = oracle.round_bf16(rng.normal(size=(T, dC)))
    kr = oracle.round_bf16(rng.normal(size=(T, dR)))
    w_uk = oracle.bf16_from_f32(rng.normal(0, 0.2, size=(dC, H * D)))
    w_uv = oracle.bf16_from_f32(rng.normal(0, 0.2, size=(dC, H * D)))
    got = oracle.mla_attend(qc, qr, c, kr, w_uk, w_uv, "causal")
    # absorbed form in f64 with exact softmax (independent of the oracle)
    Wk = oracle.f32_from_bf16(w_uk).astype(np.float64).reshape(dC, H, D)
    Wv = oracle.f32_from_bf16(w_uv).astype(np.float64).reshape(dC, H, D)
    qlat = np.einsum("chd,hid->hic", Wk, qc.astype(np.float64))
    s = (np.einsum("hic,tc->hit", qlat, c) + np.einsum("hir,tr->hit", qr, kr)) / math.sqrt(D + dR)
    lim = np.array(_limits("causal", nq, T))
    s = np.where(np.arange(T)[None, None, :] <= lim[None, :, None], s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    olat = np.einsum("hit,tc->hic", w, c)
    want = np.einsum("hic,chd->hid", olat, Wv)
    err = np.abs(got - want)
    assert err.max() < 0.05 and err.mean() < 0.01
    # the reference's head-major read of token-major buffers differs (H > 1)
    compat = oracle.mla_attend(qc, qr, c, kr, w_uk, w_uv, "causal", head_major_compat=True)
    assert np.abs(compat - got).max() > 0.05
