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


# ---- matmulBatched3D (mha.go:759-785), RMSNorm, GELU, bias ---------------

def _bf16w_f64(a, w_bf16):
    """f64 brute force of a[M,K] @ widen(w[K,N]): every product and sum in
    f64 from the widened weight bits, written as explicit loops over the
    index roles (row i of a, column j of w) so that no library routine can
    hide a transposition."""
    wf = oracle.f32_from_bf16(w_bf16).astype(np.float64)
    a64 = a.astype(np.float64)
    M, K = a64.shape
    N = wf.shape[1]
    out = np.zeros((M, N))
    for i in range(M):
        for k in range(K):
            out[i, :] += a64[i, k] * wf[k, :]
    return out


def _close_to_f64(got, want, K):
    # f32 accumulation of K products with |terms| <~ 3: error << 1e-5 * sqrt(K)
    return np.abs(got - want).max() <= 2e-6 * K


def test_matmul_bf16w_against_f64_brute_force():
    rng = np.random.default_rng(20)
    for M, K, N in [(1, 7, 3), (5, 33, 11), (9, 64, 40), (3, 130, 17)]:
        a = rng.normal(size=(M, K)).astype(np.float32)
        w = oracle.bf16_from_f32(rng.normal(size=(K, N)))
        got = oracle.matmul_bf16w(a, w)
        assert got.shape == (M, N)
        assert _close_to_f64(got, _bf16w_f64(a, w), K)
        # A planted transposed-index mistake (w read as [N,K] row-major, the
        # slip a checker and a kernel could share) fails the same check.
        w_t = np.ascontiguousarray(w.reshape(-1)[: K * N].reshape(N, K).T)
        bad = oracle.matmul_bf16w(a, w_t)
        assert not _close_to_f64(bad, _bf16w_f64(a, w), K)
    # Widening is exact: weights that are bf16 integers and integer
    # activations give exact integer products (no rounding anywhere).
    a = rng.integers(-8, 9, size=(4, 16)).astype(np.float32)
    w = oracle.bf16_from_f32(rng.integers(-8, 9, size=(16, 6)).astype(np.float32))
    assert np.array_equal(oracle.matmul_bf16w(a, w),
                          a.astype(np.int64) @ oracle.f32_from_bf16(w).astype(np.int64))


def test_matmul_bf16w_sums_k_ascending_in_f32():
    # Go's loop adds k ascending in f32 (ulp(1e8) = 8, so a 1 added to 1e8
    # is lost): the three orders below give 0, 0 and 1; a k-descending loop
    # would give 1 for the second.
    a = np.array([[1e8, 1.0, -1e8]], np.float32)
    w = oracle.bf16_from_f32(np.ones((3, 1), np.float32))
    assert oracle.matmul_bf16w(a, w)[0, 0] == 0.0
    a = np.array([[1.0, 1e8, -1e8]], np.float32)
    assert oracle.matmul_bf16w(a, w)[0, 0] == 0.0
    a = np.array([[1e8, -1e8, 1.0]], np.float32)
    assert oracle.matmul_bf16w(a, w)[0, 0] == 1.0


def test_rmsnorm_known_answers_rmsnorm_test():
    one = oracle.bf16_from_f32(np.ones(4, np.float32))
    two = oracle.bf16_from_f32(np.full(4, 2.0, np.float32))
    # rmsnorm_test.go:14-25 (hand computed), :27-39, :41-60, :62-75
    y = oracle.rmsnorm(np.array([[1, 2, 3, 4]], np.float32), one, eps=0.0)
    assert np.allclose(y[0], [0.3651, 0.7303, 1.0954, 1.4606], atol=1e-3)
    y = oracle.rmsnorm(np.array([[2, 2, 2, 2]], np.float32), one, eps=0.0)
    assert np.allclose(y[0], 1.0, atol=1e-3)
    y = oracle.rmsnorm(np.array([[1, 2, 3, 4], [2, 2, 2, 2]], np.float32), one, eps=0.0)
    assert np.allclose(y[0], [0.3651, 0.7303, 1.0954, 1.4606], atol=1e-3)
    assert np.allclose(y[1], 1.0, atol=1e-3)
    y = oracle.rmsnorm(np.array([[2, 2, 2, 2]], np.float32), two, eps=0.0)
    assert np.allclose(y[0], 2.0, atol=1e-3)


def test_rmsnorm_against_f64_and_closed_forms():
    rng = np.random.default_rng(21)
    rows, d, eps = 6, 48, 1e-5
    x = rng.normal(0, 3, size=(rows, d)).astype(np.float32)
    g = oracle.bf16_from_f32(rng.normal(1, 0.3, size=d))
    gf = oracle.f32_from_bf16(g).astype(np.float64)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * gf[None, :]
    got = oracle.rmsnorm(x, g, eps)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # constant row c: gamma * c / sqrt(c^2 + eps)
    for c in (0.5, -3.0, 40.0):
        xr = np.full((1, d), c, np.float32)
        want_c = gf * c / math.sqrt(c * c + eps)
        assert np.allclose(oracle.rmsnorm(xr, g, eps)[0], want_c, rtol=2e-6, atol=0)
        # eps -> 0 (here exactly 0): +-gamma by the sign of c
        assert np.allclose(oracle.rmsnorm(xr, g, 0.0)[0], np.sign(c) * gf, rtol=2e-6, atol=0)
    # eps enters under the root: a planted eps-outside-the-root variant
    # (x / (rms + eps)) misses the constant-row closed form at small c.
    c, big_eps = 0.01, 1e-4
    xr = np.full((1, d), c, np.float32)
    ok = gf * c / math.sqrt(c * c + big_eps)
    planted = gf * c / (abs(c) + big_eps)
    assert np.allclose(oracle.rmsnorm(xr, g, big_eps)[0], ok, rtol=2e-6)
    assert not np.allclose(planted, ok, rtol=1e-3)
    # rows are normalised independently and scale-invariant (eps = 0)
    y1 = oracle.rmsnorm(x, g, 0.0)
    y2 = oracle.rmsnorm(x * np.float32(4.0), g, 0.0)
    assert np.allclose(y1, y2, rtol=1e-6, atol=1e-6)


def test_gelu_against_erf_closed_form():
    # mlp_test.go:30-52: gelu(1) ~ 0.8413; gelu(0) = 0; gelu(-1) ~ -0.1587
    assert abs(oracle.gelu(np.array([1.0], np.float32))[0] - 0.8413) < 1e-4
    assert abs(oracle.gelu(np.array([-1.0], np.float32))[0] + 0.1587) < 1e-4
    assert oracle.gelu(np.array([0.0], np.float32))[0] == 0.0
    x = np.linspace(-8, 8, 4001, dtype=np.float32)
    want = np.array([0.5 * float(v) * (1 + math.erf(float(v) / math.sqrt(2))) for v in x])
    got = oracle.gelu(x)
    assert np.abs(got - want).max() <= 4e-7 * np.abs(x).max()
    # gelu(x) - gelu(-x) = x (odd part of x*Phi(x)); exact up to f32 rounding
    assert np.allclose(got - oracle.gelu(-x), x, rtol=0, atol=2e-6)
    # large |x|: identity and zero tails
    assert oracle.gelu(np.array([10.0], np.float32))[0] == 10.0
    assert oracle.gelu(np.array([-10.0], np.float32))[0] == 0.0


def test_add_bias_exact():
    rng = np.random.default_rng(22)
    y = rng.normal(size=(5, 9)).astype(np.float32)
    b = oracle.bf16_from_f32(rng.normal(size=9))
    got = oracle.add_bias(y, b)
    want = (y + oracle.f32_from_bf16(b)[None, :]).astype(np.float32)   # one f32 add each
    assert np.array_equal(got, want)
    # the bias broadcasts over rows by column (i % outDim in linear.go:99-101)
    assert not np.array_equal(got, (y + oracle.f32_from_bf16(b)[:5, None].repeat(9, 1)))


# ---- the CPU-baseline port (mha.go:283-348) ------------------------------

def _baseline_case(KVH, H, D, T, cap, seed):
    rng = np.random.default_rng(seed)
    rows = rng.normal(size=(T, KVH * D)).astype(np.float32)
    kb = np.zeros(cap * KVH * D, np.uint16)
    vb = np.zeros(cap * KVH * D, np.uint16)
    vrows = rng.normal(size=(T, KVH * D)).astype(np.float32)
    oracle.kv_copy_into(kb, rows[: T - 1], 0, T - 1, KVH * D)
    oracle.kv_copy_into(vb, vrows[: T - 1], 0, T - 1, KVH * D)
    q = rng.normal(size=(H, D)).astype(np.float32)
    return rows, vrows, kb, vb, q


@pytest.mark.parametrize("H,T", [(4, 33), (8, 100)])
def test_ref_gqa_decode_step_one_kv_head(H, T):
    # With one kv head the reference's head-major read of its token-major
    # buffer is the logical layout, so one decode step is plain attention of
    # q over all T cached rows (the new row included).
    KVH, D, cap = 1, 16, 160
    rows, vrows, kb, vb, q = _baseline_case(KVH, H, D, T, cap, 23)
    newlen, out = oracle.ref_gqa_decode_step(kb, vb, cap, T - 1, rows[T - 1], vrows[T - 1], q,
                                             H, KVH, D)
    assert newlen == T
    k = oracle.round_bf16(rows).reshape(1, T, D)
    v = oracle.round_bf16(vrows).reshape(1, T, D)
    # the appended row's bytes are BF16FromF32 of the new row
    assert np.array_equal(kb[(T - 1) * D: T * D], oracle.bf16_from_f32(rows[T - 1]))
    same = oracle.gqa_attend(q[:, None, :], k, v, "causal")[:, 0, :]
    assert np.array_equal(out, same)
    exact = oracle.exact_attention_f64(q[:, None, :], np.repeat(k, H, 0), np.repeat(v, H, 0),
                                       [T - 1])[:, 0, :]
    err = np.abs(out - exact)
    assert err.max() < 0.1 and err.mean() < 0.02


def test_ref_gqa_decode_step_reads_flat_buffer_head_major():
    # With two kv heads the reference indexes the widened buffer as
    # [KVH][T][D] although rows were stored token-major: kv head h reads the
    # flat elements [h*T*D, (h+1)*T*D).  The port reproduces that read.
    KVH, H, D, T, cap = 2, 4, 8, 21, 64
    rows, vrows, kb, vb, q = _baseline_case(KVH, H, D, T, cap, 24)
    _, out = oracle.ref_gqa_decode_step(kb, vb, cap, T - 1, rows[T - 1], vrows[T - 1], q,
                                        H, KVH, D)
    kflat = oracle.round_bf16(rows).reshape(-1)[: KVH * T * D].reshape(KVH, T, D)
    vflat = oracle.round_bf16(vrows).reshape(-1)[: KVH * T * D].reshape(KVH, T, D)
    g = H // KVH
    exact = oracle.exact_attention_f64(q[:, None, :], np.repeat(kflat, g, 0),
                                       np.repeat(vflat, g, 0), [T - 1])[:, 0, :]
    err = np.abs(out - exact)
    assert err.max() < 0.1 and err.mean() < 0.02
    logical = oracle.round_bf16(rows).reshape(T, KVH, D).transpose(1, 0, 2)
    vlog = oracle.round_bf16(vrows).reshape(T, KVH, D).transpose(1, 0, 2)
    corrected = oracle.exact_attention_f64(q[:, None, :], np.repeat(logical, g, 0),
                                           np.repeat(vlog, g, 0), [T - 1])[:, 0, :]
    assert np.abs(out - corrected).max() > 0.1
