"""CPU oracle for relux's KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

ctypes/numpy front end of oracle/liboracle.so (a plain-C restatement of the
reference's Go arithmetic, oracle/relux_oracle.c) plus the page-table state
model in oracle/paged.py.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker.  The
product (relux_amd/) never imports it.

Parity status per function (what pins it; see tests/test_oracle.py):
  bf16_from_f32 / f32_from_bf16  pinned: dtype_test.go known answers, an
                                 independent float-rounding formulation over
                                 2^24 inputs, NaN/Inf/denormal edge cases.
  fastexp32                      pinned: reference constants, closed-form
                                 error band against exp, exact value at 0.
  softmax_rows                   pinned: normalisation, -20 cutoff, argmax.
  matmul / matmul_transb         pinned: f64 brute force.
  matmul_bf16w                   pinned: f64 brute force on non-square shapes
                                 (a planted transposed-index read fails it),
                                 exact integer products, k-ascending f32 sum.
  rmsnorm                        pinned: rmsnorm_test.go known answers, f64
                                 restatement, constant-row closed form
                                 gamma*c/sqrt(c^2+eps) and its eps->0 limit.
  gelu                           pinned: mlp_test.go values, f64
                                 0.5*x*(1+erf(x/sqrt2)) via math.erf,
                                 gelu(x)-gelu(-x) = x.
  add_bias                       pinned: exact f32 add of widened bias.
  ref_gqa_decode_step            pinned: equals gqa_attend and exact f64
                                 attention at one kv head; with two, the
                                 reference's flat head-major read.
  rope_tables / rope_apply       pinned: rope_test.go known answers, norm
                                 invariance, overflow error.
  kv_copy_into                   pinned: kvcache_test.go known answers.
  gqa_attend / mla_attend        pinned: independent f64 exact-softmax numpy
                                 attention within the fastexp32 band; MLA
                                 decompress-all == absorbed form.
  greedy / sample / spec_accept  pinned: sampler_test.go cases, r-sweep
                                 frequencies against each stage's stated
                                 distribution, hand-computed penalties,
                                 acceptance / resample distributions
                                 (oracle/sampling.py, tests/test_sampling.py).
  paged model                    pinned: invariants (append(a||b);
                                 rollback(|b|) == append(a); gather after
                                 compact == before; eviction == dense
                                 attention over surviving tokens).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i = ctypes.c_int
_i64 = ctypes.c_int64


def lib():
    """Load liboracle.so, building it with its Makefile if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        L = ctypes.CDLL(_SO)
        sig = {
            "orc_bf16_from_f32": ([ctypes.c_float], ctypes.c_uint16),
            "orc_f32_from_bf16": ([ctypes.c_uint16], ctypes.c_float),
            "orc_bf16_from_f32_n": ([_f32p, _u16p, _i64], None),
            "orc_f32_from_bf16_n": ([_u16p, _f32p, _i64], None),
            "orc_fastexp32": ([ctypes.c_float], ctypes.c_float),
            "orc_fastexp32_n": ([_f32p, _f32p, _i64], None),
            "orc_softmax_rows": ([_f32p, _i, _i], None),
            "orc_matmul": ([_f32p, _f32p, _f32p, _i, _i, _i], None),
            "orc_matmul_transb": ([_f32p, _f32p, _f32p, _i, _i, _i], None),
            "orc_matmul_bf16w": ([_f32p, _f32p, _u16p, _i, _i, _i], None),
            "orc_rope_tables": ([_i, ctypes.c_float, _i, _f32p, _f32p], None),
            "orc_rope_apply": ([_f32p, _f32p, _i, _i, _i, _i, _i, _f32p, _f32p, _i], _i),
            "orc_kv_copy_into": ([_u16p, _f32p, _i, _i, _i], None),
            "orc_gqa_attend": ([_f32p, _f32p, _f32p, _i, _i, _i, _i, _i, _i, _f32p], None),
            "orc_mla_attend": ([_f32p, _f32p, _f32p, _f32p, _u16p, _u16p, _i, _i, _i, _i, _i, _i,
                                _i, _i, _f32p], None),
            "orc_ref_gqa_decode_step": ([_u16p, _u16p, _i, _i, _f32p, _f32p, _f32p, _i, _i, _i,
                                         _f32p], _i),
            "orc_rmsnorm": ([_f32p, _u16p, ctypes.c_float, _i, _i, _f32p], None),
            "orc_gelu_n": ([_f32p, _f32p, _i64], None),
            "orc_add_bias": ([_f32p, _u16p, _i, _i], None),
            "orc_greedy": ([_f32p, _i], _i),
            "orc_sample": ([_f32p, _i, _f32p, _i32p, ctypes.c_void_p, _i, ctypes.c_float,
                            ctypes.c_void_p], _i),
            "orc_spec_accept": ([_f32p, _f32p, _i32p, _i, _i, _f32p, _f32p, _i32p,
                                 ctypes.POINTER(ctypes.c_int)], _i),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def bf16_from_f32(x):
    """BF16FromF32 (dtype_convert.go:15-24), elementwise; uint16 result."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_from_f32_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f32_from_bf16(b):
    """F32FromBF16 (dtype_convert.go:32-35)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().orc_f32_from_bf16_n(b.reshape(-1), out.reshape(-1), b.size)
    return out


def round_bf16(x):
    """Value of x after a bf16 store (BF16FromF32 then widen)."""
    return f32_from_bf16(bf16_from_f32(x))


def fastexp32(x):
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.float32)
    lib().orc_fastexp32_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def softmax_rows(m):
    m = _f32(m).copy()
    rows, cols = m.shape
    lib().orc_softmax_rows(m, rows, cols)
    return m


def matmul(a, b):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float32)
    lib().orc_matmul(out, a, b, M, K, N)
    return out


def matmul_transb(a, b):
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[0]
    out = np.empty((M, N), np.float32)
    lib().orc_matmul_transb(out, a, b, M, K, N)
    return out


def rope_tables(head_dim, base, max_seq):
    half = head_dim // 2
    c = np.empty(max_seq * half, np.float32)
    s = np.empty(max_seq * half, np.float32)
    lib().orc_rope_tables(head_dim, base, max_seq, c, s)
    return c, s


def rope_apply(x, start_pos, tables, max_seq):
    """RotaryEmbedding.Apply (rope.go:130-180); raises where Go panics."""
    x = _f32(x)
    cos_t, sin_t = tables
    head_dim = x.shape[-1]
    rank1 = 1 if x.ndim == 1 else 0
    seq_len = 1 if x.ndim == 1 else x.shape[-2]
    rows = x.size // head_dim
    out = np.empty_like(x)
    rc = lib().orc_rope_apply(x.reshape(-1), out.reshape(-1), rows, seq_len, rank1, head_dim,
                              start_pos, cos_t, sin_t, max_seq)
    if rc != 0:
        raise IndexError("RotaryEmbedding.Apply: position >= maxSeqLen")
    return out


def matmul_bf16w(a, w_bf16):
    """matmulBatched3D pure-Go branch (mha.go:774-784): a[M,K] @ widen(w[K,N])."""
    a = _f32(a)
    w = np.ascontiguousarray(w_bf16, np.uint16)
    M, K = a.shape
    N = w.shape[1]
    out = np.empty((M, N), np.float32)
    lib().orc_matmul_bf16w(out, a, w, M, K, N)
    return out


def rmsnorm(x, gamma_bf16, eps=1e-5):
    x = _f32(x)
    rows, d = x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm(x, np.ascontiguousarray(gamma_bf16, np.uint16), eps, rows, d, out)
    return out


def gelu(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_gelu_n(x.reshape(-1), y.reshape(-1), x.size)
    return y


def add_bias(y, b_bf16):
    y = _f32(y).copy()
    lib().orc_add_bias(y, np.ascontiguousarray(b_bf16, np.uint16), y.shape[0], y.shape[1])
    return y


def kv_copy_into(dst, src, start_row, seq_len, row_size):
    src = _f32(src)
    lib().orc_kv_copy_into(dst, src.reshape(-1), start_row, seq_len, row_size)


MASK = {"ref": 0, "causal": 1, "none": 2}


def gqa_attend(q, k, v, mask="causal"):
    """mha.go:298-348 restated.  q [H,nq,D]; k,v [KVH,T,D] (widened floats)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    H, nq, D = q.shape
    KVH, T, _ = k.shape
    out = np.empty((H, nq, D), np.float32)
    lib().orc_gqa_attend(q, k, v, H, KVH, D, nq, T, MASK[mask], out)
    return out


def mla_attend(qc, qr, c, kr, w_uk, w_uv, mask="causal", head_major_compat=False):
    """mla.go:316-377 restated.  qc [H,nq,D], qr [H,nq,dR], c [T,dC], kr [T,dR]
    (widened floats), w_uk/w_uv bf16 uint16 [dC, H*D]."""
    qc, qr, c, kr = _f32(qc), _f32(qr), _f32(c), _f32(kr)
    H, nq, D = qc.shape
    dR = qr.shape[2]
    T, dC = c.shape
    out = np.empty((H, nq, D), np.float32)
    lib().orc_mla_attend(qc, qr, c, kr, np.ascontiguousarray(w_uk, np.uint16),
                         np.ascontiguousarray(w_uv, np.uint16), H, D, dC, dR, nq, T, MASK[mask],
                         1 if head_major_compat else 0, out)
    return out


def ref_gqa_decode_step(kbuf, vbuf, cap, length, k_new, v_new, q, H, KVH, D):
    """One reference decode step of one sequence (the CPU baseline)."""
    out = np.empty((H, D), np.float32)
    return lib().orc_ref_gqa_decode_step(kbuf, vbuf, cap, length, _f32(k_new), _f32(v_new),
                                         _f32(q), H, KVH, D, out), out


def exact_attention_f64(q, k, v, mask_limit):
    """Independent f64 attention with exact exp (a textbook restatement used
    to pin the oracle): q [H,nq,D], k,v [H,T,D] already GQA-expanded,
    mask_limit[i] = last key index query i may see."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    H, nq, D = q.shape
    T = k.shape[1]
    s = np.einsum("hid,htd->hit", q, k) / np.sqrt(D)
    j = np.arange(T)[None, None, :]
    lim = np.asarray(mask_limit)[None, :, None]
    s = np.where(j <= lim, s, -np.inf)
    s -= s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("hit,htd->hid", w, v)
