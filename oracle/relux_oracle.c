/*
 * relux_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic of relux's pure-Go KV-cache and
 * cached-attention path (github.com/xDarkicex/relux, internal/transformer).
 * It is the CHECKER for the HIP library in relux_amd/: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path never calls it and must fail loudly without its HIP .so.
 *
 * Every function cites the reference file:line it restates.  Build with
 * -O2 -ffp-contract=off (oracle/Makefile) so that `sum += a*b` stays a
 * separate f32 multiply then f32 add, as Go compiles it for GOAMD64=v1.
 *
 * Pinning (what checks each function against something it does not restate):
 *   orc_bf16_from_f32 / orc_f32_from_bf16  - reference dtype_test.go:10-99
 *        known answers + exhaustive RNE property over all 2^32 inputs
 *        against an independent float-rounding formulation (tests).
 *   orc_fastexp32     - closed form 2^(x/ln2) error band and the reference's
 *        documented constants (tests/test_oracle.py).
 *   orc_softmax_rows  - rows sum to 1, cutoff at diff<-20, fastexp weights.
 *   orc_matmul*       - brute-force f64 products on small shapes
 *        (orc_matmul_bf16w also against a planted transposed read).
 *   orc_rmsnorm / orc_gelu_n / orc_add_bias - rmsnorm_test.go and
 *        mlp_test.go known answers, f64 closed forms (constant row,
 *        erf), exact bias adds.
 *   orc_ref_gqa_decode_step - equals orc_gqa_attend at one kv head.
 *   orc_rope_*        - reference rope_test.go:10-63 known answers,
 *        rotation-norm invariance, overflow error (rope_test.go:84-95).
 *   orc_kv_copy_into  - reference kvcache_test.go:16-106 known answers.
 *   orc_gqa_attend / orc_mla_attend - f64 exact-softmax attention written
 *        independently in numpy (tests), within the fastexp32 error band;
 *        MLA decompressed form == absorbed form (linear-algebra identity).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* dtype_convert.go:15-24 -- integer round-to-nearest-even on the bit
 * pattern, with no NaN special case (a NaN whose low half rounds up can
 * carry into the exponent). */
uint16_t orc_bf16_from_f32(float x) {
    uint32_t u = f2u(x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* dtype_convert.go:32-35 -- zero-extend into the high half. */
float orc_f32_from_bf16(uint16_t b) { return u2f((uint32_t)b << 16); }

void orc_bf16_from_f32_n(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_bf16_from_f32(src[i]);
}

void orc_f32_from_bf16_n(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f32_from_bf16(src[i]);
}

/* mha.go:823-833 -- Schraudolph-style exp.  factor = f32(2^23/ln2),
 * bias = f32(127*2^23 - 405000); one f32 multiply, one f32 add, then
 * truncation toward zero to int32 and a bit reinterpretation. */
float orc_fastexp32(float x) {
    if (x < -87.0f) return 0.0f;
    if (x > 87.0f) return u2f(0x7F800000u);
    const float factor = (float)(8388608.0 / 0.6931471805599453);
    const float bias = (float)(127.0 * 8388608.0 - 405000.0);
    volatile float t = factor * x; /* keep mul and add separate */
    float s = t + bias;
    return u2f((uint32_t)(int32_t)s);
}

void orc_fastexp32_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fastexp32(x[i]);
}

/* mha.go:837-861 -- row max, w = diff<-20 ? 0 : fastexp32(diff),
 * ascending f32 sum, multiply by f32(1/sum). */
void orc_softmax_rows(float *m, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float *row = m + (int64_t)r * cols;
        float mx = row[0];
        for (int j = 1; j < cols; j++)
            if (row[j] > mx) mx = row[j];
        float sum = 0.0f;
        for (int j = 0; j < cols; j++) {
            float diff = row[j] - mx;
            row[j] = (diff < -20.0f) ? 0.0f : orc_fastexp32(diff);
            sum += row[j];
        }
        float inv = 1.0f / sum;
        for (int j = 0; j < cols; j++) row[j] *= inv;
    }
}

/* matmul.go:15-27 -- C[M,N] = A[M,K] @ B[K,N], k ascending, f32 acc.
 * Every C[i][j] is the reference's `sum += a*b` chain (0 first, then k
 * ascending, one f32 multiply and one f32 add per step); the loops only run
 * the chains of one row side by side (k outer, j inner) so that B is read
 * row by row.  The result is bit-identical to the i,j,k loop. */
void orc_matmul(float *out, const float *a, const float *b, int M, int K, int N) {
    for (int i = 0; i < M; i++) {
        float *o = out + (int64_t)i * N;
        for (int j = 0; j < N; j++) o[j] = 0.0f;
        for (int k = 0; k < K; k++) {
            const float aik = a[(int64_t)i * K + k];
            const float *bk = b + (int64_t)k * N;
            for (int j = 0; j < N; j++) o[j] += aik * bk[j];
        }
    }
}

/* matmul.go:32-44 -- C[M,N] = A[M,K] @ B[N,K]^T, k ascending. */
void orc_matmul_transb(float *out, const float *a, const float *b, int M, int K, int N) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float sum = 0.0f;
            for (int k = 0; k < K; k++) sum += a[(int64_t)i * K + k] * b[(int64_t)j * K + k];
            out[(int64_t)i * N + j] = sum;
        }
}

/* mha.go:759-785 (pure-Go branch) -- out[M,N] = a[M,K] @ widen(bf16 b[K,N]).
 * Same chains as orc_matmul (k ascending from 0, separate f32 multiply and
 * add), run row-side-by-side on a widened copy of b. */
void orc_matmul_bf16w(float *out, const float *a, const uint16_t *b, int M, int K, int N) {
    float *bw = (float *)malloc(sizeof(float) * (size_t)K * N);
    for (int64_t e = 0; e < (int64_t)K * N; e++) bw[e] = orc_f32_from_bf16(b[e]);
    orc_matmul(out, a, bw, M, K, N);
    free(bw);
}

/* rope.go:50-75 -- theta_i = f32(1 / f32(pow(base, 2i/d))), angle =
 * f32(f64(pos) * f64(theta)), cos/sin evaluated in f64 then rounded. */
void orc_rope_tables(int head_dim, float base, int max_seq, float *cos_t, float *sin_t) {
    int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++)
        for (int i = 0; i < half; i++) {
            float p = (float)pow((double)base, (double)(2 * i) / (double)head_dim);
            float theta = 1.0f / p;
            float angle = (float)((double)pos * (double)theta);
            cos_t[(int64_t)pos * half + i] = (float)cos((double)angle);
            sin_t[(int64_t)pos * half + i] = (float)sin((double)angle);
        }
}

/* rope.go:130-180 -- rotate pairs.  Position of row r is start_pos when
 * start_pos > 0 (every row, the reference's offset behaviour), 0 for a
 * rank-1 input, else r % seq_len.  Returns -1 where the reference panics
 * (position >= maxSeqLen), else 0. */
int orc_rope_apply(const float *x, float *out, int rows, int seq_len, int rank1, int head_dim,
                   int start_pos, const float *cos_t, const float *sin_t, int max_seq) {
    int half = head_dim / 2;
    for (int r = 0; r < rows; r++) {
        int pos = start_pos > 0 ? start_pos : (rank1 ? 0 : r % seq_len);
        if (pos >= max_seq) return -1;
        const float *c = cos_t + (int64_t)pos * half;
        const float *s = sin_t + (int64_t)pos * half;
        const float *xr = x + (int64_t)r * head_dim;
        float *o = out + (int64_t)r * head_dim;
        for (int i = 0; i < half; i++) {
            float x0 = xr[2 * i], x1 = xr[2 * i + 1];
            volatile float a = x0 * c[i], b = x1 * s[i];
            volatile float e = x1 * c[i], f = x0 * s[i];
            o[2 * i] = a - b;
            o[2 * i + 1] = e + f;
        }
    }
    return 0;
}

/* kvcache.go:407-423 (bf16 branch) -- copy seq_len rows of row_size
 * elements into dst at row start_row, converting with BF16FromF32.  The
 * source is consumed flat, row r = src[r*row_size ...]: for a
 * [1,KVH,n,D] tensor with n>1 and KVH>1 this copies head-major data into
 * token-major rows (the reference's byte image, reproduced exactly). */
void orc_kv_copy_into(uint16_t *dst, const float *src, int start_row, int seq_len, int row_size) {
    for (int r = 0; r < seq_len; r++)
        for (int j = 0; j < row_size; j++)
            dst[(int64_t)(start_row + r) * row_size + j] = orc_bf16_from_f32(src[(int64_t)r * row_size + j]);
}

/* Mask rule shared by the attention restatements.
 *   0: reference rule, mha.go:340 / mla.go:368 -- mask j>i only when
 *      seqQ == totalLen (a chunk on a non-empty cache is unmasked);
 *   1: causal with cache offset -- query i sits at T-nq+i, mask j > T-nq+i;
 *   2: no mask. */
static inline int masked(int mode, int i, int j, int nq, int T) {
    if (mode == 0) return (nq == T) && (j > i);
    if (mode == 1) return j > T - nq + i;
    return 0;
}

/* mha.go:298-348 -- GQA expand (head h reads kv head h/(H/KVH)), scores by
 * matmulFloat32TransB, *= f32(1/sqrt(f64 D)), mask, softmaxRows, P@V by
 * matmulFloat32.  q,out: [H][nq][D]; k,v: [KVH][T][D] (already widened). */
void orc_gqa_attend(const float *q, const float *k, const float *v, int H, int KVH, int D, int nq,
                    int T, int mask_mode, float *out) {
    int g = H / KVH;
    float scale = (float)(1.0 / sqrt((double)D));
    float *w = (float *)malloc(sizeof(float) * (size_t)nq * T);
    for (int h = 0; h < H; h++) {
        const float *qh = q + (int64_t)h * nq * D;
        const float *kh = k + (int64_t)(h / g) * T * D;
        const float *vh = v + (int64_t)(h / g) * T * D;
        orc_matmul_transb(w, qh, kh, nq, D, T);
        for (int i = 0; i < nq; i++)
            for (int j = 0; j < T; j++) {
                w[(int64_t)i * T + j] *= scale;
                if (masked(mask_mode, i, j, nq, T)) w[(int64_t)i * T + j] = -INFINITY;
            }
        orc_softmax_rows(w, nq, T);
        orc_matmul(out + (int64_t)h * nq * D, w, vh, nq, T, D);
    }
    free(w);
}

/* mla.go:316-377 -- decompress every cached latent, kcAll = C @ W_UK and
 * vAll = C @ W_UV (matmulBatched3D, k ascending over dC), broadcast k^R,
 * S = Qc Kc^T + Qr Kr^T (two separate sums, added), *= f32(1/sqrt(f64(D+dR))),
 * mask, softmaxRows, P @ V.
 *   qc: [H][nq][D], qr: [H][nq][dR], c: [T][dC], kr: [T][dR] (widened),
 *   w_uk, w_uv: bf16 [dC][H*D], out: [H][nq][D].
 * head_major_compat = 1 reads the token-major kcAll/vAll buffers as
 * [H][T][D] exactly as mla.go:348-356 indexes them; 0 uses the logical
 * per-head slice kc[h][t][d] = kcAll[t][h*D+d] (as mla.go:159-161 does for
 * the uncached path). */
void orc_mla_attend(const float *qc, const float *qr, const float *c, const float *kr,
                    const uint16_t *w_uk, const uint16_t *w_uv, int H, int D, int dC, int dR, int nq,
                    int T, int mask_mode, int head_major_compat, float *out) {
    int HD = H * D;
    float *kc_all = (float *)malloc(sizeof(float) * (size_t)T * HD);
    float *v_all = (float *)malloc(sizeof(float) * (size_t)T * HD);
    orc_matmul_bf16w(kc_all, c, w_uk, T, dC, HD);
    orc_matmul_bf16w(v_all, c, w_uv, T, dC, HD);
    float *kh = (float *)malloc(sizeof(float) * (size_t)T * D);
    float *vh = (float *)malloc(sizeof(float) * (size_t)T * D);
    float *w = (float *)malloc(sizeof(float) * (size_t)nq * T);
    float *wr = (float *)malloc(sizeof(float) * (size_t)nq * T);
    float scale = (float)(1.0 / sqrt((double)(D + dR)));
    for (int h = 0; h < H; h++) {
        for (int t = 0; t < T; t++)
            for (int d = 0; d < D; d++) {
                int64_t src = head_major_compat ? ((int64_t)h * T + t) * D + d : (int64_t)t * HD + (int64_t)h * D + d;
                kh[(int64_t)t * D + d] = kc_all[src];
                vh[(int64_t)t * D + d] = v_all[src];
            }
        orc_matmul_transb(w, qc + (int64_t)h * nq * D, kh, nq, D, T);
        orc_matmul_transb(wr, qr + (int64_t)h * nq * dR, kr, nq, dR, T);
        for (int64_t i = 0; i < (int64_t)nq * T; i++) w[i] += wr[i];
        for (int i = 0; i < nq; i++)
            for (int j = 0; j < T; j++) {
                w[(int64_t)i * T + j] *= scale;
                if (masked(mask_mode, i, j, nq, T)) w[(int64_t)i * T + j] = -INFINITY;
            }
        orc_softmax_rows(w, nq, T);
        orc_matmul(out + (int64_t)h * nq * D, w, vh, nq, T, D);
    }
    free(kc_all); free(v_all); free(kh); free(vh); free(w); free(wr);
}

/* One reference GQA decode step for ONE sequence, timed as the CPU
 * baseline: mha.go:283-348 after the projections.
 *   1. Append: copyInto of the new token's K and V (kvcache.go:286-287);
 *   2. View + ToF32: widen the WHOLE capacity buffer (tensor.go:139-142,
 *      kvcache.go:371-377 returns the full backing slice);
 *   3. GQA expand by copy (mha.go:299-316);
 *   4. attention loops (mha.go:323-348).
 * kbuf/vbuf: bf16 [cap][KVH*D] contiguous cache with `len` rows filled;
 * k_new/v_new: f32 [KVH*D]; q: [H][D]; out: [H][D].  Returns the new len. */
int orc_ref_gqa_decode_step(uint16_t *kbuf, uint16_t *vbuf, int cap, int len, const float *k_new,
                            const float *v_new, const float *q, int H, int KVH, int D, float *out) {
    int row = KVH * D;
    orc_kv_copy_into(kbuf, k_new, len, 1, row);
    orc_kv_copy_into(vbuf, v_new, len, 1, row);
    int T = len + 1;
    int64_t nel = (int64_t)cap * row;
    float *kw = (float *)malloc(sizeof(float) * nel);
    float *vw = (float *)malloc(sizeof(float) * nel);
    orc_f32_from_bf16_n(kbuf, kw, nel);
    orc_f32_from_bf16_n(vbuf, vw, nel);
    int g = H / KVH;
    float *ke = (float *)malloc(sizeof(float) * (size_t)H * T * D);
    float *ve = (float *)malloc(sizeof(float) * (size_t)H * T * D);
    for (int h = 0; h < H; h++) {
        memcpy(ke + (int64_t)h * T * D, kw + (int64_t)(h / g) * T * D, sizeof(float) * (size_t)T * D);
        memcpy(ve + (int64_t)h * T * D, vw + (int64_t)(h / g) * T * D, sizeof(float) * (size_t)T * D);
    }
    orc_gqa_attend(q, ke, ve, H, H, D, 1, T, 0, out);
    free(kw); free(vw); free(ke); free(ve);
    return T;
}

/* rmsnorm.go:69-116 -- per row: sumSq ascending in f32, meanSq = sumSq/f32(d),
 * rstd = f32(1/sqrt(f64(meanSq + eps))), out = (x*rstd)*gamma. */
void orc_rmsnorm(const float *x, const uint16_t *gamma, float eps, int rows, int d, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (int64_t)r * d;
        float sum = 0.0f;
        for (int j = 0; j < d; j++) sum += xr[j] * xr[j];
        float mean = sum / (float)d;
        float rstd = (float)(1.0 / sqrt((double)(mean + eps)));
        for (int j = 0; j < d; j++) {
            volatile float t = xr[j] * rstd;
            out[(int64_t)r * d + j] = t * orc_f32_from_bf16(gamma[j]);
        }
    }
}

/* mlp.go:448-451 -- 0.5*x*(1 + f32(erf(f64(x)/sqrt2))), f32 products. */
void orc_gelu_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float e = (float)erf((double)x[i] / 1.4142135623730951);
        volatile float h = 0.5f * x[i];
        y[i] = h * (1.0f + e);
    }
}

/* linear.go:65-106 and the bias adds of mlp.go:103-140 -- y[i][j] += f32(bf16 b[j]). */
void orc_add_bias(float *y, const uint16_t *b, int rows, int cols) {
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < cols; j++) y[(int64_t)i * cols + j] += orc_f32_from_bf16(b[j]);
}
