// Fused pre-attention step: projection of the new tokens' hidden states,
// RoPE, and the paged append -- for a GQA layer (Q/K/V; RoPE on Q and K) and
// for an MLA layer (q_c, q_r, c^KV, k^R; RoPE on q_r and k^R, the latent row
// appended).
//
// Reference restated (GQA mha.go:250-289, MLA mla.go:279-314): q = x.W_q, k = x.W_k, v = x.W_v
// (matmulBatched3D, bf16 weights widened, f32 sums), RoPE of q and k at the
// cache position (rope.go:130-180: pairs (2i, 2i+1) rotated by
// (cos, sin)[pos][i]), then Append of k and v (kvcache.go:240-316, bf16
// round-to-nearest-even).  Here the three projections are one GEMM against
// a packed weight matrix (features = the H q-heads, then the KVH k-heads,
// then the KVH v-heads, each D features), stored as 1 KB MFMA fragments of
// 16 features x 32 k so that every weight load streams contiguous memory.
//
// The same kernel runs the step after attention (mha.go:356-360 W_O,
// mla.go:384-389; the transformer block's residual add): out = x.W (+ the
// residual), no RoPE, no append.
//
// Work-group = 16 output features x all rows (at most 64); its 4 waves take
// contiguous ranges of the 32-wide k-steps (software-pipelined chunks of 8
// weight fragments) and meet in LDS.  MFMA 16x16x32: A = x rows, B = Wp
// rows.  bf16 activations enter as they are; f32 activations as a pair
// hi = bf16(x), lo = bf16(x - hi) multiplied separately into the same f32
// accumulator (bf16 products are exact in f32), which keeps the product sum
// within ~2^-17 of the f32-activation one -- the kernel streams the weights
// from HBM, so the second product costs no time.  The result lane holds 4
// rows of one feature, so a RoPE pair partner (feature ^ 1) is one lane
// away.
#include "rlx_common.h"

namespace rlx {

constexpr int kProjMaxRows = 64;

// Packed weights: the output features of up to 4 matrices m[k][n] (widths
// wd[i], the reference's in-row/out-col layout), concatenated, in
// MFMA-fragment blocks: element (n, k) at ((n/16 * K/32 + k/32) * 16 + n%16)
// * 32 + k%32, so the B fragment of one (16-feature, 32-k) step is 1 KB of
// contiguous memory.
struct PackSrc {
    const void *m[4];
    int wd[4];
};
__global__ void pack_proj_kernel(PackSrc src, int w_bf16, int K, int N, uint16_t *__restrict__ out) {
    __shared__ uint16_t tile[32][33];
    const int n0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, n = n0 + tx;
        uint16_t v = 0;
        if (k < K && n < N) {
            int i = 0, nn = n;
            while (i < 3 && nn >= src.wd[i]) nn -= src.wd[i++];
            const int64_t off = (int64_t)k * src.wd[i] + nn;
            v = w_bf16 ? ((const uint16_t *)src.m[i])[off] : bf16_rne(((const float *)src.m[i])[off]);
        }
        tile[r][tx] = v;
    }
    __syncthreads();
    const int KS = K / 32;
    for (int r = ty; r < 32; r += 8) {
        const int n = n0 + r, k = k0 + tx;
        if (n < N && k < K)
            out[(((int64_t)(n >> 4) * KS + (k >> 5)) * 16 + (n & 15)) * 32 + (k & 31)] = tile[tx][r];
    }
}

constexpr int kProjWaves = 4;   // k split over the waves of a work-group
constexpr int kProjChunk = 8;   // k-steps of W held in registers at once per wave

// Output layouts (features in packed order, each part a multiple of 16):
//   kProjGQA: q (H heads x D, RoPE)    -> q_out [rows][H][D]
//             k (KVH x D, RoPE)        -> K pages (k-step-major)
//             v (KVH x D)              -> dim-major V pages
//   kProjMLA: q_c (H x D)              -> q_out  [rows][H][D]
//             q_r (H x d_r, RoPE)      -> q_out2 [rows][H][d_r]
//             c^KV (d_c)               -> latent rows [0, d_c)
//             k^R (d_r, RoPE)          -> latent rows [d_c, d_c + d_r)
//   kProjOut:  out (N = features)      -> q_out [rows][N] (+ q_out2, the
//                                         residual, in the same dtype)
constexpr int kProjGQA = 0;
constexpr int kProjMLA = 1;
constexpr int kProjOut = 2;

template <bool ARG, bool XBF16, int MODEL>
__global__ __launch_bounds__(64 * kProjWaves) void qkv_project_kernel(
    typename PlanSel<ARG>::T plan, const Patch *__restrict__ patches, int n_patch,
    const AppendTok *__restrict__ toks, const int32_t *__restrict__ pos_dev, int tok_off,
    int pos_off, int rows, const void *__restrict__ x, int x_bf16, int K,
    const uint16_t *__restrict__ wp, int H, int KVH, int D, const float *__restrict__ rcos,
    const float *__restrict__ rsin, void *__restrict__ q_out, void *__restrict__ q_out2,
    int q_bf16, uint16_t *__restrict__ kpool, uint16_t *__restrict__ vpool,
    int32_t *__restrict__ table, int P) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    if (blockIdx.x == 0) {
        for (int i = tid; i < n_patch; i += 64 * kProjWaves) {
            const Patch pt = plan_patch<ARG>(patches, i);
            table[pt.idx] = pt.val;
        }
    }
    const int n0 = blockIdx.x * 16;
    const int MT = (rows + 15) / 16;
    const int KS = K / 32;
    fl4 acc[kProjMaxRows / 16];
#pragma unroll
    for (int m = 0; m < kProjMaxRows / 16; m++) acc[m] = fl4{0.f, 0.f, 0.f, 0.f};
    // This work-group's weight blocks: KS fragments of 1 KB, contiguous.
    const uint16_t *wblk = wp + (int64_t)blockIdx.x * KS * 512 + (col * 32 + grp * 8);
    // Wave w takes a contiguous range of k-steps, in chunks of kProjChunk
    // fragments.  Software pipeline: the activations of chunk c are loaded,
    // then the weights of chunk c + 1, then chunk c is multiplied -- loads
    // retire in order, so waiting for chunk c's operands leaves chunk c + 1's
    // weights in flight.
    // Wave-uniform bounds (scalar registers).  Loads past a wave's range are
    // clamped to its last k-step (in bounds) and their products skipped, so
    // no load sits in a branch.
    const int per = (KS + kProjWaves - 1) / kProjWaves;
    const int ks_lo = __builtin_amdgcn_readfirstlane(wave * per);
    const int ks_hi = __builtin_amdgcn_readfirstlane(min(KS, wave * per + per));
    auto load_w = [&](u32x4 (&wf)[kProjChunk], int base) {
#pragma unroll
        for (int j = 0; j < kProjChunk; j++)
            wf[j] = __builtin_nontemporal_load((const u32x4 *)(wblk + (int64_t)min(base + j, ks_hi - 1) * 512));
    };
    // Activations of row tile m: bf16 as loaded, or f32 split into hi + lo.
    auto split2 = [](float a, float b) {  // {hi pair, lo pair}
        const uint16_t ha = bf16_rne(a), hb = bf16_rne(b);
        const float ra = bf16_f32(ha), rb = bf16_f32(hb);
        const uint16_t la = (fabsf(ra) < INFINITY) ? bf16_rne(a - ra) : (uint16_t)0;
        const uint16_t lb = (fabsf(rb) < INFINITY) ? bf16_rne(b - rb) : (uint16_t)0;
        return u32x2{(uint32_t)ha | ((uint32_t)hb << 16), (uint32_t)la | ((uint32_t)lb << 16)};
    };
    auto load_x = [&](u32x4 (&xf)[kProjChunk], u32x4 (&xl)[kProjChunk], int base, int m) {
        const int r = min(m * 16 + col, rows - 1);
#pragma unroll
        for (int j = 0; j < kProjChunk; j++) {
            const int64_t off = (int64_t)r * K + min(base + j, ks_hi - 1) * 32 + grp * 8;
            if constexpr (XBF16) {
                xf[j] = *(const u32x4 *)((const uint16_t *)x + off);
            } else {
                const float4 f0 = *(const float4 *)((const float *)x + off);
                const float4 f1 = *(const float4 *)((const float *)x + off + 4);
                const u32x2 p0 = split2(f0.x, f0.y), p1 = split2(f0.z, f0.w);
                const u32x2 p2 = split2(f1.x, f1.y), p3 = split2(f1.z, f1.w);
                xf[j] = u32x4{p0[0], p1[0], p2[0], p3[0]};
                xl[j] = u32x4{p0[1], p1[1], p2[1], p3[1]};
            }
        }
    };
    auto mul = [&](const u32x4 (&wf)[kProjChunk], const u32x4 (&xf)[kProjChunk],
                   const u32x4 (&xl)[kProjChunk], int base, int m) {
#pragma unroll
        for (int j = 0; j < kProjChunk; j++)
            if (base + j < ks_hi) {
                // C[m = row][n = feature]: A = x rows, B = Wp rows.
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xf[j]),
                                                                 __builtin_bit_cast(bf16x8, wf[j]), acc[m], 0, 0, 0);
                if constexpr (!XBF16)
                    acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xl[j]),
                                                                     __builtin_bit_cast(bf16x8, wf[j]), acc[m], 0, 0, 0);
            }
    };
    u32x4 wa[kProjChunk], wb[kProjChunk], xf[kProjChunk], xl[kProjChunk];
    if (ks_lo < ks_hi) load_w(wa, ks_lo);
    for (int base = ks_lo; base < ks_hi; base += 2 * kProjChunk) {
        // chunk at base in wa; next chunk into wb
        for (int m = 0; m < MT; m++) {
            load_x(xf, xl, base, m);
            if (m == MT - 1 && base + kProjChunk < ks_hi) load_w(wb, base + kProjChunk);
            mul(wa, xf, xl, base, m);
        }
        const int b2 = base + kProjChunk;
        if (b2 >= ks_hi) break;
        for (int m = 0; m < MT; m++) {
            load_x(xf, xl, b2, m);
            if (m == MT - 1 && b2 + kProjChunk < ks_hi) load_w(wa, b2 + kProjChunk);
            mul(wb, xf, xl, b2, m);
        }
    }
    // ---- k-split merge: the other waves hand their sums to wave 0 ----------
    __shared__ fl4 red[kProjWaves - 1][kProjMaxRows / 16][64];
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < kProjMaxRows / 16; m++)
            if (m < MT) red[wave - 1][m][lane] = acc[m];
    }
    __syncthreads();
    if (wave != 0) return;
    const int n = n0 + col;
    if constexpr (MODEL == kProjOut) {
        // out[r][n] = x.W (+ residual[r][n]), in q_bf16's dtype.
        const int N = gridDim.x * 16;
#pragma unroll
        for (int m = 0; m < kProjMaxRows / 16; m++) {
            if (m >= MT) break;
            fl4 y = acc[m];
#pragma unroll
            for (int w = 0; w < kProjWaves - 1; w++) y += red[w][m][lane];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = m * 16 + grp * 4 + i;
                if (r >= rows) continue;
                const int64_t o = (int64_t)r * N + n;
                float v = y[i];
                if (q_out2)
                    v += q_bf16 ? bf16_f32(((const uint16_t *)q_out2)[o]) : ((const float *)q_out2)[o];
                if (q_bf16)
                    ((uint16_t *)q_out)[o] = bf16_rne(v);
                else
                    ((float *)q_out)[o] = v;
            }
        }
        return;
    }
    // part of the output this work-group's 16 features belong to (uniform),
    // feature index within the part, RoPE head width (0: no rotation)
    int part, nn, hw;
    if constexpr (MODEL == kProjGQA) {
        const int NQ = H * D, NK = KVH * D;
        part = n < NQ ? 0 : (n < NQ + NK ? 1 : 2);
        nn = n - (part == 0 ? 0 : (part == 1 ? NQ : NQ + NK));
        hw = part < 2 ? D : 0;
    } else {
        const int NQC = H * D, NQR = H * kMlaDr;
        part = n < NQC ? 0 : (n < NQC + NQR ? 1 : (n < NQC + NQR + kMlaDc ? 2 : 3));
        nn = n - (part == 0 ? 0 : (part == 1 ? NQC : (part == 2 ? NQC + NQR : NQC + NQR + kMlaDc)));
        hw = (part == 1 || part == 3) ? kMlaDr : 0;
    }
    const int hdim = (MODEL == kProjGQA) ? D : (part == 1 ? kMlaDr : D);
    const int head = nn / hdim, d = nn - head * hdim;
    const int dr = hw ? nn % hw : 0;  // dim within the rotated head
#pragma unroll
    for (int m = 0; m < kProjMaxRows / 16; m++) {
        if (m >= MT) break;
        fl4 y = acc[m];
#pragma unroll
        for (int w = 0; w < kProjWaves - 1; w++) y += red[w][m][lane];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = m * 16 + grp * 4 + i;  // C row of element i
            float v = y[i];
            const float partner = __shfl_xor(v, 1);
            const bool live = r < rows;
            if (hw) {
                // RoPE: (x0, x1) -> (x0 c - x1 s, x1 c + x0 s), products rounded
                // separately as in rope.go.
                const int p = live ? (ARG ? ((const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + pos_off))[r]
                                           : pos_dev[r])
                                   : 0;
                if (p >= 0) {
                    const float c = rcos[(int64_t)p * (hw / 2) + (dr >> 1)];
                    const float s = rsin[(int64_t)p * (hw / 2) + (dr >> 1)];
                    v = (dr & 1) ? __fadd_rn(__fmul_rn(v, c), __fmul_rn(partner, s))
                                 : __fsub_rn(__fmul_rn(v, c), __fmul_rn(partner, s));
                }
            }
            if (!live) continue;
            const bool to_q = (MODEL == kProjGQA) ? part == 0 : part < 2;
            if (to_q) {
                void *dst = (MODEL == kProjMLA && part == 1) ? q_out2 : q_out;
                const int64_t o = ((int64_t)r * H + head) * hdim + d;
                if (q_bf16)
                    ((uint16_t *)dst)[o] = bf16_rne(v);
                else
                    ((float *)dst)[o] = v;
                continue;
            }
            const AppendTok tk = plan_tok<ARG>(toks, tok_off, r);
            if constexpr (MODEL == kProjGQA) {
                if (part == 1)
                    kpool[((int64_t)tk.page * KVH + head) * P * D + k_page_off(tk.slot, d, D)] = bf16_rne(v);
                else
                    vpool[(((int64_t)tk.page * KVH + head) * D + d) * P + tk.slot] = bf16_rne(v);
            } else {
                kpool[((int64_t)tk.page * P + tk.slot) * kMlaRow + (part == 2 ? 0 : kMlaDc) + nn] = bf16_rne(v);
            }
        }
    }
}

hipError_t launch_pack_proj(hipStream_t s, int n_mats, const void *const *mats, const int *widths,
                            int w_bf16, int K, uint16_t *out) {
    PackSrc src{};
    int N = 0;
    for (int i = 0; i < 4; i++) {
        src.m[i] = i < n_mats ? mats[i] : mats[0];
        src.wd[i] = i < n_mats ? widths[i] : 0;
        N += src.wd[i];
    }
    pack_proj_kernel<<<dim3((N + 31) / 32, (K + 31) / 32), 256, 0, s>>>(src, w_bf16, K, N, out);
    return hipGetLastError();
}

hipError_t launch_proj(hipStream_t s, int model, const PlanArg *plan, const Patch *patches,
                       int n_patch, const AppendTok *toks, const int32_t *pos, int tok_off,
                       int pos_off, int rows, const void *x, int x_bf16, int K, const uint16_t *wp,
                       int H, int KVH, int D, const float *rcos, const float *rsin, void *q_out,
                       void *q_out2, int q_bf16, uint16_t *kpool, uint16_t *vpool, int32_t *table,
                       int P, hipEvent_t e0, hipEvent_t e1) {
    if (rows <= 0 || rows > kProjMaxRows || K % 32 != 0 || D % 16 != 0) return hipErrorInvalidValue;
    // kProjOut: N = D (the output features), H and KVH unused.
    const int N = model == kProjGQA ? (H + 2 * KVH) * D
                                    : (model == kProjMLA ? H * (D + kMlaDr) + kMlaRow : D);
#define RLX_PROJ_LAUNCH(ARGV, XB, MODELV, PLANV)                                                  \
    return launch_timed(qkv_project_kernel<ARGV, XB, MODELV>, dim3(N / 16), dim3(64 * kProjWaves), \
                        s, e0, e1, PLANV, patches, n_patch, toks, pos, tok_off, pos_off, rows, x,  \
                        x_bf16, K, wp, H, KVH, D, rcos, rsin, q_out, q_out2, q_bf16, kpool, vpool, \
                        table, P)
#define RLX_PROJ_MODEL(MODELV)                                                                    \
    if (plan && x_bf16)                                                                           \
        RLX_PROJ_LAUNCH(true, true, MODELV, *plan);                                               \
    else if (plan)                                                                                \
        RLX_PROJ_LAUNCH(true, false, MODELV, *plan);                                              \
    else if (x_bf16)                                                                              \
        RLX_PROJ_LAUNCH(false, true, MODELV, NoPlan{0});                                          \
    else                                                                                          \
        RLX_PROJ_LAUNCH(false, false, MODELV, NoPlan{0});
    if (model == kProjGQA) {
        RLX_PROJ_MODEL(kProjGQA)
    } else if (model == kProjMLA) {
        RLX_PROJ_MODEL(kProjMLA)
    } else {
        RLX_PROJ_MODEL(kProjOut)
    }
#undef RLX_PROJ_MODEL
#undef RLX_PROJ_LAUNCH
    return hipGetLastError();
}

}  // namespace rlx
