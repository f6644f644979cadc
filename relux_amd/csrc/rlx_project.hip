// Fused pre-attention step of a GQA layer: Q/K/V projection of the new
// tokens' hidden states, RoPE on Q and K, and the paged append of K and V.
//
// Reference restated (mha.go:250-289): q = x.W_q, k = x.W_k, v = x.W_v
// (matmulBatched3D, bf16 weights widened, f32 sums), RoPE of q and k at the
// cache position (rope.go:130-180: pairs (2i, 2i+1) rotated by
// (cos, sin)[pos][i]), then Append of k and v (kvcache.go:240-316, bf16
// round-to-nearest-even).  Here the three projections are one GEMM against
// a packed weight matrix (features = the H q-heads, then the KVH k-heads,
// then the KVH v-heads, each D features), stored as 1 KB MFMA fragments of
// 16 features x 32 k so that every weight load streams contiguous memory.
//
// Work-group = 16 output features x all rows (at most 64); its 4 waves take
// contiguous ranges of the 32-wide k-steps (software-pipelined chunks of 8
// weight fragments) and meet in LDS.  MFMA 16x16x32: A = x
// rows (converted to bf16), B = Wp rows.  The result lane holds 4 rows of
// one feature, so a RoPE pair partner (feature ^ 1) is one lane away.
#include "rlx_common.h"

namespace rlx {

constexpr int kProjMaxRows = 64;

// Packed weights: feature n < H*D from w_q[k][n], then w_k, then w_v, in
// MFMA-fragment blocks: element (n, k) at ((n/16 * K/32 + k/32) * 16 + n%16)
// * 32 + k%32, so the B fragment of one (16-feature, 32-k) step is 1 KB of
// contiguous memory.
__global__ void pack_qkv_kernel(const void *__restrict__ w_q, const void *__restrict__ w_k,
                                const void *__restrict__ w_v, int w_bf16, int K, int NQ, int NK,
                                uint16_t *__restrict__ out) {
    __shared__ uint16_t tile[32][33];
    const int N = NQ + 2 * NK;
    const int n0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, n = n0 + tx;
        uint16_t v = 0;
        if (k < K && n < N) {
            const void *src;
            int nn, ld;
            if (n < NQ) { src = w_q; nn = n; ld = NQ; }
            else if (n < NQ + NK) { src = w_k; nn = n - NQ; ld = NK; }
            else { src = w_v; nn = n - NQ - NK; ld = NK; }
            const int64_t off = (int64_t)k * ld + nn;
            v = w_bf16 ? ((const uint16_t *)src)[off] : bf16_rne(((const float *)src)[off]);
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

template <bool ARG, bool XBF16>
__global__ __launch_bounds__(64 * kProjWaves) void qkv_project_kernel(
    typename PlanSel<ARG>::T plan, const Patch *__restrict__ patches, int n_patch,
    const AppendTok *__restrict__ toks, const int32_t *__restrict__ pos_dev, int tok_off,
    int pos_off, int rows, const void *__restrict__ x, int x_bf16, int K,
    const uint16_t *__restrict__ wp, int H, int KVH, int D, const float *__restrict__ rcos,
    const float *__restrict__ rsin, void *__restrict__ q_out, int q_bf16,
    uint16_t *__restrict__ kpool, uint16_t *__restrict__ vpool, int32_t *__restrict__ table,
    int P) {
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
    auto load_x = [&](u32x4 (&xf)[kProjChunk], int base, int m) {
        const int r = min(m * 16 + col, rows - 1);
#pragma unroll
        for (int j = 0; j < kProjChunk; j++) {
            const int64_t off = (int64_t)r * K + min(base + j, ks_hi - 1) * 32 + grp * 8;
            if constexpr (XBF16) {
                xf[j] = *(const u32x4 *)((const uint16_t *)x + off);
            } else {
                const float4 f0 = *(const float4 *)((const float *)x + off);
                const float4 f1 = *(const float4 *)((const float *)x + off + 4);
                xf[j][0] = pack_bf16x2(f0.x, f0.y);
                xf[j][1] = pack_bf16x2(f0.z, f0.w);
                xf[j][2] = pack_bf16x2(f1.x, f1.y);
                xf[j][3] = pack_bf16x2(f1.z, f1.w);
            }
        }
    };
    auto mul = [&](const u32x4 (&wf)[kProjChunk], const u32x4 (&xf)[kProjChunk], int base, int m) {
#pragma unroll
        for (int j = 0; j < kProjChunk; j++)
            if (base + j < ks_hi)
                // C[m = row][n = feature]: A = x rows, B = Wp rows.
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xf[j]),
                                                                 __builtin_bit_cast(bf16x8, wf[j]), acc[m], 0, 0, 0);
    };
    u32x4 wa[kProjChunk], wb[kProjChunk], xf[kProjChunk];
    if (ks_lo < ks_hi) load_w(wa, ks_lo);
    for (int base = ks_lo; base < ks_hi; base += 2 * kProjChunk) {
        // chunk at base in wa; next chunk into wb
        for (int m = 0; m < MT; m++) {
            load_x(xf, base, m);
            if (m == MT - 1 && base + kProjChunk < ks_hi) load_w(wb, base + kProjChunk);
            mul(wa, xf, base, m);
        }
        const int b2 = base + kProjChunk;
        if (b2 >= ks_hi) break;
        for (int m = 0; m < MT; m++) {
            load_x(xf, b2, m);
            if (m == MT - 1 && b2 + kProjChunk < ks_hi) load_w(wa, b2 + kProjChunk);
            mul(wb, xf, b2, m);
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
    const int NQ = H * D, NK = KVH * D;
    const int part = n < NQ ? 0 : (n < NQ + NK ? 1 : 2);  // q, k, v (uniform per work-group)
    const int nn = n - (part == 0 ? 0 : (part == 1 ? NQ : NQ + NK));
    const int head = nn / D, d = nn - head * D;
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
            if (part < 2) {
                // RoPE: (x0, x1) -> (x0 c - x1 s, x1 c + x0 s), products rounded
                // separately as in rope.go.
                const int p = live ? (ARG ? ((const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + pos_off))[r]
                                           : pos_dev[r])
                                   : 0;
                if (p >= 0) {
                    const float c = rcos[(int64_t)p * (D / 2) + (d >> 1)];
                    const float s = rsin[(int64_t)p * (D / 2) + (d >> 1)];
                    v = (d & 1) ? __fadd_rn(__fmul_rn(v, c), __fmul_rn(partner, s))
                                : __fsub_rn(__fmul_rn(v, c), __fmul_rn(partner, s));
                }
            }
            if (!live) continue;
            if (part == 0) {
                const int64_t o = ((int64_t)r * H + head) * D + d;
                if (q_bf16)
                    ((uint16_t *)q_out)[o] = bf16_rne(v);
                else
                    ((float *)q_out)[o] = v;
            } else {
                const AppendTok tk = plan_tok<ARG>(toks, tok_off, r);
                if (part == 1)
                    kpool[(((int64_t)tk.page * KVH + head) * P + tk.slot) * D + d] = bf16_rne(v);
                else
                    vpool[(((int64_t)tk.page * KVH + head) * D + d) * P + tk.slot] = bf16_rne(v);
            }
        }
    }
}

hipError_t launch_pack_qkv(hipStream_t s, const void *w_q, const void *w_k, const void *w_v,
                           int w_bf16, int K, int NQ, int NK, uint16_t *out) {
    const int N = NQ + 2 * NK;
    pack_qkv_kernel<<<dim3((N + 31) / 32, (K + 31) / 32), 256, 0, s>>>(w_q, w_k, w_v, w_bf16, K, NQ,
                                                                      NK, out);
    return hipGetLastError();
}

hipError_t launch_qkv_project(hipStream_t s, const PlanArg *plan, const Patch *patches,
                              int n_patch, const AppendTok *toks, const int32_t *pos, int tok_off,
                              int pos_off, int rows, const void *x, int x_bf16, int K,
                              const uint16_t *wp, int H, int KVH, int D, const float *rcos,
                              const float *rsin, void *q_out, int q_bf16, uint16_t *kpool,
                              uint16_t *vpool, int32_t *table, int P) {
    if (rows <= 0 || rows > kProjMaxRows || K % 32 != 0 || D % 16 != 0) return hipErrorInvalidValue;
    const int N = (H + 2 * KVH) * D;
#define RLX_PROJ_LAUNCH(ARGV, XB, PLANV)                                                          \
    qkv_project_kernel<ARGV, XB><<<N / 16, 64 * kProjWaves, 0, s>>>(                              \
        PLANV, patches, n_patch, toks, pos, tok_off, pos_off, rows, x, x_bf16, K, wp, H, KVH, D,  \
        rcos, rsin, q_out, q_bf16, kpool, vpool, table, P)
    if (plan && x_bf16)
        RLX_PROJ_LAUNCH(true, true, *plan);
    else if (plan)
        RLX_PROJ_LAUNCH(true, false, *plan);
    else if (x_bf16)
        RLX_PROJ_LAUNCH(false, true, NoPlan{0});
    else
        RLX_PROJ_LAUNCH(false, false, NoPlan{0});
#undef RLX_PROJ_LAUNCH
    return hipGetLastError();
}

}  // namespace rlx
