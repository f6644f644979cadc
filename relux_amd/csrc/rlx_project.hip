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
// Two kernels: at decode sizes (at most 32 rows) proj_skinny_kernel streams
// the weights with every load in flight at once (below); otherwise
// qkv_project_kernel: work-group = 16 output features x all rows (at most
// 64); its 4 waves take contiguous ranges of the 32-wide k-steps
// (software-pipelined chunks of 8 weight fragments) and meet in LDS.
// MFMA 16x16x32: A = x rows, B = Wp rows.  bf16 activations enter as they
// are; f32 activations as a pair
// hi = bf16(x), lo = bf16(x - hi) multiplied separately into the same f32
// accumulator (bf16 products are exact in f32), which keeps the product sum
// within ~2^-17 of the f32-activation one -- the kernel streams the weights
// from HBM, so the second product costs no time.  The result lane holds 4
// rows of one feature, so a RoPE pair partner (feature ^ 1) is one lane
// away.
#include "rlx_common.h"

namespace rlx {

constexpr int kProjMaxRows = 64;

// Packed weights: the output features of up to 4 matrices m[k][n] (the
// reference's in-row/out-col layout; matrix i holds nh[i] heads of tw[i]
// columns), concatenated with each head padded to pw[i] features by zero
// columns, in MFMA-fragment blocks: element (n, k) at ((n/16 * K/32 + k/32)
// * 16 + n%16) * 32 + k%32, so the B fragment of one (16-feature, 32-k) step
// is 1 KB of contiguous memory.
__global__ void pack_proj_kernel(PackSrc src, int w_bf16, int K, int KP, int N, uint16_t *__restrict__ out) {
    __shared__ uint16_t tile[32][33];
    const int n0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int k = k0 + r, n = n0 + tx;
        uint16_t v = 0;
        if (k < K && n < N) {
            int i = 0, nn = n;
            while (i < 3 && nn >= src.nh[i] * src.pw[i]) nn -= src.nh[i] * src.pw[i++];
            const int head = nn / src.pw[i], d = nn - head * src.pw[i];
            if (d < src.tw[i]) {
                const int64_t off = (int64_t)k * src.nh[i] * src.tw[i] + head * src.tw[i] + d;
                v = w_bf16 ? ((const uint16_t *)src.m[i])[off] : bf16_rne(((const float *)src.m[i])[off]);
            }
        }
        tile[r][tx] = v;
    }
    __syncthreads();
    const int KS = KP / 32;  // (rows K .. KP - 1: zero weights)
    for (int r = ty; r < 32; r += 8) {
        const int n = n0 + r, k = k0 + tx;
        if (n < N && k < KP)
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

// Output placement of one lane: feature n (lane col = n % 16) of the 4 rows
// m*16 + grp*4 + i of lane group grp.  proj_place_plan and proj_place_rope
// read what the plan and the RoPE tables hold for them (positions, append
// slots, (cos, sin)), so a kernel can issue those loads before its products
// and find them done at the output stage; proj_store then rotates and
// writes.  Every lane of the
// wave calls proj_store (a RoPE pair partner, feature n ^ 1, is one lane
// away).  kProjOut: N = D output features, plus the residual; no placement.
struct ProjPlace {
    int part, nn, hw;      // output part, feature within it, features per RoPE head (0: none)
    int tw;                // rotated dims per RoPE head (the RoPE tables' width)
    int rot;               // bit i: row i rotates (position >= 0)
    float c[4], s[4];      // RoPE (cos, sin) of each row
    int page[4], slot[4];  // append slot of each row (k / v / latent parts)
};

// Part of packed feature n: output part, feature within it, features per
// RoPE head and rotated dims per head (0, 0: no RoPE).
template <int MODEL>
__device__ __forceinline__ void proj_part(const ProjDims &pd, int n, int &part, int &nn, int &hw, int &tw) {
    part = 0;
    nn = n;
    hw = tw = 0;
    if constexpr (MODEL == kProjGQA) {
        const int NQ = pd.H * pd.DW, NK = pd.KVH * pd.DW;
        part = n < NQ ? 0 : (n < NQ + NK ? 1 : 2);
        nn = n - (part == 0 ? 0 : (part == 1 ? NQ : NQ + NK));
        hw = part < 2 ? pd.DW : 0;  // (features past D: zero weights, no rotation)
        tw = part < 2 ? pd.D : 0;
    } else if constexpr (MODEL == kProjMLA) {
        const int NQC = pd.H * pd.DW, NQR = pd.H * pd.DRP;
        part = n < NQC ? 0 : (n < NQC + NQR ? 1 : (n < NQC + NQR + pd.DCP ? 2 : 3));
        nn = n - (part == 0 ? 0 : (part == 1 ? NQC : (part == 2 ? NQC + NQR : NQC + NQR + pd.DCP)));
        hw = (part == 1 || part == 3) ? pd.DRP : 0;
        tw = hw ? pd.DR : 0;
    }
}

// Plan reads of the placement (no load depends on another): part, RoPE
// positions (pos < 0: no rotation), append slots.
template <bool ARG, int MODEL>
__device__ __forceinline__ void proj_place_plan(ProjPlace &o, int pos[4], int m, int n, int grp,
                                                int rows, const AppendTok *__restrict__ toks,
                                                const int32_t *__restrict__ pos_dev, int tok_off,
                                                int pos_off, const ProjDims &pd) {
    if constexpr (MODEL != kProjOut) {
        proj_part<MODEL>(pd, n, o.part, o.nn, o.hw, o.tw);
        const bool to_q = (MODEL == kProjGQA) ? o.part == 0 : o.part < 2;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = min(m * 16 + grp * 4 + i, rows - 1);
            pos[i] = -1;
            if (o.hw)
                pos[i] = ARG ? ((const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + pos_off))[r]
                             : pos_dev[r];
            o.page[i] = o.slot[i] = 0;
            if (!to_q) {
                const AppendTok tk = plan_tok<ARG>(toks, tok_off, r);
                o.page[i] = tk.page;
                o.slot[i] = tk.slot;
            }
        }
    }
}

// RoPE (cos, sin) of the placement's rows at their positions.
template <int MODEL>
__device__ __forceinline__ void proj_place_rope(ProjPlace &o, const int pos[4],
                                                const float *__restrict__ rcos,
                                                const float *__restrict__ rsin) {
    if constexpr (MODEL != kProjOut) {
        const int dr = o.hw ? o.nn % o.hw : 0;  // dim within the rotated head
        o.rot = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o.c[i] = o.s[i] = 0.f;
            if (pos[i] >= 0 && dr < o.tw) {  // (padding dims past tw: zero weights, no rotation)
                o.rot |= 1 << i;
                o.c[i] = rcos[(int64_t)pos[i] * (o.tw / 2) + (dr >> 1)];
                o.s[i] = rsin[(int64_t)pos[i] * (o.tw / 2) + (dr >> 1)];
            }
        }
    }
}

// Placement of an output wave's 16 rows when the plan is in the kernel
// arguments: the positions are wave-uniform scalar loads (one per row), so
// the RoPE (cos, sin) reads wait for those only.  n0 = the tile's first
// feature (a part boundary is a multiple of 16, so the part is uniform).
template <int MODEL>
__device__ __forceinline__ void proj_place_kernarg(ProjPlace &o, int m, int n0, int col, int grp,
                                                   int rows, int pos_off, const ProjDims &pd,
                                                   const float *__restrict__ rcos,
                                                   const float *__restrict__ rsin) {
    if constexpr (MODEL != kProjOut) {
        typedef const __attribute__((address_space(4))) int32_t kint;
        int part, nn0, hw, tw;
        proj_part<MODEL>(pd, n0, part, nn0, hw, tw);
        o.part = part;
        o.nn = nn0 + col;
        o.hw = hw;
        o.tw = tw;
        o.rot = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) o.c[i] = o.s[i] = 0.f;
        if (hw && rcos) {  // tables given: row 0 exists, so every load is in bounds
            // the wave's 16 row positions (scalar loads), the lane's 4 rows
            // (group grp) picked as they arrive: constant indices only, so
            // nothing goes through a private array
            int mine[4] = {0, 0, 0, 0};
            kint *kp = (kint *)(kernarg_plan() + pos_off);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int v = __builtin_amdgcn_readfirstlane(kp[min(m * 16 + j, rows - 1)]);
                if ((j >> 2) == grp) mine[j & 3] = v;
            }
            const int dr = o.nn % hw;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = mine[i];
                o.rot |= (p >= 0 && dr < tw) << i;
                // unconditional (no branch, so no wait at a join): row max(p, 0),
                // pair min(dr, tw - 1) / 2 (padding dims past tw do not rotate)
                const int64_t t = (int64_t)max(p, 0) * (tw / 2) + (min(dr, tw - 1) >> 1);
                o.c[i] = rcos[t];
                o.s[i] = rsin[t];
            }
        }
    }
}

// Append slots of the wave's 16 rows from the kernel-argument plan (scalar
// loads), the lane's 4 rows (group grp) picked as they arrive into
// sp / ss[4] (constant indices only: no private array).
__device__ __forceinline__ void proj_slots_kernarg_load(int sp[4], int ss[4], int m, int rows, int tok_off,
                                                        int grp) {
    typedef const __attribute__((address_space(4))) int32_t kint;
    kint *kt = (kint *)(kernarg_plan() + tok_off);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int r = min(m * 16 + j, rows - 1);
        const int pg = __builtin_amdgcn_readfirstlane(kt[r * 4]);
        const int sl = __builtin_amdgcn_readfirstlane(kt[r * 4 + 1]);
        if ((j >> 2) == grp) {
            sp[j & 3] = pg;
            ss[j & 3] = sl;
        }
    }
}
__device__ __forceinline__ void proj_slots_pick(ProjPlace &o, const int sp[4], const int ss[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o.page[i] = sp[i];
        o.slot[i] = ss[i];
    }
}

template <int MODEL>
__device__ __forceinline__ void proj_store(const ProjPlace &o, fl4 y, int m, int n, int grp,
                                           int rows, const ProjDims &pd,
                                           void *__restrict__ q_out, void *__restrict__ q_out2,
                                           int q_bf16, uint16_t *__restrict__ kpool,
                                           uint16_t *__restrict__ vpool, int P) {
    if constexpr (MODEL == kProjOut) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = m * 16 + grp * 4 + i;
            if (r >= rows || n >= pd.D) continue;  // (features past D: packed padding)
            const int64_t off = (int64_t)r * pd.D + n;
            float v = y[i];
            if (q_out2)
                v += q_bf16 ? bf16_f32(((const uint16_t *)q_out2)[off]) : ((const float *)q_out2)[off];
            if (q_bf16)
                ((uint16_t *)q_out)[off] = bf16_rne(v);
            else
                ((float *)q_out)[off] = v;
        }
        return;
    } else {
        const int part = o.part, nn = o.nn, hw = o.hw;
        const int H = pd.H, KVH = pd.KVH;
        const int hdim = (MODEL == kProjGQA) ? pd.DW : (part == 1 ? pd.DRP : pd.DW);
        const int head = nn / hdim, d = nn - head * hdim;
        const int dr = hw ? nn % hw : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = m * 16 + grp * 4 + i;  // C row of element i
            float v = y[i];
            const float partner = __shfl_xor(v, 1);
            if (o.rot & (1 << i)) {
                // RoPE: (x0, x1) -> (x0 c - x1 s, x1 c + x0 s), products rounded
                // separately as in rope.go.
                const float c = o.c[i], sn = o.s[i];
                v = (dr & 1) ? __fadd_rn(__fmul_rn(v, c), __fmul_rn(partner, sn))
                             : __fsub_rn(__fmul_rn(v, c), __fmul_rn(partner, sn));
            }
            if (r >= rows) continue;
            const bool to_q = (MODEL == kProjGQA) ? part == 0 : part < 2;
            if (to_q) {
                // (q_r heads are DRP features wide, of which DR are stored)
                void *dst = (MODEL == kProjMLA && part == 1) ? q_out2 : q_out;
                const int qw = (MODEL == kProjMLA && part == 1) ? pd.DR : pd.D;
                if (d >= qw) continue;
                const int64_t off = ((int64_t)r * H + head) * qw + d;
                if (q_bf16)
                    ((uint16_t *)dst)[off] = bf16_rne(v);
                else
                    ((float *)dst)[off] = v;
                continue;
            }
            if constexpr (MODEL == kProjGQA) {
                if (d >= pd.D) continue;  // (packed padding features)
                const int DS = pd.DS;  // the pool's dims per head (DS - D padding dims: zeroed apart)
                if (part == 1)
                    kpool[((int64_t)o.page[i] * KVH + head) * P * DS + k_page_off(o.slot[i], d, DS)] = bf16_rne(v);
                else
                    vpool[(((int64_t)o.page[i] * KVH + head) * DS + d) * P + o.slot[i]] = bf16_rne(v);
            } else {
                // latent c^KV dims < DC, k^R dims < DR (the row's padding is zeroed apart)
                if (part == 2 ? nn >= pd.DC : nn >= pd.DR) continue;
                kpool[((int64_t)o.page[i] * P + o.slot[i]) * kMlaRow + (part == 2 ? 0 : kMlaDc) + nn] = bf16_rne(v);
            }
        }
    }
}

// Activations as MFMA A operands: bf16 pairs {hi, lo} of two f32 values
// (lo = bf16(x - hi), zero where hi is not finite).
__device__ __forceinline__ u32x2 proj_split2(float a, float b) {
    const uint16_t ha = bf16_rne(a), hb = bf16_rne(b);
    const float ra = bf16_f32(ha), rb = bf16_f32(hb);
    const uint16_t la = (fabsf(ra) < INFINITY) ? bf16_rne(a - ra) : (uint16_t)0;
    const uint16_t lb = (fabsf(rb) < INFINITY) ? bf16_rne(b - rb) : (uint16_t)0;
    return u32x2{(uint32_t)ha | ((uint32_t)hb << 16), (uint32_t)la | ((uint32_t)lb << 16)};
}

template <bool ARG, bool XBF16, int MODEL>
__global__ __launch_bounds__(64 * kProjWaves) void qkv_project_kernel(
    typename PlanSel<ARG>::T plan, const Patch *__restrict__ patches, int n_patch,
    const AppendTok *__restrict__ toks, const int32_t *__restrict__ pos_dev, int tok_off,
    int pos_off, int rows, const void *__restrict__ x, int x_bf16, int K,
    const uint16_t *__restrict__ wp, const ProjDims pd, const float *__restrict__ rcos,
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
                const u32x2 p0 = proj_split2(f0.x, f0.y), p1 = proj_split2(f0.z, f0.w);
                const u32x2 p2 = proj_split2(f1.x, f1.y), p3 = proj_split2(f1.z, f1.w);
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
#pragma unroll
    for (int m = 0; m < kProjMaxRows / 16; m++) {
        if (m >= MT) break;
        fl4 y = acc[m];
#pragma unroll
        for (int w = 0; w < kProjWaves - 1; w++) y += red[w][m][lane];
        ProjPlace pl;
        int pos[4];
        proj_place_plan<ARG, MODEL>(pl, pos, m, n, grp, rows, toks, pos_dev, tok_off, pos_off, pd);
        proj_place_rope<MODEL>(pl, pos, rcos, rsin);
        proj_store<MODEL>(pl, y, m, n, grp, rows, pd, q_out, q_out2, q_bf16, kpool, vpool, P);
    }
}

// Decode-size projection (at most 32 rows, K a multiple of 256 up to 4096):
// the weight stream is the whole cost, so every wave issues all of its loads
// before its first product.  Work-group = K/256 waves x TPW feature tiles of
// 16: wave w takes k-steps [8w, 8w + 8), loads the TPW x 8 weight fragments,
// then the activations of that range (MT row tiles, used for all TPW
// tiles), and multiplies; the waves' sums meet in LDS and are added in wave
// order, so the result does not depend on timing.  Each work-group reads
// all of x from L2; TPW = 2 halves that traffic when there are more tiles
// than one round of work-groups.
constexpr int kSkPer = 8;        // k-steps per wave
constexpr int kSkMaxWaves = 16;  // K <= 4096
constexpr int kSkMaxRows = 32;
constexpr int kSkXRow = 528;                // bytes per staged activation row (512 + pad)
constexpr int kSkXRegion = 16 * kSkXRow;    // one wave's 16 rows x 8 k-steps

template <bool ARG, bool XBF16, int MODEL, int MT, int TPW>
__global__ __launch_bounds__(64 * kSkMaxWaves) void proj_skinny_kernel(
    typename PlanSel<ARG>::T plan, const Patch *__restrict__ patches, int n_patch,
    const AppendTok *__restrict__ toks, const int32_t *__restrict__ pos_dev, int tok_off,
    int pos_off, int rows, const void *__restrict__ x, int K, const uint16_t *__restrict__ wp,
    int NT, const ProjDims pd, const float *__restrict__ rcos, const float *__restrict__ rsin,
    void *__restrict__ q_out, void *__restrict__ q_out2, int q_bf16,
    uint16_t *__restrict__ kpool, uint16_t *__restrict__ vpool, int32_t *__restrict__ table, int P) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nwave = blockDim.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    if (blockIdx.x == 0) {
        for (int i = tid; i < n_patch; i += blockDim.x) {
            const Patch pt = plan_patch<ARG>(patches, i);
            table[pt.idx] = pt.val;
        }
    }
    const int KS = K / 32;
    const int ks_lo = wave * kSkPer;  // this wave's k-steps: [ks_lo, ks_lo + 8)
    // Output waves: (t, m) = (wave / MT, wave % MT).
    const int et = wave / MT, em = wave - (wave / MT) * MT;
    const int etile = min((int)blockIdx.x * TPW + et, NT - 1);
    constexpr bool kEarly = ARG && XBF16;
    ProjPlace pl;
    int pos[4];
    // Per-wave LDS region (per row tile): the activations staged in MFMA
    // order, later the wave's sums for the merge.
    __shared__ __attribute__((aligned(16))) unsigned char lds[kSkMaxWaves * kSkXRegion];
    // Activations first (L2 hits).  bf16: whole 128-byte lines, instruction
    // (pair p, half h) = rows 8h..8h+7 of row tile m x k-steps 2p, 2p+1, each
    // lane 16 bytes (row lane / 8, chunk lane % 8); they reach the MFMA
    // order through LDS.  f32: the A operands directly (lane = row col,
    // group grp), split into hi/lo once the weights are issued.
    u32x4 xf[MT][kSkPer], xl[MT][kSkPer];
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
        for (int j = 0; j < kSkPer; j++) {
            if constexpr (XBF16) {
                const int r = min(m * 16 + (j & 1) * 8 + (lane >> 3), rows - 1);
                const int64_t off = (int64_t)r * K + (ks_lo + (j & ~1)) * 32 + (lane & 7) * 8;
                xf[m][j] = *(const u32x4 *)((const uint16_t *)x + off);
            } else {
                const int r = min(m * 16 + col, rows - 1);
                const int64_t off = (int64_t)r * K + (ks_lo + j) * 32 + grp * 8;
                xf[m][j] = __builtin_bit_cast(u32x4, *(const float4 *)((const float *)x + off));
                xl[m][j] = __builtin_bit_cast(u32x4, *(const float4 *)((const float *)x + off + 4));
            }
        }
    }
    // Then every weight fragment of the work-group's tiles in this k-range.
    u32x4 wf[TPW][kSkPer];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int tile = min((int)blockIdx.x * TPW + t, NT - 1);
        const uint16_t *wblk = wp + (int64_t)tile * KS * 512 + (col * 32 + grp * 8);
#pragma unroll
        for (int j = 0; j < kSkPer; j++)
            wf[t][j] = __builtin_nontemporal_load((const u32x4 *)(wblk + (int64_t)(ks_lo + j) * 512));
    }
    // Keep every load above the products (the scheduler would otherwise
    // interleave them to save registers, leaving a few in flight).
    __builtin_amdgcn_sched_barrier(0);
    // RoPE table reads of the output waves behind them: they retire with the
    // last fragment, so the output stage waits for no further load.
    int sp[4] = {0, 0, 0, 0}, ss[4] = {0, 0, 0, 0};  // append slots of the lane's rows
    if (kEarly && wave < TPW * MT) {
        proj_place_kernarg<MODEL>(pl, em, etile * 16, col, grp, rows, pos_off, pd, rcos, rsin);
        if constexpr (MODEL != kProjOut) {
            const bool to_q = (MODEL == kProjGQA) ? pl.part == 0 : pl.part < 2;
            if (!to_q) proj_slots_kernarg_load(sp, ss, em, rows, tok_off, grp);
        }
    }
    if constexpr (XBF16) {
        // Through this wave's region: rows of 512 bytes + 16 of padding, so
        // the 16 rows of one MFMA read fall on distinct banks.  A wave's LDS
        // accesses run in order: no barrier between its writes and reads.
#pragma unroll
        for (int m = 0; m < MT; m++) {
            unsigned char *reg = lds + (wave * MT + m) * kSkXRegion;
#pragma unroll
            for (int j = 0; j < kSkPer; j++)
                *(u32x4 *)(reg + ((j & 1) * 8 + (lane >> 3)) * kSkXRow + (j >> 1) * 128 + (lane & 7) * 16) = xf[m][j];
#pragma unroll
            for (int j = 0; j < kSkPer; j++)
                xf[m][j] = *(const u32x4 *)(reg + col * kSkXRow + j * 64 + grp * 16);
        }
    } else {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int j = 0; j < kSkPer; j++) {
                const float4 f0 = __builtin_bit_cast(float4, xf[m][j]);
                const float4 f1 = __builtin_bit_cast(float4, xl[m][j]);
                const u32x2 p0 = proj_split2(f0.x, f0.y), p1 = proj_split2(f0.z, f0.w);
                const u32x2 p2 = proj_split2(f1.x, f1.y), p3 = proj_split2(f1.z, f1.w);
                xf[m][j] = u32x4{p0[0], p1[0], p2[0], p3[0]};
                xl[m][j] = u32x4{p0[1], p1[1], p2[1], p3[1]};
            }
    }
    fl4 acc[TPW][MT];
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[t][m] = fl4{0.f, 0.f, 0.f, 0.f};
    auto mul = [&](int t, int j) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            // C[m = row][n = feature]: A = x rows, B = Wp rows.
            acc[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, xf[m][j]), __builtin_bit_cast(bf16x8, wf[t][j]), acc[t][m], 0, 0, 0);
            if constexpr (!XBF16)
                acc[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, xl[m][j]), __builtin_bit_cast(bf16x8, wf[t][j]), acc[t][m], 0, 0, 0);
        }
    };
    // K is a multiple of 256 (the launcher's condition): every wave has 8
    // k-steps and multiplies without conditions, each product waiting only
    // for its own fragment.
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int j = 0; j < kSkPer; j++) mul(t, j);
    // ---- k-split merge: wave (t, m) of the first TPW*MT adds the sums ------
    // (each wave's sums go to the start of its own region, which only it
    // has read so far)
    fl4 *red = (fl4 *)lds;
    const int rstride = MT * kSkXRegion / 16;  // fl4 per wave
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int m = 0; m < MT; m++) red[wave * rstride + (t * MT + m) * 64 + lane] = acc[t][m];
    __syncthreads();
    if (wave >= TPW * MT) return;
    if ((int)blockIdx.x * TPW + et >= NT || em * 16 >= rows) return;
    if constexpr (kEarly) {
        if constexpr (MODEL != kProjOut) {
            const bool to_q = (MODEL == kProjGQA) ? pl.part == 0 : pl.part < 2;
            if (!to_q) proj_slots_pick(pl, sp, ss);
        }
    } else {
        proj_place_plan<ARG, MODEL>(pl, pos, em, etile * 16 + col, grp, rows, toks, pos_dev, tok_off,
                                    pos_off, pd);
        proj_place_rope<MODEL>(pl, pos, rcos, rsin);
    }
    fl4 y = red[wave * 64 + lane];
    for (int w = 1; w < nwave; w++) y += red[w * rstride + wave * 64 + lane];
    proj_store<MODEL>(pl, y, em, etile * 16 + col, grp, rows, pd, q_out, q_out2, q_bf16, kpool,
                      vpool, P);
}

// Zeros in the stored dims past the caller's of the appended rows (recycled
// pages hold earlier tokens' bytes there): GQA K and V dims [D, DS) of
// every kv head; MLA latent dims [DC, 512) and rope dims [512 + DR, 576).
// Thread i of the launch takes element i of the flattened (row, dim) list.
template <bool ARG>
__global__ void proj_pad_zero_kernel(typename PlanSel<ARG>::T plan, const AppendTok *__restrict__ toks,
                                     int tok_off, int rows, int model, const ProjDims pd,
                                     uint16_t *__restrict__ kpool, uint16_t *__restrict__ vpool, int P) {
    const int per = model == kProjGQA ? 2 * pd.KVH * (pd.DS - pd.D) : (kMlaDc - pd.DC) + (kMlaDr - pd.DR);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (per <= 0 || i >= (int64_t)rows * per) return;
    const int r = (int)(i / per), e = (int)(i - (int64_t)r * per);
    const AppendTok tk = plan_tok<ARG>(toks, tok_off, r);
    if (model == kProjGQA) {
        const int pad = pd.DS - pd.D, kv = e / pad % pd.KVH, d = pd.D + e % pad;
        if (e < pd.KVH * pad)
            kpool[((int64_t)tk.page * pd.KVH + kv) * P * pd.DS + k_page_off(tk.slot, d, pd.DS)] = 0;
        else
            vpool[(((int64_t)tk.page * pd.KVH + kv) * pd.DS + d) * P + tk.slot] = 0;
    } else {
        const int d = e < kMlaDc - pd.DC ? pd.DC + e : kMlaDc + pd.DR + (e - (kMlaDc - pd.DC));
        kpool[((int64_t)tk.page * P + tk.slot) * kMlaRow + d] = 0;
    }
}

hipError_t launch_proj_pad_zero(hipStream_t s, int model, const PlanArg *plan, const AppendTok *toks,
                                int tok_off, int rows, const ProjDims &pd, uint16_t *kpool,
                                uint16_t *vpool, int P) {
    const int per = model == kProjGQA ? 2 * pd.KVH * (pd.DS - pd.D) : (kMlaDc - pd.DC) + (kMlaDr - pd.DR);
    if (per <= 0 || rows <= 0) return hipSuccess;
    const int64_t n = (int64_t)rows * per;
    const dim3 g((unsigned)((n + 255) / 256));
    if (plan)
        proj_pad_zero_kernel<true><<<g, 256, 0, s>>>(*plan, toks, tok_off, rows, model, pd, kpool, vpool, P);
    else
        proj_pad_zero_kernel<false><<<g, 256, 0, s>>>(NoPlan{0}, toks, tok_off, rows, model, pd, kpool, vpool, P);
    return hipGetLastError();
}

hipError_t launch_pack_proj(hipStream_t s, const PackSrc &src, int w_bf16, int K, uint16_t *out) {
    int N = 0;
    for (int i = 0; i < 4; i++) N += src.nh[i] * src.pw[i];
    const int KP = (K + 31) / 32 * 32;
    pack_proj_kernel<<<dim3((N + 31) / 32, KP / 32), 256, 0, s>>>(src, w_bf16, K, KP, N, out);
    return hipGetLastError();
}

hipError_t launch_proj(hipStream_t s, int model, const PlanArg *plan, const Patch *patches,
                       int n_patch, const AppendTok *toks, const int32_t *pos, int tok_off,
                       int pos_off, int rows, const void *x, int x_bf16, int K, const uint16_t *wp,
                       const ProjDims &pd, const float *rcos, const float *rsin, void *q_out,
                       void *q_out2, int q_bf16, uint16_t *kpool, uint16_t *vpool, int32_t *table,
                       int P, int cus, hipEvent_t e0, hipEvent_t e1) {
    // kProjOut: N = D (the output features), H and KVH unused.
    const int N = proj_features(model, pd);
    if (rows <= 0 || rows > kProjMaxRows || K % 32 != 0 || N % 16 != 0) return hipErrorInvalidValue;
    // Decode-size calls: proj_skinny_kernel, when its operands fit 128
    // registers per lane (activations MT x 8 fragments, twice for f32;
    // weights TPW x 8).  TPW = 2 when one tile per work-group would take
    // more than one round of resident work-groups (its LDS holds one
    // work-group per CU).
    const int NT = N / 16, MT = (rows + 15) / 16;
    const int nw = K / (32 * kSkPer);
    static const int sk_mode = [] {
        const char *e = getenv("RLX_PROJ_TPW");  // tuning override: 0 = no skinny kernel, 1, 2
        return e ? atoi(e) : -1;
    }();
    // Wave (t, m) of the work-group writes tile t's row tile m: it needs
    // at least TPW * MT waves.
    if (sk_mode != 0 && rows <= kSkMaxRows && K % (32 * kSkPer) == 0 && nw >= MT && nw * MT <= kSkMaxWaves &&
        (x_bf16 || MT == 1)) {
        int tpw = sk_mode > 0 ? sk_mode : (NT > cus ? 2 : 1);
        if (!x_bf16 || MT == 2 || nw < 2) tpw = 1;
        const dim3 grid((NT + tpw - 1) / tpw), block(64 * nw);
#define RLX_SK_LAUNCH(ARGV, XB, MODELV, MTV, TPWV, PLANV)                                              \
    return launch_timed(proj_skinny_kernel<ARGV, XB, MODELV, MTV, TPWV>, grid, block, s, e0, e1, PLANV, \
                        patches, n_patch, toks, pos, tok_off, pos_off, rows, x, K, wp, NT, pd,          \
                        rcos, rsin, q_out, q_out2, q_bf16, kpool, vpool, table, P)
#define RLX_SK_SHAPE(ARGV, MODELV, PLANV)                                                              \
    if (!x_bf16) RLX_SK_LAUNCH(ARGV, false, MODELV, 1, 1, PLANV);                                      \
    if (MT == 2) RLX_SK_LAUNCH(ARGV, true, MODELV, 2, 1, PLANV);                                       \
    if (tpw == 2) RLX_SK_LAUNCH(ARGV, true, MODELV, 1, 2, PLANV);                                      \
    RLX_SK_LAUNCH(ARGV, true, MODELV, 1, 1, PLANV);
#define RLX_SK_MODEL(MODELV)                 \
    if (plan) {                              \
        RLX_SK_SHAPE(true, MODELV, *plan)    \
    } else {                                 \
        RLX_SK_SHAPE(false, MODELV, NoPlan{0}) \
    }
        if (model == kProjGQA) {
            RLX_SK_MODEL(kProjGQA)
        } else if (model == kProjMLA) {
            RLX_SK_MODEL(kProjMLA)
        } else {
            RLX_SK_MODEL(kProjOut)
        }
#undef RLX_SK_MODEL
#undef RLX_SK_SHAPE
#undef RLX_SK_LAUNCH
    }
#define RLX_PROJ_LAUNCH(ARGV, XB, MODELV, PLANV)                                                  \
    return launch_timed(qkv_project_kernel<ARGV, XB, MODELV>, dim3(N / 16), dim3(64 * kProjWaves), \
                        s, e0, e1, PLANV, patches, n_patch, toks, pos, tok_off, pos_off, rows, x,  \
                        x_bf16, K, wp, pd, rcos, rsin, q_out, q_out2, q_bf16, kpool, vpool,        \
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
