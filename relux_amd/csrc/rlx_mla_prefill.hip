// MLA chunked prefill, step 1: expand the cached latents of the sequences in
// the call into per-head keys and values (the decompressed form costs 5.9
// TFLOP on config 4 against 16.4 TFLOP for the absorbed form, because here
// every query row of a head reuses the same expanded K/V tile).
//
//   K_c[h][t][d] = sum_c C[t][c] W_UK[c][h*D+d]     (row-major per head)
//   V^T[h][d][t] = sum_c C[t][c] W_UV[c][h*D+d]     (dim-major per head: the
//                                                    A-operand order of P.V)
//
// C rows come straight from the paged latent pool.  MFMA needs the contracted
// index (c) contiguous per lane in both operands, so W is first transposed to
// W^T[h*D+d][c].  The K_c launch puts features on the MFMA M side (a lane
// ends with consecutive dims of one token: row-major K_c); the V^T launch
// puts tokens there (consecutive tokens of one dim: dim-major V^T).  The
// GEMM itself is mla_expand_kernel below.
#include "rlx_common.h"

#include <algorithm>

namespace rlx {

// W [rows][cols] -> WT [cols][rows], bf16, 64x64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t *__restrict__ w,
                                                             uint16_t *__restrict__ wt,
                                                             int rows, int cols) {
    __shared__ uint16_t tile[64][66];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int r = i / 64, c = i % 64;
        if (r0 + r < rows && c0 + c < cols) tile[r][c] = w[(int64_t)(r0 + r) * cols + c0 + c];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int c = i / 64, r = i % 64;
        if (r0 + r < rows && c0 + c < cols) wt[(int64_t)(c0 + c) * rows + r0 + r] = tile[r][c];
    }
}

// Expansion GEMM, persistent: one 8-wave work-group per CU walks the tiles
// blockIdx.x, blockIdx.x + gridDim.x, ...  A tile is 256 features (W^T rows)
// x 128 tokens (latent rows), c in 8 ring stages of 64; the ring runs on
// across tile boundaries, so only the first tile of a work-group waits for
// memory.  Stage = A [256][64] + B [128][64] bf16 (48 KB), 3 stages, filled
// by global_load_lds (6 per wave per stage); chunk c of an LDS row r sits at
// physical chunk c ^ (r & 7), which keeps the MFMA fragment reads
// conflict-free.  Wave (wf, wt) = (wave & 3, wave >> 2) owns features
// [64 wf, 64 wf + 64) x tokens [64 wt, 64 wt + 64): 4 x 4 MFMA 16x16x32
// tiles, two k-steps per stage.  Tile t = (work item t / n_mt, feature tile
// t % n_mt): with gridDim.x a multiple of n_mt a work-group keeps one
// feature tile, and the work-groups of one XCD (b mod 8) share a few, which
// stay in that XCD's L2 while the token tiles stream past.  (The output,
// 1 GB per launch on config 4, costs about as much as the GEMM itself: 0.42
// ms without the stores against 0.73-0.87 ms with them.)
constexpr int kXM = 256;               // features per tile
constexpr int kXN = 128;               // tokens per tile
constexpr int kXK = 64;                // c per stage
constexpr int kXS = 3;                 // ring stages
constexpr int kXSteps = kMlaDc / kXK;  // stages per tile
constexpr int kXStage = (kXM + kXN) * kXK;  // bf16 per stage
constexpr int kXLoadsA = kXM * kXK / 8 / 64 / 8;  // 64-lane A loads per wave per stage (4)
constexpr int kXLoadsB = kXN * kXK / 8 / 64 / 8;  // B loads (2)
constexpr int kXLoads = kXLoadsA + kXLoadsB;

template <int OUT_V>
__global__ __launch_bounds__(512, 1) void mla_expand_kernel(
    const uint16_t *__restrict__ pool, const int32_t *__restrict__ table,
    const AttRow *__restrict__ rows, const int2 *__restrict__ work, int n_work,
    const uint16_t *__restrict__ wt, int N, int H, int P, int dps, uint16_t *__restrict__ dst) {
    // Ring loads left in L2 (no non-temporal hint): the latent rows (B),
    // which every feature tile reads, in both kernels; the W^T tile (A),
    // which the work-group re-reads for each token tile, for K_c only.
    // Measured (config 4, rocprof, K_c / V^T µs): hinted 767 / 849; A kept
    // 743 / 889; B kept 765 / 789; both kept 728 / 822.
    constexpr bool keep_a = OUT_V == 0, keep_b = true;
    __shared__ __attribute__((aligned(16))) uint16_t ring[kXS * kXStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: scalar registers)
    const int col = lane & 15, grp = lane >> 4;
    const int wf = wave & 3, wtk = wave >> 2;
    const int n_mt = (N + kXM - 1) / kXM;
    const int n_tiles = n_mt * n_work;
    const int my_tiles = (n_tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int G = my_tiles * kXSteps;  // ring stages this work-group runs
    const uint32_t ring0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)ring);

    // Per-lane load geometry (the same in every stage): load i of this wave
    // fills 64 consecutive physical chunks of the stage.
    uint32_t a_off[kXLoadsA];  // byte offset of this lane's W^T chunk in a feature tile
    int a_row[kXLoadsA];
#pragma unroll
    for (int i = 0; i < kXLoadsA; i++) {
        const int q = (wave * kXLoadsA + i) * 64 + lane;
        const int r = q >> 3, c = (q & 7) ^ (r & 7);
        a_row[i] = r;
        a_off[i] = (uint32_t)(r * kMlaDc + c * 8) * 2;
    }
    int b_row[kXLoadsB], b_chunk[kXLoadsB];
#pragma unroll
    for (int i = 0; i < kXLoadsB; i++) {
        const int q = (wave * kXLoadsB + i) * 64 + lane;
        const int r = q >> 3;
        b_row[i] = r;
        b_chunk[i] = (q & 7) ^ (r & 7);
    }

    // Issue side: state of the tile whose stages are being loaded.
    const uint16_t *b_ptr[kXLoadsB];
    const uint16_t *a_base = wt;
    int a_lim = kXM - 1;  // last live feature row of the tile
    auto issue_tile_setup = [&](int ti) {
        const int t = (int)blockIdx.x + ti * (int)gridDim.x;
        const int m = t % n_mt;
        const int2 wk = work[t / n_mt];
        const AttRow R = rows[wk.x];
        a_base = wt + (int64_t)m * kXM * kMlaDc;
        a_lim = min(kXM, N - m * kXM) - 1;
        // Pages of the tile's 128 tokens (at most 9: P is a multiple of 16),
        // read as wave-uniform scalars and selected per lane.
        const int t_hi = min(wk.y + kXN, R.len) - 1;
        const int p_lo = wk.y / P, p_hi = t_hi / P;
        int pg[9];
#pragma unroll
        for (int k = 0; k < 9; k++) pg[k] = table[R.tab + min(p_lo + k, p_hi)];
#pragma unroll
        for (int i = 0; i < kXLoadsB; i++) {
            const int tok = min(wk.y + b_row[i], t_hi);
            const int k = tok / P - p_lo;
            int page = pg[0];
#pragma unroll
            for (int kk = 1; kk < 9; kk++) page = (k == kk) ? pg[kk] : page;
            b_ptr[i] = pool + ((int64_t)page * P + tok % P) * kMlaRow + b_chunk[i] * 8;
        }
    };
    auto issue = [&](int g) {
        if (g % kXSteps == 0) issue_tile_setup(g / kXSteps);
        const int c0 = (g % kXSteps) * kXK;
        const uint32_t st = ring0 + (uint32_t)((g % kXS) * kXStage * 2);
        const uint16_t *ab = a_base + c0;
        if (a_lim == kXM - 1 && keep_a) {
#pragma unroll
            for (int i = 0; i < kXLoadsA; i++)
                lds_dma16_keep(ab, a_off[i], st + (uint32_t)((wave * kXLoadsA + i) * 64 * 16));
        } else if (a_lim == kXM - 1) {
#pragma unroll
            for (int i = 0; i < kXLoadsA; i++)
                lds_dma16(ab, a_off[i], st + (uint32_t)((wave * kXLoadsA + i) * 64 * 16));
        } else {  // last feature tile of an N that is not a multiple of 256
#pragma unroll
            for (int i = 0; i < kXLoadsA; i++) {
                const uint32_t off = a_off[i] - (uint32_t)((a_row[i] - min(a_row[i], a_lim)) * kMlaDc * 2);
                lds_dma16(ab, off, st + (uint32_t)((wave * kXLoadsA + i) * 64 * 16));
            }
        }
        if (keep_b) {
#pragma unroll
            for (int i = 0; i < kXLoadsB; i++)
                lds_dma16_keep(b_ptr[i] + c0, st + (uint32_t)(kXM * kXK * 2 + (wave * kXLoadsB + i) * 64 * 16));
        } else {
#pragma unroll
            for (int i = 0; i < kXLoadsB; i++)
                lds_dma16(b_ptr[i] + c0, st + (uint32_t)(kXM * kXK * 2 + (wave * kXLoadsB + i) * 64 * 16));
        }
    };
    static_assert(kXS == 3, "the stage wait covers one stage ahead");

    fl4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fl4{0.f, 0.f, 0.f, 0.f};

    const int mo = 8 * (grp >> 1) + 16 * (grp & 1);
    for (int g = 0; g < kXS - 1 && g < G; g++) issue(g);
    for (int g = 0; g < G; g++) {
        // This wave's loads of stage g landed (stage g + 1, issued after it,
        // may still be in flight; loads retire in issue order).
        if (g + 1 < G) RLX_WAIT_VM(kXLoads); else RLX_WAIT_VM(0);
        ring_barrier();  // stage g visible; stage (g - 1) % kXS no longer read
        if (g + kXS - 1 < G) issue(g + kXS - 1);
        const uint16_t *A = ring + (g % kXS) * kXStage;
        const uint16_t *B = A + kXM * kXK;
#pragma unroll
        for (int kk = 0; kk < kXK / 32; kk++) {
            u32x4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = wf * 64 + i * 16 + col, rb = wtk * 64 + i * 16 + col;
                fa[i] = *(const u32x4 *)(A + ra * kXK + (((kk * 4 + grp) ^ (ra & 7)) << 3));
                fb[i] = *(const u32x4 *)(B + rb * kXK + (((kk * 4 + grp) ^ (rb & 7)) << 3));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = OUT_V ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                            __builtin_bit_cast(bf16x8, fb[i]), __builtin_bit_cast(bf16x8, fa[j]), acc[i][j], 0, 0, 0)
                                      : __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                            __builtin_bit_cast(bf16x8, fa[i]), __builtin_bit_cast(bf16x8, fb[j]), acc[i][j], 0, 0, 0);
        }
        if (g % kXSteps != kXSteps - 1) continue;
        // Tile done: acc[i][j][e] = out[m = 16 i + 4 grp + e][n = 16 j + col]
        // of this wave's block, m = feature (K_c) or token (V^T), contiguous
        // in memory.  Sub-tiles i and i + 1 are paired with one row swap
        // (v_permlane16_swap: odd 16-lane rows of the first operand <-> even
        // rows of the second), after which lane (col, grp) holds the 8
        // consecutive m 16 i + 8 (grp >> 1) + 16 (grp & 1) .. + 7: one
        // 16-byte store, 64 contiguous bytes per output row per instruction.
        const int t = (int)blockIdx.x + (g / kXSteps) * (int)gridDim.x;
        const int f0 = (t % n_mt) * kXM + wf * 64;
        const int2 wk = work[t / n_mt];
        const AttRow R = rows[wk.x];
        const int tk0 = wk.y + wtk * 64;
        const int Tp = R.nsplit;
        const int DP = 1 << dps;  // padded head dim: feature f is dim f % DP of head f / DP
        uint16_t *db = dst + (int64_t)R.part * H * DP;
#pragma unroll
        for (int i = 0; i < 4; i += 2)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t x[2], y[2];
                x[0] = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
                x[1] = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
                y[0] = pack_bf16x2(acc[i + 1][j][0], acc[i + 1][j][1]);
                y[1] = pack_bf16x2(acc[i + 1][j][2], acc[i + 1][j][3]);
                acc[i][j] = fl4{0.f, 0.f, 0.f, 0.f};
                acc[i + 1][j] = fl4{0.f, 0.f, 0.f, 0.f};
                u32x4 w;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const auto sw = __builtin_amdgcn_permlane16_swap(x[h], y[h], false, false);
                    w[h] = sw[0];
                    w[2 + h] = sw[1];
                }
                const int m = 16 * i + mo, n = 16 * j + col;
                if (OUT_V) {
                    const int f = f0 + n, tk = tk0 + m;
                    if (f < N) *(u32x4 *)(db + (int64_t)f * Tp + tk) = w;
                } else {
                    const int f = f0 + m, tk = tk0 + n;
                    if (f < N) *(u32x4 *)(db + ((int64_t)(f >> dps) * Tp + tk) * DP + (f & (DP - 1))) = w;
                }
            }
    }
}

// W [dc][H*D] -> WT [H*DP][512] with zeros for dims d >= D of every head and
// for latent channels c >= dc (the expansion then writes exact zeros for
// the padded dims, and the zero-padded channels of the latent rows meet
// zero weights), 64x64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_pad_kernel(const uint16_t *__restrict__ w,
                                                            uint16_t *__restrict__ wt, int dc,
                                                            int H, int D, int DP) {
    __shared__ uint16_t tile[64][66];
    const int c0 = blockIdx.y * 64;   // latent channels
    const int f0 = blockIdx.x * 64;   // padded features h * DP + d
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int r = i / 64, k = i % 64;  // channel c0 + r, feature f0 + k
        const int f = f0 + k, h = f / DP, d = f - h * DP;
        tile[r][k] = (c0 + r < dc && d < D && h < H) ? w[(int64_t)(c0 + r) * H * D + h * D + d] : 0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += blockDim.x) {
        const int k = i / 64, r = i % 64;
        if (f0 + k < H * DP) wt[(int64_t)(f0 + k) * kMlaDc + c0 + r] = tile[r][k];
    }
}

hipError_t launch_mla_wt(hipStream_t s, const uint16_t *w_uk, const uint16_t *w_uv, int H, int D,
                         int dc, int DP, uint16_t *wt_k, uint16_t *wt_v) {
    if (D > DP || DP % 64 != 0 || dc > kMlaDc) return hipErrorInvalidValue;
    if (D == DP && dc == kMlaDc) {
        const int N = H * D;
        dim3 tg((N + 63) / 64, (kMlaDc + 63) / 64);
        transpose_bf16_kernel<<<tg, 256, 0, s>>>(w_uk, wt_k, kMlaDc, N);
        transpose_bf16_kernel<<<tg, 256, 0, s>>>(w_uv, wt_v, kMlaDc, N);
    } else {
        dim3 tg(H * DP / 64, kMlaDc / 64);
        transpose_pad_kernel<<<tg, 256, 0, s>>>(w_uk, wt_k, dc, H, D, DP);
        transpose_pad_kernel<<<tg, 256, 0, s>>>(w_uv, wt_v, dc, H, D, DP);
    }
    return hipGetLastError();
}

// Rope keys of the call, kr[part + t][0 .. 64) = latent row t's k^R (the
// last 64 entries of the stored row), zero for padding rows t >= len.  One
// block per expansion work item (sequence, 128 tokens); 16-byte chunks.  The
// FA2 kernel then reads each 64-key block's rope keys as one contiguous 8 KB
// region through a running pointer, like K_c.
__global__ __launch_bounds__(256) void mla_rope_gather_kernel(const uint16_t *__restrict__ pool,
                                                              const int32_t *__restrict__ table,
                                                              const AttRow *__restrict__ rows,
                                                              const int2 *__restrict__ work, int P,
                                                              uint16_t *__restrict__ kr) {
    const int2 wk = work[blockIdx.x];
    const AttRow R = rows[wk.x];
    for (int e = threadIdx.x; e < 128 * (kMlaDr / 8); e += blockDim.x) {
        const int t = wk.y + e / (kMlaDr / 8), ch = e % (kMlaDr / 8);
        u32x4 v = u32x4{0, 0, 0, 0};
        if (t < R.len) {
            const int page = table[R.tab + t / P];
            v = *(const u32x4 *)(pool + ((int64_t)page * P + t % P) * kMlaRow + kMlaDc + ch * 8);
        }
        *(u32x4 *)(kr + ((int64_t)R.part + t) * kMlaDr + ch * 8) = v;
    }
}

hipError_t launch_mla_rope_gather(hipStream_t s, const uint16_t *pool, const int32_t *table,
                                  const AttRow *rows, const int2 *work, int n_work, int P,
                                  uint16_t *kr) {
    if (n_work <= 0) return hipSuccess;
    mla_rope_gather_kernel<<<n_work, 256, 0, s>>>(pool, table, rows, work, P, kr);
    return hipGetLastError();
}

hipError_t launch_mla_expand(hipStream_t s, const uint16_t *pool, const int32_t *table,
                             const AttRow *rows, const int2 *work, int n_work, int H, int DP, int P,
                             const uint16_t *wt_k, const uint16_t *wt_v, uint16_t *kc, uint16_t *vt,
                             int cus) {
    if (DP != 128 && DP != 256) return hipErrorInvalidValue;
    const int dps = DP == 128 ? 7 : 8;
    const int N = H * DP;
    if (n_work <= 0) return hipSuccess;
    const int tiles = (N + kXM - 1) / kXM * n_work;
    const int grid = std::max(1, std::min(tiles, cus));
    mla_expand_kernel<0><<<grid, 512, 0, s>>>(pool, table, rows, work, n_work, wt_k, N, H, P, dps, kc);
    mla_expand_kernel<1><<<grid, 512, 0, s>>>(pool, table, rows, work, n_work, wt_v, N, H, P, dps, vt);
    return hipGetLastError();
}

}  // namespace rlx
