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
// W^T[h*D+d][c].  GEMM tile: 128 tokens x 128 features per 256-thread
// work-group, 32-wide c steps staged in LDS (double buffered), each wave a
// 64 x 64 block of 4 x 4 MFMA 16x16x32 tiles.  The K_c launch puts features
// on the MFMA M side (a lane ends with 4 consecutive dims of one token: one
// 8-byte store into the row-major K_c); the V^T launch puts tokens there (4
// consecutive tokens of one dim: one 8-byte store into the dim-major V^T).
#include "rlx_common.h"

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

constexpr int kDT = 128;  // tokens per tile
constexpr int kDF = 128;  // features per tile
constexpr int kDK = 32;   // c per step
constexpr int kDP = kDK + 8;  // LDS row pitch (bf16)

// work[i] = (call row, first token of the tile).  out_kind 0: K_c, 1: V^T.
template <int OUT_V>
__global__ __launch_bounds__(256) void mla_decompress_kernel(
    const uint16_t *__restrict__ pool, const int32_t *__restrict__ table,
    const AttRow *__restrict__ rows, const int2 *__restrict__ work,
    const uint16_t *__restrict__ wt, int H, int P, uint16_t *__restrict__ dst) {
    __shared__ uint16_t As[2][kDT * kDP];  // latent rows [token][c]
    __shared__ uint16_t Bs[2][kDF * kDP];  // W^T rows [feature][c]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int2 wk = work[blockIdx.x];
    const AttRow R = rows[wk.x];
    const int t0 = wk.y;
    const int f0 = blockIdx.y * kDF;
    const int wt_m = (wave >> 1) * 64;  // this wave's 64 x 64 block
    const int wt_n = (wave & 1) * 64;

    u32x4 ra[2], rb[2];
    auto load = [&](int c0) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int c = tid + 256 * u;  // 512 chunks: row = c / 4, part = c % 4
            const int r = c >> 2, part = c & 3;
            const int t = t0 + r;
            ra[u] = u32x4{0, 0, 0, 0};
            if (t < R.len) {
                const int page = table[R.tab + t / P];
                ra[u] = *(const u32x4 *)(pool + ((int64_t)page * P + t % P) * kMlaRow + c0 + part * 8);
            }
            rb[u] = *(const u32x4 *)(wt + (int64_t)(f0 + r) * kMlaDc + c0 + part * 8);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int c = tid + 256 * u;
            const int r = c >> 2, part = c & 3;
            *(u32x4 *)&As[buf][r * kDP + part * 8] = ra[u];
            *(u32x4 *)&Bs[buf][r * kDP + part * 8] = rb[u];
        }
    };

    fl4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fl4{0.f, 0.f, 0.f, 0.f};

    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int c0 = 0; c0 < kMlaDc; c0 += kDK) {
        const bool has_next = c0 + kDK < kMlaDc;
        if (has_next) load(c0 + kDK);
        // M side: features (K_c) or tokens (V^T); N side: the other.
        const uint16_t *Ms = OUT_V ? As[buf] : Bs[buf];
        const uint16_t *Ns = OUT_V ? Bs[buf] : As[buf];
        const int mbase = OUT_V ? wt_m : wt_n;
        const int nbase = OUT_V ? wt_n : wt_m;
        bf16x8 am[4], bn[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            am[i] = __builtin_bit_cast(bf16x8, *(const u32x4 *)&Ms[(mbase + i * 16 + col) * kDP + grp * 8]);
            bn[i] = __builtin_bit_cast(bf16x8, *(const u32x4 *)&Ns[(nbase + i * 16 + col) * kDP + grp * 8]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am[i], bn[j], acc[i][j], 0, 0, 0);
        if (has_next) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // acc[i][j][e] = out[m = mbase + 16i + 4grp + e][n = nbase + 16j + col]
    const int Tp = R.nsplit;
    const int64_t seq_base = (int64_t)R.part * H * 128;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            u32x2 w;
            w[0] = (uint32_t)bf16_rne(acc[i][j][0]) | ((uint32_t)bf16_rne(acc[i][j][1]) << 16);
            w[1] = (uint32_t)bf16_rne(acc[i][j][2]) | ((uint32_t)bf16_rne(acc[i][j][3]) << 16);
            if (OUT_V) {
                // m = token (4 consecutive), n = feature
                const int t = t0 + wt_m + i * 16 + grp * 4;
                const int f = f0 + wt_n + j * 16 + col;
                const int h = f / 128, d = f % 128;
                *(u32x2 *)(dst + seq_base + ((int64_t)h * 128 + d) * Tp + t) = w;
            } else {
                // m = feature (4 consecutive), n = token
                const int f = f0 + wt_n + i * 16 + grp * 4;
                const int t = t0 + wt_m + j * 16 + col;
                const int h = f / 128, d = f % 128;
                *(u32x2 *)(dst + seq_base + ((int64_t)h * Tp + t) * 128 + d) = w;
            }
        }
}

hipError_t launch_mla_expand(hipStream_t s, const uint16_t *pool, const int32_t *table,
                             const AttRow *rows, const int2 *work, int n_work, const uint16_t *w_uk,
                             const uint16_t *w_uv, int H, int D, int P, uint16_t *wt_k,
                             uint16_t *wt_v, uint16_t *kc, uint16_t *vt) {
    if (D != 128) return hipErrorInvalidValue;
    const int N = H * D;
    dim3 tg((N + 63) / 64, (kMlaDc + 63) / 64);
    transpose_bf16_kernel<<<tg, 256, 0, s>>>(w_uk, wt_k, kMlaDc, N);
    transpose_bf16_kernel<<<tg, 256, 0, s>>>(w_uv, wt_v, kMlaDc, N);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (n_work <= 0) return hipSuccess;
    dim3 g(n_work, N / kDF);
    mla_decompress_kernel<0><<<g, 256, 0, s>>>(pool, table, rows, work, wt_k, H, P, kc);
    mla_decompress_kernel<1><<<g, 256, 0, s>>>(pool, table, rows, work, wt_v, H, P, vt);
    return hipGetLastError();
}

}  // namespace rlx
