// MLA absorbed decode over the paged bf16 latent cache.
//
// The reference decompresses every cached latent each step (mla.go:316-377):
//   K^C = C.W_UK, V = C.W_UV, s = (q_c.k_c + q_r.k_r)/sqrt(D+dR), o = softmax(s).V.
// Because K^C and V are linear in C the same numbers follow from
//   q_lat[h] = W_UK[:,h] q_c[h]            (absorb, once per query)
//   s[h,t]   = q_lat[h].c_t + q_r[h].k^R_t  (576-wide dot on the raw cache row)
//   o_lat[h] = sum_t p[h,t] c_t             (512-wide)
//   o[h]     = W_UV[:,h]^T o_lat[h]         (once per query)
// which reads each cached row once instead of expanding it H*D*2 times.
//
// Work item = (sequence, context split); one work-group of NW waves.
// 16-token tiles of cache rows (16 x 1152 B) stream from HBM straight into
// an LDS ring (global_load_lds).  Scores: the 18 k-steps of S^T[16 tok][16 rows] are split over the waves
// (MFMA 16x16x32, A = tile rows read from LDS) and the partial S^T are
// summed in LDS, one tile ahead of their use.  Every wave then runs the same
// online softmax; wave w owns latent channels [w*CH, (w+1)*CH), CH =
// 512 / NW, of O^T[512][16 rows] += C^T . P^T (MFMA 16x16x16, A = tile
// columns read transposed from LDS, B = P^T straight from the softmax
// registers).
#include "rlx_common.h"

#include <algorithm>

namespace rlx {

__device__ __forceinline__ int mla_key_limit(int mask_mode, int len, int nq, int qi) {
    if (mask_mode == kMaskCausal) return len - nq + qi;
    if (mask_mode == kMaskRef) return (nq == len) ? qi : len - 1;
    return len - 1;
}

// Split an f32 into a bf16 pair with hi + lo = x to ~16 more bits than hi
// alone (x - hi is exact in f32; non-finite x keeps lo = 0).  MFMA products
// of bf16 operands are exact in f32, so W.hi + W.lo accumulated in f32
// follows the f32 product sum closely.
__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    hi = bf16_rne(x);
    const float h = bf16_f32(hi);
    lo = (fabsf(h) < INFINITY) ? bf16_rne(x - h) : (uint16_t)0;
}

// q_lat[row][h][c] = bf16(qscale * sum_d q_nope[row][h][d] * W_UK[c][h*D+d])
// for c < d_c (0 for d_c <= c < 512: the stored latent rows are zero there)
// and q_lat[row][h][512+r] = bf16(qscale * q_rope[row][h][r]) for r < d_r (0
// past it).  Block = (head, 64 latent channels, 16 query rows); wave w
// computes C[16 channels][16 rows] = W_UK_h[c0+16w .., :] . q^T with MFMA
// 16x16x32 over the head's D dims (KS = ceil(D / 32) k-steps, dims past D
// load zeros): A = 8 consecutive W_UK dims of one channel per lane, B = 8
// consecutive query dims of one row per lane (f32 queries as hi + lo bf16
// pairs).  Every load is issued before the first product, so the kernel
// costs one memory round trip.
template <int KS>
__device__ __forceinline__ void absorb_block(int h, int by, int bz, const void *__restrict__ q_nope,
                                             const void *__restrict__ q_rope, int q_bf16,
                                             const uint16_t *__restrict__ w_uk, int H, int D,
                                             int dc, int dr, int total_q, float qscale,
                                             uint16_t *__restrict__ qlat) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int c0 = by * 64 + wave * 16;
    const int r0 = bz * 16;
    const int row = min(r0 + col, total_q - 1);  // rows past the end load the last row
    const bool cv = c0 + col < dc;
    const uint16_t *wa = w_uk + (int64_t)(cv ? c0 + col : 0) * H * D + (int64_t)h * D + grp * 8;
    u32x4 a[KS], bh[KS], bl[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const bool dv = ks * 32 + grp * 8 < D;
        a[ks] = (cv && dv) ? *(const u32x4 *)(wa + ks * 32) : u32x4{0, 0, 0, 0};
    }
    const int64_t qoff = ((int64_t)row * H + h) * D + grp * 8;
    if (q_bf16) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const bool dv = ks * 32 + grp * 8 < D;
            bh[ks] = dv ? *(const u32x4 *)((const uint16_t *)q_nope + qoff + ks * 32) : u32x4{0, 0, 0, 0};
            bl[ks] = u32x4{0, 0, 0, 0};
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const bool dv = ks * 32 + grp * 8 < D;
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (dv) {
                const float *qf = (const float *)q_nope + qoff + ks * 32;
                const float4 f0 = *(const float4 *)qf, f1 = *(const float4 *)(qf + 4);
                v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
                v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint16_t h0, l0, h1, l1;
                split_bf16(v[2 * i], h0, l0);
                split_bf16(v[2 * i + 1], h1, l1);
                bh[ks][i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                bl[ks][i] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            }
        }
    }
    fl4 acc = fl4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[ks]),
                                                      __builtin_bit_cast(bf16x8, bh[ks]), acc, 0, 0, 0);
    if (!q_bf16) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[ks]),
                                                          __builtin_bit_cast(bf16x8, bl[ks]), acc, 0, 0, 0);
    }
    // C[4 grp + i][col]: channels c0 + 4 grp + i of row r0 + col.
    if (r0 + col < total_q) {
        u32x2 o;
        o[0] = (uint32_t)bf16_rne(acc[0] * qscale) | ((uint32_t)bf16_rne(acc[1] * qscale) << 16);
        o[1] = (uint32_t)bf16_rne(acc[2] * qscale) | ((uint32_t)bf16_rne(acc[3] * qscale) << 16);
        *(u32x2 *)(qlat + ((int64_t)(r0 + col) * H + h) * kMlaRow + c0 + 4 * grp) = o;
    }
    if (by == 0) {
        for (int i = threadIdx.x; i < 16 * kMlaDr; i += blockDim.x) {
            const int r = i / kMlaDr, k = i - r * kMlaDr;
            if (r0 + r >= total_q) continue;
            float x = 0.f;
            if (k < dr) {
                const int64_t off = ((int64_t)(r0 + r) * H + h) * dr + k;
                x = q_bf16 ? bf16_f32(((const uint16_t *)q_rope)[off]) : ((const float *)q_rope)[off];
            }
            qlat[((int64_t)(r0 + r) * H + h) * kMlaRow + kMlaDc + k] = bf16_rne(x * qscale);
        }
    }
}

template <int KS>
__global__ __launch_bounds__(256) void mla_absorb_kernel(const void *__restrict__ q_nope,
                                                         const void *__restrict__ q_rope,
                                                         int q_bf16,
                                                         const uint16_t *__restrict__ w_uk,
                                                         int H, int D, int dc, int dr, int total_q,
                                                         float qscale, uint16_t *__restrict__ qlat) {
    absorb_block<KS>(blockIdx.x, blockIdx.y, blockIdx.z, q_nope, q_rope, q_bf16, w_uk, H, D, dc, dr,
                     total_q, qscale, qlat);
}

// The absorb and the step's latent append in one launch
// (rlx_mla_append_attend): blocks [0, H * 8 * nz) absorb (head fastest, then
// the 64-channel block, then the 16-row tile), the rest run the append's
// threads.  Neither part reads what the other writes: the attention that
// reads both is the next launch.
template <int KS, bool ARG>
__global__ __launch_bounds__(256) void mla_absorb_append_kernel(
    typename PlanSel<ARG>::T plan, const void *__restrict__ q_nope, const void *__restrict__ q_rope,
    int q_bf16, const uint16_t *__restrict__ w_uk, int H, int D, int dc, int dr, int total_q,
    float qscale, uint16_t *__restrict__ qlat, int nz, uint16_t *__restrict__ pool,
    int32_t *__restrict__ table, const Patch *__restrict__ patches, int n_patch,
    const AppendTok *__restrict__ toks, int tok_off, int n_tok, const void *__restrict__ c_src,
    const void *__restrict__ kr_src, int src_bf16, int P) {
    const int nb = H * (kMlaDc / 64) * nz;
    const int b = blockIdx.x;
    if (b < nb) {
        const int rest = b / H;
        absorb_block<KS>(b - rest * H, rest % (kMlaDc / 64), rest / (kMlaDc / 64), q_nope, q_rope,
                         q_bf16, w_uk, H, D, dc, dr, total_q, qscale, qlat);
        return;
    }
    mla_append_thread<ARG>((int64_t)(b - nb) * blockDim.x + threadIdx.x, pool, table, patches,
                           n_patch, toks, tok_off, n_tok, c_src, kr_src, src_bf16, dc, dr, P);
}

// LDS tile layout: 16 token rows x 72 chunks of 16 B (576 bf16), no padding.
// Logical chunk c of row r lives at physical chunk c ^ mla_swz(r), which
// stays inside the row's aligned group of 8 chunks.  The swizzle keeps the
// two read patterns free of bank conflicts: score reads (8 lanes = 8 rows,
// one chunk each) see 8 distinct chunk slots, and transpose reads (16 lanes
// = 4 rows x one 32-B chunk pair) see 4 distinct chunk pairs.
__device__ __forceinline__ int mla_swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// Token bounds of a row's splits: the row's ceil(len / 16) tiles are dealt
// out evenly, split s of n covering [b(s), b(s + 1)) with b(s) = 16 *
// floor(s * tiles / n) (b(n) = len), so a row's splits differ by at most one
// tile, the partial last tile included (rounding token bounds down to a
// tile gave an 8193-token row's last split 36 tiles against 34).  The host
// keeps n <= len / 64, so no split is empty.
__device__ __forceinline__ int mla_split_bound(int len, int n, int s) {
    const int tiles = (len + 15) >> 4;
    return s >= n ? len : (int)(((int64_t)s * tiles / n) << 4);
}

// Shape per query-row tile count: 4 waves and two work-groups per CU (80 KB
// of LDS each); a 4-stage ring for up to 16 query rows, 3 stages for 32.
template <int NQT> struct MlaShape {
    static constexpr int NW = 4;                      // waves
    static constexpr int S = NQT == 1 ? 4 : 3;        // LDS ring stages
    static constexpr int WGS = 2;                     // resident work-groups per CU
    static constexpr int LOADS = 16 * kMlaRow / 8 / 64;  // 64-lane loads per tile (18)
    static constexpr int CH = kMlaDc / NW;            // latent channels per wave
};

// KEEP: ring loads without the non-temporal hint, for calls whose head
// groups re-read the same latent rows (they then meet them in L2: 128 heads
// at 8k, 66.4 -> 61.3 us); single-group calls keep the hint (config 3:
// 53.0 against 58.0 us without it).
template <int NQT, bool ARG, bool KEEP>
__global__ __launch_bounds__(64 * MlaShape<NQT>::NW, MlaShape<NQT>::WGS) void mla_decode_kernel(
    typename PlanSel<ARG>::T plan, const uint16_t *__restrict__ pool,
    const int32_t *__restrict__ table, const AttRow *__restrict__ rows,
    const int2 *__restrict__ work, int n_rows, const uint16_t *__restrict__ qlat, int H, int P,
    int mask_mode, uint16_t *__restrict__ part_o, float *__restrict__ part_ml) {
    using SH = MlaShape<NQT>;
    constexpr int NW = SH::NW, S = SH::S, CH = SH::CH, MT = CH / 16;
    constexpr int QRP = 16 * NQT;
    constexpr int TILE = 16 * kMlaRow;  // bf16 per stage
    // Tile loads per wave: the 18 64-lane loads of a tile go round-robin to
    // the waves, so the first 18 % NW waves issue one more.
    constexpr int LB = SH::LOADS / NW + 1, LS = SH::LOADS / NW;
    constexpr int KB = 18 / NW + 1, KSM = 18 / NW;  // score k-steps per wave
    __shared__ __attribute__((aligned(16))) uint16_t ring[S * TILE];
    __shared__ fl4 spart[2][NW][NQT][64];  // [tile parity][wave] partial scores

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int2 wk = plan_work<ARG>(work, n_rows, blockIdx.x);
    const AttRow R = plan_row<ARG>(rows, wk.x);
    // This work item's query rows: rows [q0, q0 + qn) of the sequence's
    // H x nq (query-major: row qi H + h), one head group of a call with more
    // rows than a work-group holds.
    const int QR = R.qn;
    const int t_begin = mla_split_bound(R.len, R.nsplit, wk.y);
    const int t_end = mla_split_bound(R.len, R.nsplit, wk.y + 1);
    const int ntiles = (t_end - t_begin + 15) / 16;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)ring;

    float m_run[NQT], l_part[NQT];
    fl4 acc[NQT][MT];
#pragma unroll
    for (int nt = 0; nt < NQT; nt++) {
        m_run[nt] = -INFINITY;
        l_part[nt] = 0.f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[nt][mt] = fl4{0.f, 0.f, 0.f, 0.f};
    }

    // Tile j (16 tokens) streams straight from HBM into ring stage j % S
    // (global_load_lds, 16 B per lane, non-temporal).  One instruction fills
    // 64 consecutive physical chunks; load i of the tile's 18 (1152 chunks)
    // is issued by wave i % NW.  A lane's chunk (row, swizzled column) is
    // the same in every tile, so its byte offset is computed once; rows past
    // the live length (last tile only) re-read the last live row, so every
    // staged value is a finite cache value and masked tokens contribute
    // exact zeros.  The page of tile j0 + l is fetched by lane l, 64 tiles at
    // a time, and read back with readlane: no table load in the loop.
    int lrow[LB], lcol[LB];
    uint32_t loff[LB];
#pragma unroll
    for (int k = 0; k < LB; k++) {
        const int pch = 64 * (NW * k + wave) + lane;
        const int r = min(pch / 72, 15);  // (waves that skip load k never use it)
        lrow[k] = r;
        lcol[k] = ((pch - (pch / 72) * 72) ^ mla_swz(r)) * 8;
        loff[k] = (uint32_t)(r * kMlaRow + lcol[k]) * 2;
    }
    const uint32_t ring0 = __builtin_amdgcn_readfirstlane(ring_lds);
    auto fetch_pages = [&](int j0) {
        const int j = j0 + lane;
        return (j < ntiles) ? table[R.tab + (t_begin + 16 * j) / P] : 0;
    };
    int pg = fetch_pages(0);
    auto issue_tile = [&](int j) {
        if ((j & 63) == 0 && j > 0) {
            pg = fetch_pages(j);
            asm volatile("" ::"v"(pg));  // wait for the refill here (rare)
        }
        const int t0 = t_begin + 16 * j;
        const int page = __builtin_amdgcn_readlane(pg, j & 63);
        const uint16_t *src = pool + ((int64_t)page * P + t0 % P) * kMlaRow;
        const uint32_t dst = ring0 + (uint32_t)((j % S) * TILE * 2);
        const int lim = R.len - 1 - t0;  // last live row of the tile
        if (lim >= 15) {
#pragma unroll
            for (int k = 0; k < LB; k++) {
                if (k == LS && wave >= SH::LOADS % NW) break;
                if constexpr (KEEP)
                    lds_dma16_keep(src, loff[k], __builtin_amdgcn_readfirstlane(dst + (uint32_t)(64 * (NW * k + wave)) * 16));
                else
                    lds_dma16(src, loff[k], __builtin_amdgcn_readfirstlane(dst + (uint32_t)(64 * (NW * k + wave)) * 16));
            }
        } else {
#pragma unroll
            for (int k = 0; k < LB; k++) {
                if (k == LS && wave >= SH::LOADS % NW) break;
                const uint32_t off = (uint32_t)(min(lrow[k], lim) * kMlaRow + lcol[k]) * 2;
                if constexpr (KEEP)
                    lds_dma16_keep(src, off, __builtin_amdgcn_readfirstlane(dst + (uint32_t)(64 * (NW * k + wave)) * 16));
                else
                    lds_dma16(src, off, __builtin_amdgcn_readfirstlane(dst + (uint32_t)(64 * (NW * k + wave)) * 16));
            }
        }
    };
    // Wait until this wave's loads of the awaited tile landed, given how many
    // tiles it issued after that one (loads retire in issue order).
    auto wait_tile = [&](int ahead) {
        const bool big = wave < SH::LOADS % NW;
        switch (ahead) {
#define RLX_MLA_WAIT(A)                                        \
    case A:                                                    \
        if (big) RLX_WAIT_VM(A * LB); else RLX_WAIT_VM(A * LS); \
        break;
            RLX_MLA_WAIT(1)
            RLX_MLA_WAIT(2)
            RLX_MLA_WAIT(3)
            RLX_MLA_WAIT(4)
            RLX_MLA_WAIT(5)
#undef RLX_MLA_WAIT
            default: RLX_WAIT_VM(0); break;
        }
    };
    static_assert(S - 3 <= 5, "wait_tile covers at most 5 tiles ahead");

    for (int j = 0; j < S - 1 && j < ntiles; j++) issue_tile(j);

    // Score k-steps (MFMA 16x16x32, 32 channels each): 18 per tile, split
    // over the waves (5/5/4/4 or 3/3/2/2/2/2/2/2).  B operand = q_lat^T, 8
    // channels per lane.
    const int ks0 = wave * KSM + min(wave, 18 % NW);
    const int nks = wave < 18 % NW ? KB : KSM;
    u32x4 qb[NQT][KB];
    int klim[NQT];
#pragma unroll
    for (int nt = 0; nt < NQT; nt++) {
        const int qr = nt * 16 + col;
        klim[nt] = R.len - 1;
#pragma unroll
        for (int kk = 0; kk < KB; kk++) qb[nt][kk] = u32x4{0, 0, 0, 0};
        if (qr < QR) {
            const int qg = R.q0 + qr;
            const int qi = qg / H;
            const int h = qg - qi * H;
            klim[nt] = mla_key_limit(mask_mode, R.len, R.nq, qi);
            const uint16_t *qp = qlat + ((int64_t)(R.qrow + qi) * H + h) * kMlaRow + grp * 8;
#pragma unroll
            for (int kk = 0; kk < KB; kk++)
                if (kk < nks) qb[nt][kk] = *(const u32x4 *)(qp + (ks0 + kk) * 32);
        }
    }

    // Make the compiler complete the q loads here, once: the ring loads are
    // invisible to it, so a wait it placed inside the loop would also drain
    // the ring on every tile.
#pragma unroll
    for (int nt = 0; nt < NQT; nt++)
#pragma unroll
        for (int kk = 0; kk < KB; kk++) asm volatile("" ::"v"(qb[nt][kk]));

    // Partial scores of tile j over this wave's k-steps: A operands read from
    // ring stage j % S, products into sc[nt].
    const int sw = mla_swz(col);
    auto score_reads = [&](int j, u32x4(&a)[KB]) {
        const uint16_t *trow = ring + (j % S) * TILE + col * kMlaRow;
#pragma unroll
        for (int kk = 0; kk < KB; kk++) {
            const int kc = kk < nks ? kk : nks - 1;  // (a wave with fewer k-steps re-reads its last)
            a[kk] = *(const u32x4 *)(trow + ((((ks0 + kc) * 4 + grp) ^ sw) << 3));
        }
    };
    auto score_mfma = [&](const u32x4(&a)[KB], fl4(&sc)[NQT]) {
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            sc[nt] = fl4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KB; kk++)
                if (kk < nks)
                    sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[kk]),
                                                                     __builtin_bit_cast(bf16x8, qb[nt][kk]), sc[nt], 0, 0, 0);
        }
    };
    // P.V operand: 4 consecutive tokens of one channel per lane, from the
    // row-major tile with the LDS transpose read (lane (g, j) fetches 4
    // channels of row 4g + j/4 and the 16-lane group exchanges them so that
    // lane j ends up with channel j of rows 4g..4g+3).
    const int trr = 4 * grp + (col >> 2);
    const int tsw = mla_swz(trr);
    const int tr_off = trr * kMlaRow + (col & 1) * 4;

    // Software pipeline, one barrier per tile: iteration j scores tile j + 1
    // while it runs the softmax and P.V of tile j (whose partial scores were
    // written in iteration j - 1).  The barrier at the top of iteration j
    // publishes tile j + 1 and spart[j & 1], and retires iteration j - 1's
    // reads of ring stage (j - 1) % S (refilled here with tile j + S - 1) and
    // of spart[(j + 1) & 1] (rewritten here).  Ring stages in use: tile j
    // (P.V), tile j + 1 (scores), tiles j + 2 .. j + S - 1 (in flight).
    // Every LDS read of an iteration is issued before its first use, so one
    // wait covers the partial scores, the next tile's score operands and the
    // P.V operands.
    if (ntiles > 0) {
        wait_tile(min(S - 2, ntiles - 1));
        ring_barrier();
        u32x4 a0[KB];
        fl4 sc0[NQT];
        score_reads(0, a0);
        score_mfma(a0, sc0);
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) spart[0][wave][nt][lane] = sc0[nt];
    }
    for (int j = 0; j < ntiles; j++) {
        const bool more = j + 1 < ntiles;
        if (more) wait_tile(min(S - 3, ntiles - 2 - j));
        ring_barrier();
        const int t0 = t_begin + 16 * j;
        const uint16_t *T = ring + (j % S) * TILE;
        fl4 sp[NW][NQT];
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) sp[w][nt] = spart[j & 1][w][nt][lane];
        // (On the last tile stage (j + 1) % S holds a consumed tile and no
        // load in flight: reading it is harmless and its scores are dropped.)
        u32x4 an[KB];
        score_reads(j + 1, an);
        sh4 av[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int lc = (wave * CH + mt * 16) / 8 + ((col >> 1) & 1);
            av[mt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) sh4 *)(T + tr_off + ((lc ^ tsw) << 3)));
        }
        fl4 sn[NQT];
        score_mfma(an, sn);
        sh4 pb[NQT];
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            fl4 sc = sp[0][nt];
#pragma unroll
            for (int w = 1; w < NW; w++) sc += sp[w][nt];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + grp * 4 + i;
                sc[i] = (t <= klim[nt]) ? sc[i] : -INFINITY;
                mx = fmaxf(mx, sc[i]);
            }
            mx = rows4_max(mx);
            const float m_new = fmaxf(m_run[nt], mx);
            // A head that has seen only masked keys keeps m = -inf: its
            // weights and factor come out as exact zeros (acc and l are zero).
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            float p[4];
            const float c = __builtin_amdgcn_exp2f(m_run[nt] - m_use);
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(sc[i] - m_use);
            // The P.V product consumes bf16 weights: normalise by the same ones.
            u32x2 pw;
            pw[0] = pack_bf16x2(p[0], p[1]);
            pw[1] = pack_bf16x2(p[2], p[3]);
            l_part[nt] = add_bf16x2(pw[1], add_bf16x2(pw[0], l_part[nt] * c));
            m_run[nt] = m_new;
            if (__builtin_amdgcn_ballot_w64(c != 1.f)) {  // some head's max moved
#pragma unroll
                for (int mt = 0; mt < MT; mt++) acc[nt][mt] *= c;
            }
            pb[nt] = __builtin_bit_cast(sh4, pw);
        }
        if (more) {
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) spart[(j + 1) & 1][wave][nt][lane] = sn[nt];
        }
        // Refill the stage the barrier released (tile j - 1's) with tile
        // j + S - 1.  Issued here, after the iteration's LDS reads, score
        // products and softmax rather than right after the barrier: a load
        // that stalls on memory back-pressure then holds up only the P.V
        // products (8k: 52.8 -> 52.4 us, 32k: 188.5 -> 185.0 us).
        if (j + S - 1 < ntiles) issue_tile(j + S - 1);
        // O^T += C^T . P^T over this wave's CH latent channels.
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av[mt], pb[nt], acc[nt][mt], 0, 0, 0);
    }

    const int pidx = R.part + wk.y;
    // The unnormalised latent partial is stored as bf16 (the merge weighs
    // and sums it in f32).  A lane's accumulators hold 4 channels of one
    // query row, so stored as they are, each store instruction would write
    // 16 pieces of 32 bytes, 1 KB apart; the wave's 128 channels x 16 rows
    // go through LDS instead (the ring, free once every wave is past its
    // last tile; rows padded by 16 bytes against bank conflicts) and leave
    // as 256 contiguous bytes per query row.
    constexpr int SP = CH + 8;  // staging row pitch, bf16
    static_assert(NW * NQT * 16 * SP <= S * TILE, "the staging rows fit the ring");
    __syncthreads();
    uint16_t *stg = ring + wave * NQT * 16 * SP;
#pragma unroll
    for (int nt = 0; nt < NQT; nt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const u32x2 pk = {pack_bf16x2(acc[nt][mt][0], acc[nt][mt][1]),
                              pack_bf16x2(acc[nt][mt][2], acc[nt][mt][3])};
            *(u32x2 *)(stg + (nt * 16 + col) * SP + mt * 16 + grp * 4) = pk;
        }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NQT; nt++) {
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int r = it * 4 + (lane >> 4), ch = (lane & 15) * 8;
            const u32x4 v = *(const u32x4 *)(stg + (nt * 16 + r) * SP + ch);
            __builtin_nontemporal_store(
                v, (u32x4 *)(part_o + ((int64_t)pidx * QRP + nt * 16 + r) * kMlaDc + wave * CH + ch));
        }
        const int qr = nt * 16 + col;
        const float lt = rows4_sum(l_part[nt]);
        if (wave == 0 && grp == 0) {
            float *pm = part_ml + ((int64_t)pidx * QRP + qr) * 2;
            pm[0] = m_run[nt];
            pm[1] = lt;
        }
    }
}

// Row of the call that holds global query row q: binary search on the
// rows' first query rows (field qrow), from the arguments or the device.
template <bool ARG>
__device__ __forceinline__ int plan_qrow_row(const AttRow *rows, int n_rows, int q) {
    int lo = 0, hi = n_rows - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        int first;
        if constexpr (ARG) {
            const __attribute__((address_space(4))) int32_t *p =
                (const __attribute__((address_space(4))) int32_t *)kernarg_plan();
            first = p[mid * 8 + 3];
        } else {
            first = rows[mid].qrow;
        }
        if (first <= q)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Plan row holding head h of global query row q: the sequence's row (found
// by its first query row), or -- when the sequence's H x nq query rows were
// cut into head groups of QRP rows, consecutive plan rows of one sequence --
// the group that holds row (q - qrow) H + h.
template <bool ARG>
__device__ __forceinline__ AttRow mla_group_row(const AttRow *rows, int n_rows, int one_q, int q, int h,
                                               int H, int QRP) {
    const int ri = one_q ? q : plan_qrow_row<ARG>(rows, n_rows, q);  // the sequence's last plan row
    const AttRow R = plan_row<ARG>(rows, ri);
    const int all = H * R.nq;
    if (R.qn >= all) return R;
    const int groups = (all + QRP - 1) / QRP;
    return plan_row<ARG>(rows, ri - (groups - 1) + ((q - R.qrow) * H + h) / QRP);
}

// The step after the split loop, for head h and RPB consecutive query rows
// of the call: merge each query row's split partials into the normalised
// latent output
//   o_lat = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s     (512 channels)
// and project it, out[d] = sum_c o_lat[c] * W_UV[c][h*D + d] (mla.go:384-389
// applies W_UV to P.V; here it applies to the merged latent, the same sum
// by linearity).  The RPB rows share one read of the head's W_UV slice.
// D (the head dim, a multiple of 8 up to DMAX) and d_c are runtime values:
// octets past D and channels past d_c take no part.
// Every global load is issued at the start, so the block costs one memory
// round trip: thread t loads channels 2t, 2t+1 (bf16 pair) of up to 16
// splits per row, and -- as thread (g, o) of G channel groups x D/8 dim
// octets -- 8 consecutive W_UV dims of each of its group's first WB
// channels (16 B per load).  Wave j computes row j's merge weights in LDS,
// o_lat goes to LDS, each thread accumulates its 8 dims over its channels
// with f32 FMAs of the exactly widened bf16 weights, and the groups are
// summed in LDS.
template <int DMAX>
struct MlaOutShape {
    static constexpr int OCT = DMAX / 8;                           // dim octets
    static constexpr int G = (256 / OCT >= 32) ? 32 : (256 / OCT >= 16) ? 16 : 8;  // channel groups
    static constexpr int CPG = kMlaDc / G;                         // channels per group
    static constexpr int WB = CPG < 32 ? CPG : (DMAX >= 192 ? 16 : 32);  // weight rows loaded up front
};

template <int DMAX, int RPB, bool ARG>
__global__ __launch_bounds__(256) void mla_out_kernel(
    typename PlanSel<ARG>::T plan, const AttRow *__restrict__ rows, int n_rows, int total_q, int one_q,
    const uint16_t *__restrict__ part_o, const float *__restrict__ part_ml,
    const uint16_t *__restrict__ w_uv, int H, int D, int dc, int QRP, void *__restrict__ out,
    int out_bf16) {
    using SH = MlaOutShape<DMAX>;
    constexpr int SB = 16;  // splits per batch of loads
    constexpr int OCT = SH::OCT, G = SH::G, CPG = SH::CPG, WB = SH::WB;
    static_assert(G * CPG == kMlaDc && G * OCT <= 256, "groups x octets must fit the block");
    static_assert(RPB <= 4, "one wave computes each row's merge weights");
    const int h = blockIdx.x;
    const int q0 = blockIdx.y * RPB;
    __shared__ float fac[RPB][kMaxSplits];
    __shared__ float inv_l[RPB];
    __shared__ float olat[RPB][kMlaDc];
    __shared__ float red[G][RPB][DMAX];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = t / OCT, o = t - g * OCT;
    const bool wt = g < G && o * 8 < D;  // thread takes part in the projection
    // The block's query rows: row (sequence) of the call, query index, first
    // partial (query row qr of slot part), splits.
    int64_t b0[RPB];
    int ns[RPB];
    int64_t ob[RPB];
    bool live[RPB];
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const int q = min(q0 + j, total_q - 1);
        live[j] = q0 + j < total_q;
        // one query per row (decode): query row q is row q
        const AttRow R = mla_group_row<ARG>(rows, n_rows, one_q, q, h, H, QRP);
        b0[j] = (int64_t)R.part * QRP + (q - R.qrow) * H + h - R.q0;
        ns[j] = R.nsplit;
        ob[j] = ((int64_t)q * H + h) * D;
    }
    // Loads, in the order their values are needed (the memory counter
    // retires them in issue order, so each wait covers only what it needs):
    // (m, l) of split `lane` of row `wave` (waves < RPB), then the split
    // partials, then the W_UV rows.  None is predicated: clamped addresses
    // keep every load in bounds, so no load sits behind a branch.
    int64_t bw = b0[0];
    int nw = ns[0];
#pragma unroll
    for (int j = 1; j < RPB; j++)
        if (wave == j) {
            bw = b0[j];
            nw = ns[j];
        }
    const float2 *ml = (const float2 *)(part_ml + bw * 2);
    const int64_t st = QRP;  // float2 between split slots
    float2 ml0 = make_float2(-INFINITY, 0.f);
    if (wave < RPB) ml0 = ml[min(lane, nw - 1) * st];
    const int64_t sstride = (int64_t)QRP * kMlaDc;  // bf16 between split slots
    uint32_t v[RPB][SB];
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const uint16_t *src = part_o + b0[j] * kMlaDc + 2 * t;
#pragma unroll
        for (int i = 0; i < SB; i++) v[j][i] = *(const uint32_t *)(src + (int64_t)min(i, ns[j] - 1) * sstride);
    }
    // W_UV rows cb + k (< d_c), dims h*D + 8 o .. + 8.  Rows past d_c read
    // row d_c - 1 instead: their latent channels are zero in every cached
    // row, so o_lat is exactly 0 there and the product adds nothing.
    const int cb = (g < G ? g : 0) * CPG;
    const uint16_t *wp = w_uv + (int64_t)h * D + (wt ? o * 8 : 0);
    const int64_t wstride = (int64_t)H * D;
    u32x4 w[WB];
#pragma unroll
    for (int k = 0; k < WB; k++) w[k] = *(const u32x4 *)(wp + (int64_t)min(cb + k, dc - 1) * wstride);
    // merge weights of row j by wave j: fac = 2^(m_s - M), inv_l = 1 / sum fac l
    if (wave < RPB) {
        const int j = wave;
        if (lane >= nw) ml0 = make_float2(-INFINITY, 0.f);
        float M = ml0.x;
        for (int s0 = lane + 64; s0 < nw; s0 += 64) M = fmaxf(M, ml[s0 * st].x);
#pragma unroll
        for (int k = 32; k > 0; k >>= 1) M = fmaxf(M, __shfl_xor(M, k));
        float L = 0.f;
        if (lane < nw) {
            const float f = (ml0.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ml0.x - M);
            fac[j][lane] = f;
            L = f * ml0.y;
        }
        for (int s0 = lane + 64; s0 < nw; s0 += 64) {
            const float2 e = ml[s0 * st];
            const float f = (e.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(e.x - M);
            fac[j][s0] = f;
            L += f * e.y;
        }
#pragma unroll
        for (int k = 32; k > 0; k >>= 1) L += __shfl_xor(L, k);
        if (lane == 0) inv_l[j] = (L > 0.f) ? 1.f / L : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const uint16_t *src = part_o + b0[j] * kMlaDc + 2 * t;
        float o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int i = 0; i < SB; i++) {
            if (i < ns[j]) {
                o0 += fac[j][i] * bf16_lo(v[j][i]);
                o1 += fac[j][i] * bf16_hi(v[j][i]);
            }
        }
        for (int s0 = SB; s0 < ns[j]; s0 += SB) {
#pragma unroll
            for (int i = 0; i < SB; i++) v[j][i] = *(const uint32_t *)(src + (int64_t)min(s0 + i, ns[j] - 1) * sstride);
#pragma unroll
            for (int i = 0; i < SB; i++) {
                if (s0 + i < ns[j]) {
                    o0 += fac[j][s0 + i] * bf16_lo(v[j][i]);
                    o1 += fac[j][s0 + i] * bf16_hi(v[j][i]);
                }
            }
        }
        olat[j][2 * t] = o0 * inv_l[j];
        olat[j][2 * t + 1] = o1 * inv_l[j];
    }
    __syncthreads();
    float a[RPB][8];
#pragma unroll
    for (int j = 0; j < RPB; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) a[j][i] = 0.f;
    auto fma8 = [&](const u32x4 &wv, int c) {
#pragma unroll
        for (int j = 0; j < RPB; j++) {
            const float x = olat[j][c];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[j][2 * i] += x * bf16_lo(wv[i]);
                a[j][2 * i + 1] += x * bf16_hi(wv[i]);
            }
        }
    };
#pragma unroll
    for (int k = 0; k < WB; k++) fma8(w[k], cb + k);
    for (int k0 = WB; k0 < CPG; k0 += WB) {
#pragma unroll
        for (int k = 0; k < WB; k++) w[k] = *(const u32x4 *)(wp + (int64_t)min(cb + k0 + k, dc - 1) * wstride);
#pragma unroll
        for (int k = 0; k < WB; k++) fma8(w[k], cb + k0 + k);
    }
    if (wt) {
#pragma unroll
        for (int j = 0; j < RPB; j++)
#pragma unroll
            for (int i = 0; i < 8; i++) red[g][j][o * 8 + i] = a[j][i];
    }
    __syncthreads();
    if (t < D) {
#pragma unroll
        for (int j = 0; j < RPB; j++) {
            if (!live[j]) continue;
            float val = red[0][j][t];
#pragma unroll
            for (int k = 1; k < G; k++) val += red[k][j][t];
            if (out_bf16)
                ((uint16_t *)out)[ob[j] + t] = bf16_rne(val);
            else
                ((float *)out)[ob[j] + t] = val;
        }
    }
}

// The same step for head dim 128 with the projection on the matrix cores.
// Block = (head h, RPB query rows), 4 waves; wave w produces output dims
// [32w, 32w + 32) of the block's rows:
//   out[r][d] = sum_c o_lat[r][c] W_UV[c][h*128 + d]
// as MFMA 16x16x16 bf16 tiles D[16][16 dims] over the 512 channels.  A rows
// hold the merged latent as an exact-sum bf16 pair: row 2r = hi(o_lat[r]),
// row 2r + 1 = lo = bf16(o_lat[r] - hi), so one product covers both halves
// and out[r] = D[2r] + D[2r + 1] keeps the f32 latent to ~2^-17 relative
// (bf16 products are exact in f32).  The B operand needs 4 consecutive
// channels of one dim per lane while W_UV rows are dim-contiguous: the
// block copies the head's [512 ch][128 dims] slice into LDS (whole 256-byte
// rows per 16 lanes, so every 128-byte line is requested once; 32-byte
// chunk c of channel r at slot c ^ (r & 7), so a transpose read of 32
// lanes touches every bank once) and each wave reads its operands with the
// LDS transpose read.  Loads are issued as in mla_out_kernel:
// (m, l) pairs, the split partials, then the W_UV slice (into registers);
// the slice goes to LDS after the merge, so the merge waits only for the
// partials.
template <int RPB, bool ARG>
__global__ __launch_bounds__(256) void mla_out_mfma_kernel(
    typename PlanSel<ARG>::T plan, const AttRow *__restrict__ rows, int n_rows, int total_q, int one_q,
    const uint16_t *__restrict__ part_o, const float *__restrict__ part_ml,
    const uint16_t *__restrict__ w_uv, int H, int dc, int QRP, void *__restrict__ out, int out_bf16) {
    constexpr int D = 128;                     // head dim
    constexpr int WD = D / 4;                  // output dims per wave
    constexpr int WL = kMlaDc * D / 8 / 256;   // 16-byte slice loads per lane (32)
    constexpr int SB = 16;                     // splits per batch of loads
    constexpr int OP = kMlaDc / 2 + 8;         // o_lat row pitch in bf16 pairs (32 B pad)
    static_assert(2 * RPB <= 16, "the hi and lo rows fill at most one MFMA tile");
    static_assert(RPB <= 4, "one wave computes each row's merge weights");
    const int h = blockIdx.x;
    const int q0 = blockIdx.y * RPB;
    __shared__ __attribute__((aligned(16))) uint16_t wsl[kMlaDc * D];
    __shared__ __attribute__((aligned(16))) float fac[RPB][kMaxSplits];
    __shared__ float inv_l[RPB];
    __shared__ __attribute__((aligned(16))) uint32_t olat[2 * RPB][OP];  // row 2r + s: s = 0 hi, 1 lo
    const int t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    int64_t b0[RPB];
    int ns[RPB];
    int64_t ob[RPB];
    bool live[RPB];
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const int q = min(q0 + j, total_q - 1);
        live[j] = q0 + j < total_q;
        const AttRow R = mla_group_row<ARG>(rows, n_rows, one_q, q, h, H, QRP);
        b0[j] = (int64_t)R.part * QRP + (q - R.qrow) * H + h - R.q0;
        ns[j] = R.nsplit;
        ob[j] = ((int64_t)q * H + h) * D;
    }
    int64_t bw = b0[0];
    int nw = ns[0];
#pragma unroll
    for (int j = 1; j < RPB; j++)
        if (wave == j) {
            bw = b0[j];
            nw = ns[j];
        }
    const float2 *ml = (const float2 *)(part_ml + bw * 2);
    const int64_t st = QRP;
    float2 ml0 = make_float2(-INFINITY, 0.f);
    if (wave < RPB) ml0 = ml[min(lane, nw - 1) * st];
    const int64_t sstride = (int64_t)QRP * kMlaDc;
    uint32_t v[RPB][SB];
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const uint16_t *src = part_o + b0[j] * kMlaDc + 2 * t;
#pragma unroll
        for (int i = 0; i < SB; i++) v[j][i] = *(const uint32_t *)(src + (int64_t)min(i, ns[j] - 1) * sstride);
    }
    // Slice load k of this lane: channel 128 wave + 4k + lane / 16,
    // 16-byte chunk lane % 16 of the head's 128 dims.  Channels past d_c
    // read channel d_c - 1: o_lat is exactly 0 there, so they add nothing.
    const int wc0 = 128 * wave + (lane >> 4);
    const uint16_t *wp = w_uv + (int64_t)h * D + (lane & 15) * 8;
    const int64_t wstride = (int64_t)H * D;
    u32x4 w[WL];
#pragma unroll
    for (int k = 0; k < WL; k++) w[k] = *(const u32x4 *)(wp + (int64_t)min(wc0 + 4 * k, dc - 1) * wstride);
    // Merge weights of row j by wave j, as in mla_out_kernel, except that
    // fac is written as 0 past the row's splits up to a multiple of SB: the
    // merge then reads whole float4s of weights with no per-split test
    // (the partials it pairs them with are finite clamped loads).
    if (wave < RPB) {
        const int j = wave;
        const int nz = (nw + SB - 1) / SB * SB;
        if (lane >= nw) ml0 = make_float2(-INFINITY, 0.f);
        float M = ml0.x;
        for (int s0 = lane + 64; s0 < nw; s0 += 64) M = fmaxf(M, ml[s0 * st].x);
#pragma unroll
        for (int k = 32; k > 0; k >>= 1) M = fmaxf(M, __shfl_xor(M, k));
        float L = 0.f;
        {
            const float f = (ml0.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ml0.x - M);
            fac[j][lane] = f;
            L = f * ml0.y;
        }
        for (int s0 = lane + 64; s0 < nz; s0 += 64) {
            float f = 0.f;
            if (s0 < nw) {
                const float2 e = ml[s0 * st];
                f = (e.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(e.x - M);
                L += f * e.y;
            }
            fac[j][s0] = f;
        }
#pragma unroll
        for (int k = 32; k > 0; k >>= 1) L += __shfl_xor(L, k);
        if (lane == 0) inv_l[j] = (L > 0.f) ? 1.f / L : 0.f;
    }
    ring_barrier();  // fac, inv_l (the slice loads stay in flight)
    auto merge_batch = [&](int j, int s0, float &o0, float &o1) {
        const float4 *fp = (const float4 *)&fac[j][s0];
        float4 f4[SB / 4];
#pragma unroll
        for (int u = 0; u < SB / 4; u++) f4[u] = fp[u];
#pragma unroll
        for (int i = 0; i < SB; i++) {
            const float f = f4[i / 4][i % 4];
            o0 += f * bf16_lo(v[j][i]);
            o1 += f * bf16_hi(v[j][i]);
        }
    };
#pragma unroll
    for (int j = 0; j < RPB; j++) {
        const uint16_t *src = part_o + b0[j] * kMlaDc + 2 * t;
        float o0 = 0.f, o1 = 0.f;
        merge_batch(j, 0, o0, o1);
        for (int s0 = SB; s0 < ns[j]; s0 += SB) {
#pragma unroll
            for (int i = 0; i < SB; i++) v[j][i] = *(const uint32_t *)(src + (int64_t)min(s0 + i, ns[j] - 1) * sstride);
            merge_batch(j, s0, o0, o1);
        }
        uint16_t h0, l0, h1, l1;
        split_bf16(o0 * inv_l[j], h0, l0);
        split_bf16(o1 * inv_l[j], h1, l1);
        olat[2 * j][t] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        olat[2 * j + 1][t] = (uint32_t)l0 | ((uint32_t)l1 << 16);
    }
    // The slice goes to LDS only now (the compiler would otherwise hoist
    // these stores, and their waits for the slice loads, above the merge).
    asm volatile("" ::: "memory");
    // channel wc0 + 4k: (r & 7) = 4 (k & 1) + lane / 16
#pragma unroll
    for (int k = 0; k < WL; k++) {
        const int q = lane & 15, sw = ((k & 1) << 2) | (lane >> 4);
        *(u32x4 *)(wsl + (wc0 + 4 * k) * D + ((((q >> 1) ^ sw) << 1 | (q & 1)) << 3)) = w[k];
    }
    ring_barrier();  // o_lat of every row; the slice
    // A: row m = lane % 16 (2r + s), channels 16 ks + 4 g .. + 4 (g = lane / 16).
    // B (transpose read): lane i of group g fetches dims 4 (i % 4) .. + 4 of
    // the 16-dim tile, channel 16 ks + 4 g + i / 4; lane j ends up with dim
    // j of the group's 4 channels.  That channel has (r & 7) = 4 (g & 1) + i / 4.
    const int m = lane & 15, g = lane >> 4;
    const bool arow = m < 2 * RPB;
    const uint32_t *ap = &olat[arow ? m : 0][2 * g];
    const int rsw = ((g & 1) << 2) | (m >> 2);
    const uint16_t *bp = wsl + (4 * g + (m >> 2)) * D + 4 * (m & 3);
    // Operands of KB k-steps are read before their products, so the LDS
    // round trips overlap instead of one per k-step.
    constexpr int KB = 8;
    fl4 acc[2] = {fl4{0.f, 0.f, 0.f, 0.f}, fl4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int k0 = 0; k0 < kMlaDc / 16; k0 += KB) {
        sh4 av[KB], bv[KB][2];
#pragma unroll
        for (int u = 0; u < KB; u++) {
            u32x2 a2 = u32x2{0u, 0u};
            if (arow) a2 = *(const u32x2 *)(ap + 8 * (k0 + u));
            av[u] = __builtin_bit_cast(sh4, a2);
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                bv[u][nt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) sh4 *)(bp + (k0 + u) * 16 * D + (((2 * wave + nt) ^ rsw) << 4)));
        }
#pragma unroll
        for (int u = 0; u < KB; u++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av[u], bv[u][nt], acc[nt], 0, 0, 0);
    }
    // acc[nt][i] = D[4g + i][dim 16 nt + m]: rows 2g (i = 0, 1) and 2g + 1 (i = 2, 3).
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int d = wave * WD + nt * 16 + m;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int r = 2 * g + u;
#pragma unroll
            for (int j = 0; j < RPB; j++) {
                if (j != r || !live[j]) continue;
                const float val = acc[nt][2 * u] + acc[nt][2 * u + 1];
                if (out_bf16)
                    ((uint16_t *)out)[ob[j] + d] = bf16_rne(val);
                else
                    ((float *)out)[ob[j] + d] = val;
            }
        }
    }
}

template <int NQT, bool ARG>
static void launch_mla_t(hipStream_t s, bool keep, typename PlanSel<ARG>::T plan, const uint16_t *pool,
                         const int32_t *table, const AttRow *rows, int n_rows, const int2 *work,
                         int n_work, const uint16_t *qlat, int H, int P, int mask_mode,
                         uint16_t *part_o, float *part_ml, hipEvent_t ev0, hipEvent_t ev1) {
    (void)launch_timed(keep ? mla_decode_kernel<NQT, ARG, true> : mla_decode_kernel<NQT, ARG, false>,
                       dim3(n_work), dim3(64 * MlaShape<NQT>::NW), s,
                       ev0, ev1, plan, pool, table, rows, work, n_rows, qlat, H, P, mask_mode,
                       part_o, part_ml);
}

template <int DMAX, bool ARG>
static void launch_mla_out_d(hipStream_t s, typename PlanSel<ARG>::T plan, const AttRow *rows,
                             int n_rows, int total_q, int one_q, const uint16_t *part_o, const float *part_ml,
                             const uint16_t *w_uv, int H, int D, int dc, int QRP, void *out,
                             int out_bf16, int cus) {
    // Two query rows per block share the W_UV read when that still leaves a
    // block per CU.
    if ((int64_t)H * ((total_q + 1) / 2) >= cus)
        mla_out_kernel<DMAX, 2, ARG><<<dim3(H, (total_q + 1) / 2), 256, 0, s>>>(
            plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, D, dc, QRP, out,
            out_bf16);
    else
        mla_out_kernel<DMAX, 1, ARG><<<dim3(H, total_q), 256, 0, s>>>(
            plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, D, dc, QRP, out,
            out_bf16);
}

template <bool ARG>
static void launch_mla_out(hipStream_t s, typename PlanSel<ARG>::T plan, const AttRow *rows,
                           int n_rows, int total_q, int one_q, const uint16_t *part_o, const float *part_ml,
                           const uint16_t *w_uv, int H, int hd, int dc, int QRP, void *out,
                           int out_bf16, int cus) {
    // Rows per block: the most (4, 2, 1) that still give every CU a block;
    // each block reads the head's whole W_UV slice, so fewer blocks read
    // less of it.  Measured (MLA 8k steps, ms): 16 heads x 32 rows 0.0694 /
    // 0.0655 / 0.0668 at 1 / 2 / 4; 128 heads x 8 rows 0.0964 / 0.0888 /
    // 0.0855.  RLX_MLA_OUT_RPB (1, 2 or 4) overrides the choice (tuning).
    static const int rpb_override = [] {
        const char *e = getenv("RLX_MLA_OUT_RPB");
        const int x = e ? atoi(e) : 0;
        return (x == 1 || x == 2 || x == 4) ? x : 0;
    }();
    if (hd == 128) {
        int rpb = rpb_override;
        if (!rpb)
            rpb = (int64_t)H * ((total_q + 3) / 4) >= cus   ? 4
                  : (int64_t)H * ((total_q + 1) / 2) >= cus ? 2
                                                            : 1;
        if (rpb == 4)
            mla_out_mfma_kernel<4, ARG><<<dim3(H, (total_q + 3) / 4), 256, 0, s>>>(
                plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, dc, QRP,
                out, out_bf16);
        else if (rpb == 2)
            mla_out_mfma_kernel<2, ARG><<<dim3(H, (total_q + 1) / 2), 256, 0, s>>>(
                plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, dc, QRP,
                out, out_bf16);
        else
            mla_out_mfma_kernel<1, ARG><<<dim3(H, total_q), 256, 0, s>>>(
                plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, dc, QRP,
                out, out_bf16);
    } else if (hd <= 32)
        launch_mla_out_d<32, ARG>(s, plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc, QRP, out, out_bf16, cus);
    else if (hd <= 64)
        launch_mla_out_d<64, ARG>(s, plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc, QRP, out, out_bf16, cus);
    else if (hd <= 128)
        launch_mla_out_d<128, ARG>(s, plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc, QRP, out, out_bf16, cus);
    else
        launch_mla_out_d<256, ARG>(s, plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc, QRP, out, out_bf16, cus);
}

hipError_t launch_mla_decode(hipStream_t s, const PlanArg *plan, const uint16_t *pool,
                             const int32_t *table, const AttRow *rows, int n_rows,
                             const int2 *work, int n_work,
                             const void *q_nope, const void *q_rope, int q_bf16,
                             const uint16_t *w_uk, const uint16_t *w_uv, int H, int hd, int dc,
                             int dr, int total_q, int max_nq, int P, float qscale,
                             int mask_mode, int nqt, uint16_t *qlat, uint16_t *part_o,
                             float *part_ml, void *out, int out_bf16, int cus,
                             hipEvent_t ev0, hipEvent_t ev1, const MlaAppendJob *app) {
    if (n_work <= 0) return hipSuccess;
    if (hd > 256 || hd % 8 != 0 || dc > kMlaDc || dr > kMlaDr) return hipErrorInvalidValue;
    const int nz = (total_q + 15) / 16;
    const dim3 ag(H, kMlaDc / 64, nz);
    if (app && (app->n_tok > 0 || app->n_patch > 0)) {
        // absorb + the step's append: one launch
        const int64_t aw = std::max<int64_t>((int64_t)app->n_tok * (kMlaRow / 8), app->n_patch);
        const dim3 fg((unsigned)(H * (kMlaDc / 64) * nz + (aw + 255) / 256));
        switch ((hd + 31) / 32) {
#define RLX_ABSORB_APP(KS)                                                                          \
    case KS:                                                                                        \
        if (app->plan)                                                                              \
            mla_absorb_append_kernel<KS, true><<<fg, 256, 0, s>>>(                                  \
                *app->plan, q_nope, q_rope, q_bf16, w_uk, H, hd, dc, dr, total_q, qscale, qlat, nz, \
                app->pool, app->table, app->patches, app->n_patch, app->toks, app->tok_off,         \
                app->n_tok, app->c_src, app->kr_src, app->src_bf16, app->P);                        \
        else                                                                                        \
            mla_absorb_append_kernel<KS, false><<<fg, 256, 0, s>>>(                                 \
                NoPlan{0}, q_nope, q_rope, q_bf16, w_uk, H, hd, dc, dr, total_q, qscale, qlat, nz,  \
                app->pool, app->table, app->patches, app->n_patch, app->toks, app->tok_off,         \
                app->n_tok, app->c_src, app->kr_src, app->src_bf16, app->P);                        \
        break;
            RLX_ABSORB_APP(1) RLX_ABSORB_APP(2) RLX_ABSORB_APP(3) RLX_ABSORB_APP(4)
            RLX_ABSORB_APP(5) RLX_ABSORB_APP(6) RLX_ABSORB_APP(7) RLX_ABSORB_APP(8)
#undef RLX_ABSORB_APP
            default: return hipErrorInvalidValue;
        }
    } else {
        switch ((hd + 31) / 32) {
#define RLX_ABSORB(KS) \
    case KS: mla_absorb_kernel<KS><<<ag, 256, 0, s>>>(q_nope, q_rope, q_bf16, w_uk, H, hd, dc, dr, total_q, qscale, qlat); break;
            RLX_ABSORB(1) RLX_ABSORB(2) RLX_ABSORB(3) RLX_ABSORB(4)
            RLX_ABSORB(5) RLX_ABSORB(6) RLX_ABSORB(7) RLX_ABSORB(8)
#undef RLX_ABSORB
            default: return hipErrorInvalidValue;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (nqt != 1 && nqt != 2) return hipErrorInvalidValue;
    // head groups (some sequence's H x nq rows past one work-group's) re-read
    // latent rows: keep them in L2
    const bool keep = H * max_nq > 16 * nqt;
    if (plan && nqt == 1)
        launch_mla_t<1, true>(s, keep, *plan, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                              mask_mode, part_o, part_ml, ev0, ev1);
    else if (plan)
        launch_mla_t<2, true>(s, keep, *plan, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                              mask_mode, part_o, part_ml, ev0, ev1);
    else if (nqt == 1)
        launch_mla_t<1, false>(s, keep, NoPlan{0}, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                               mask_mode, part_o, part_ml, ev0, ev1);
    else
        launch_mla_t<2, false>(s, keep, NoPlan{0}, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                               mask_mode, part_o, part_ml, ev0, ev1);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Query row q is plan row q only when every sequence has one query and
    // one plan row (no head groups).
    const int one_q = total_q == n_rows && max_nq == 1;
    if (plan)
        launch_mla_out<true>(s, *plan, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc,
                             16 * nqt, out, out_bf16, cus);
    else
        launch_mla_out<false>(s, NoPlan{0}, rows, n_rows, total_q, one_q, part_o, part_ml, w_uv, H, hd, dc,
                              16 * nqt, out, out_bf16, cus);
    return hipGetLastError();
}

int mla_decode_wgs_per_cu(int nqt) {
    int n = 0;
    hipError_t e = hipErrorInvalidValue;
    if (nqt == 1) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mla_decode_kernel<1, true, false>, 64 * MlaShape<1>::NW, 0);
    if (nqt == 2) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mla_decode_kernel<2, true, false>, 64 * MlaShape<2>::NW, 0);
    return (e == hipSuccess && n > 0) ? n : 1;
}

}  // namespace rlx
