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
// for c < 512 and q_lat[row][h][512+r] = bf16(qscale * q_rope[row][h][r]).
// Block = (head, 64 latent channels, 16 query rows); wave w computes
// C[16 channels][16 rows] = W_UK_h[c0+16w .., :] . q^T with MFMA 16x16x32
// over the head's D dims: A = 8 consecutive W_UK dims of one channel per
// lane, B = 8 consecutive query dims of one row per lane (f32 queries as
// hi + lo bf16 pairs).  Every load is issued before the first product, so
// the kernel costs one memory round trip.
template <int D>
__global__ __launch_bounds__(256) void mla_absorb_kernel(const void *__restrict__ q_nope,
                                                         const void *__restrict__ q_rope,
                                                         int q_bf16,
                                                         const uint16_t *__restrict__ w_uk,
                                                         int H, int total_q, float qscale,
                                                         uint16_t *__restrict__ qlat) {
    constexpr int KS = D / 32;
    const int h = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int c0 = blockIdx.y * 64 + wave * 16;
    const int r0 = blockIdx.z * 16;
    const int row = min(r0 + col, total_q - 1);  // rows past the end load the last row
    const uint16_t *wa = w_uk + (int64_t)(c0 + col) * H * D + (int64_t)h * D + grp * 8;
    u32x4 a[KS], bh[KS], bl[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) a[ks] = *(const u32x4 *)(wa + ks * 32);
    const int64_t qoff = ((int64_t)row * H + h) * D + grp * 8;
    if (q_bf16) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            bh[ks] = *(const u32x4 *)((const uint16_t *)q_nope + qoff + ks * 32);
            bl[ks] = u32x4{0, 0, 0, 0};
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float *qf = (const float *)q_nope + qoff + ks * 32;
            const float4 f0 = *(const float4 *)qf, f1 = *(const float4 *)(qf + 4);
            const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
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
    if (blockIdx.y == 0) {
        for (int i = threadIdx.x; i < 16 * kMlaDr; i += blockDim.x) {
            const int r = i / kMlaDr, k = i - r * kMlaDr;
            if (r0 + r >= total_q) continue;
            const int64_t off = ((int64_t)(r0 + r) * H + h) * kMlaDr + k;
            const float x = q_bf16 ? bf16_f32(((const uint16_t *)q_rope)[off]) : ((const float *)q_rope)[off];
            qlat[((int64_t)(r0 + r) * H + h) * kMlaRow + kMlaDc + k] = bf16_rne(x * qscale);
        }
    }
}

// LDS tile layout: 16 token rows x 72 chunks of 16 B (576 bf16), no padding.
// Logical chunk c of row r lives at physical chunk c ^ mla_swz(r), which
// stays inside the row's aligned group of 8 chunks.  The swizzle keeps the
// two read patterns free of bank conflicts: score reads (8 lanes = 8 rows,
// one chunk each) see 8 distinct chunk slots, and transpose reads (16 lanes
// = 4 rows x one 32-B chunk pair) see 4 distinct chunk pairs.
__device__ __forceinline__ int mla_swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// Shape per query-row tile count: 4 waves and two work-groups per CU (80 KB
// of LDS each); a 4-stage ring for up to 16 query rows, 3 stages for 32.
template <int NQT> struct MlaShape {
    static constexpr int NW = 4;                      // waves
    static constexpr int S = NQT == 1 ? 4 : 3;        // LDS ring stages
    static constexpr int WGS = 2;                     // resident work-groups per CU
    static constexpr int LOADS = 16 * kMlaRow / 8 / 64;  // 64-lane loads per tile (18)
    static constexpr int CH = kMlaDc / NW;            // latent channels per wave
};

template <int NQT, bool ARG>
__global__ __launch_bounds__(64 * MlaShape<NQT>::NW, MlaShape<NQT>::WGS) void mla_decode_kernel(
    typename PlanSel<ARG>::T plan, const uint16_t *__restrict__ pool,
    const int32_t *__restrict__ table, const AttRow *__restrict__ rows,
    const int2 *__restrict__ work, int n_rows, const uint16_t *__restrict__ qlat, int H, int P,
    int chunk, int mask_mode, float *__restrict__ part_o, float *__restrict__ part_ml) {
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
    const int QR = H * R.nq;
    const int t_begin = wk.y * chunk;
    const int t_end = min(R.len, t_begin + chunk);
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
                lds_dma16(src, loff[k], __builtin_amdgcn_readfirstlane(dst + (uint32_t)(64 * (NW * k + wave)) * 16));
            }
        } else {
#pragma unroll
            for (int k = 0; k < LB; k++) {
                if (k == LS && wave >= SH::LOADS % NW) break;
                const uint32_t off = (uint32_t)(min(lrow[k], lim) * kMlaRow + lcol[k]) * 2;
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
            const int qi = qr / H;
            const int h = qr - qi * H;
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
        if (j + S - 1 < ntiles) issue_tile(j + S - 1);
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
        // O^T += C^T . P^T over this wave's CH latent channels.
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av[mt], pb[nt], acc[nt][mt], 0, 0, 0);
    }

    const int pidx = R.part + wk.y;
#pragma unroll
    for (int nt = 0; nt < NQT; nt++) {
        const int qr = nt * 16 + col;
        const float lt = rows4_sum(l_part[nt]);
        float *po = part_o + ((int64_t)pidx * QRP + qr) * kMlaDc + wave * CH;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) __builtin_nontemporal_store(acc[nt][mt], (fl4 *)(po + mt * 16 + grp * 4));
        if (wave == 0 && grp == 0) {
            float *pm = part_ml + ((int64_t)pidx * QRP + qr) * 2;
            pm[0] = m_run[nt];
            pm[1] = lt;
        }
    }
}

// Merge the splits of one (sequence, query, head) into the normalised latent
// output o_lat[row][h][0:512] (f32 workspace).  One 256-thread block per
// query row; each thread owns channels t and t + 256 and loads them from up
// to 16 splits at once (issued before the merge weights are read, so the two
// round trips overlap); wave 0 computes the merge weights in LDS.
template <bool ARG>
__global__ __launch_bounds__(256) void mla_combine_kernel(
    typename PlanSel<ARG>::T plan, const AttRow *__restrict__ rows,
    const float *__restrict__ part_o, const float *__restrict__ part_ml, int H, int QRP,
    float *__restrict__ olat) {
    constexpr int SB = 16;  // splits per batch of loads
    const AttRow R = plan_row<ARG>(rows, blockIdx.x);
    const int qi = blockIdx.y / H;
    const int h = blockIdx.y - qi * H;
    if (qi >= R.nq) return;
    const int qr = qi * H + h;
    __shared__ float fac[kMaxSplits];
    __shared__ float inv_l;
    const int64_t b0 = (int64_t)R.part * QRP + qr;
    const int c = threadIdx.x;
    const float *src = part_o + b0 * kMlaDc + c;
    const int64_t sstride = (int64_t)QRP * kMlaDc;
    float v0[SB], v1[SB];
#pragma unroll
    for (int i = 0; i < SB; i++) {
        const int64_t o = (int64_t)min(i, R.nsplit - 1) * sstride;
        v0[i] = src[o];
        v1[i] = src[o + 256];
    }
    merge_weights(part_ml + b0 * 2, QRP, R.nsplit, fac, &inv_l);
    __syncthreads();
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int i = 0; i < SB; i++) {
        if (i < R.nsplit) {
            o0 += fac[i] * v0[i];
            o1 += fac[i] * v1[i];
        }
    }
    for (int s0 = SB; s0 < R.nsplit; s0 += SB) {
#pragma unroll
        for (int i = 0; i < SB; i++) {
            const int64_t o = (int64_t)min(s0 + i, R.nsplit - 1) * sstride;
            v0[i] = src[o];
            v1[i] = src[o + 256];
        }
#pragma unroll
        for (int i = 0; i < SB; i++) {
            if (s0 + i < R.nsplit) {
                o0 += fac[s0 + i] * v0[i];
                o1 += fac[s0 + i] * v1[i];
            }
        }
    }
    float *dst = olat + ((int64_t)(R.qrow + qi) * H + h) * kMlaDc;
    dst[c] = o0 * inv_l;
    dst[c + 256] = o1 * inv_l;
}

// out[row][h][d] = sum_c o_lat[row][h][c] * W_UV[c][h*D + d].  Block = (head,
// 16 output dims, 16 query rows); wave w takes latent channels
// [128w, 128w + 128) of the C[16 dims][16 rows] tile (MFMA 16x16x16) and the
// four partial tiles are summed in LDS.  A = 4 consecutive channels of one
// dim per lane, from the block's W_UV slice [512 c][16 d] staged in LDS and
// read with the LDS transpose read; B = 4 consecutive channels of one o_lat
// row per lane straight from memory (f32, entered as hi + lo bf16).  All
// global loads are issued before the first product.
__global__ __launch_bounds__(256) void mla_proj_kernel(const float *__restrict__ olat,
                                                       const uint16_t *__restrict__ w_uv,
                                                       int H, int D, int total_q,
                                                       void *__restrict__ out, int out_bf16) {
    constexpr int KB = kMlaDc / 16 / 4;  // k-steps per wave
    __shared__ __attribute__((aligned(16))) uint16_t wt[kMlaDc * 16];
    __shared__ fl4 red[3][64];
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * 16;
    const int r0 = blockIdx.z * 16;
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int col = lane & 15, grp = lane >> 4;
    u32x4 w[4];
    const uint16_t *ws = w_uv + (int64_t)h * D + d0 + (t & 1) * 8;
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = *(const u32x4 *)(ws + (int64_t)((t >> 1) + 128 * i) * H * D);
    const int row = min(r0 + col, total_q - 1);
    const float *ob = olat + ((int64_t)row * H + h) * kMlaDc + wave * 128 + grp * 4;
    float4 f[KB];
#pragma unroll
    for (int kb = 0; kb < KB; kb++) f[kb] = *(const float4 *)(ob + kb * 16);
#pragma unroll
    for (int i = 0; i < 4; i++) *(u32x4 *)(wt + ((t >> 1) + 128 * i) * 16 + (t & 1) * 8) = w[i];
    __syncthreads();
    // Transpose read: lane (grp, col) fetches 4 dims of channel row
    // 4 grp + col / 4 and receives dim col of channels 4 grp .. 4 grp + 3.
    const uint16_t *tr = wt + (wave * 128 + 4 * grp + (col >> 2)) * 16 + (col & 3) * 4;
    fl4 acc = fl4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
        const sh4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) sh4 *)(tr + kb * 16 * 16));
        uint16_t hx, lx, hy, ly, hz, lz, hw, lw;
        split_bf16(f[kb].x, hx, lx);
        split_bf16(f[kb].y, hy, ly);
        split_bf16(f[kb].z, hz, lz);
        split_bf16(f[kb].w, hw, lw);
        const u32x2 bh = u32x2{(uint32_t)hx | ((uint32_t)hy << 16), (uint32_t)hz | ((uint32_t)hw << 16)};
        const u32x2 bl = u32x2{(uint32_t)lx | ((uint32_t)ly << 16), (uint32_t)lz | ((uint32_t)lw << 16)};
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, __builtin_bit_cast(sh4, bh), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, __builtin_bit_cast(sh4, bl), acc, 0, 0, 0);
    }
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
    acc = ((acc + red[0][lane]) + red[1][lane]) + red[2][lane];
    // C[4 grp + i][col]: dims d0 + 4 grp + i of row r0 + col.
    if (r0 + col < total_q) {
        const int64_t o = ((int64_t)(r0 + col) * H + h) * D + d0 + 4 * grp;
        if (out_bf16) {
            u32x2 o2;
            o2[0] = (uint32_t)bf16_rne(acc[0]) | ((uint32_t)bf16_rne(acc[1]) << 16);
            o2[1] = (uint32_t)bf16_rne(acc[2]) | ((uint32_t)bf16_rne(acc[3]) << 16);
            *(u32x2 *)((uint16_t *)out + o) = o2;
        } else {
            *(fl4 *)((float *)out + o) = acc;
        }
    }
}

template <int NQT, bool ARG>
static void launch_mla_t(hipStream_t s, typename PlanSel<ARG>::T plan, const uint16_t *pool,
                         const int32_t *table, const AttRow *rows, int n_rows, const int2 *work,
                         int n_work, const uint16_t *qlat, int H, int P, int chunk, int mask_mode,
                         float *part_o, float *part_ml) {
    mla_decode_kernel<NQT, ARG><<<n_work, 64 * MlaShape<NQT>::NW, 0, s>>>(plan, pool, table, rows, work, n_rows, qlat,
                                                        H, P, chunk, mask_mode, part_o, part_ml);
}

hipError_t launch_mla_decode(hipStream_t s, const PlanArg *plan, const uint16_t *pool,
                             const int32_t *table, const AttRow *rows, int n_rows,
                             const int2 *work, int n_work,
                             const void *q_nope, const void *q_rope, int q_bf16,
                             const uint16_t *w_uk, const uint16_t *w_uv, int H, int hd,
                             int total_q, int max_nq, int P, int chunk, float qscale,
                             int mask_mode, int nqt, uint16_t *qlat, float *part_o,
                             float *part_ml, float *olat, void *out, int out_bf16,
                             hipEvent_t ev0, hipEvent_t ev1) {
    if (n_work <= 0) return hipSuccess;
    if (hd > 256 || hd % 64 != 0) return hipErrorInvalidValue;
    const dim3 ag(H, kMlaDc / 64, (total_q + 15) / 16);
    switch (hd) {
        case 64: mla_absorb_kernel<64><<<ag, 256, 0, s>>>(q_nope, q_rope, q_bf16, w_uk, H, total_q, qscale, qlat); break;
        case 128: mla_absorb_kernel<128><<<ag, 256, 0, s>>>(q_nope, q_rope, q_bf16, w_uk, H, total_q, qscale, qlat); break;
        case 192: mla_absorb_kernel<192><<<ag, 256, 0, s>>>(q_nope, q_rope, q_bf16, w_uk, H, total_q, qscale, qlat); break;
        default: mla_absorb_kernel<256><<<ag, 256, 0, s>>>(q_nope, q_rope, q_bf16, w_uk, H, total_q, qscale, qlat); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ev0) (void)hipEventRecord(ev0, s);
    if (nqt != 1 && nqt != 2) return hipErrorInvalidValue;
    if (plan && nqt == 1)
        launch_mla_t<1, true>(s, *plan, pool, table, rows, n_rows, work, n_work, qlat, H, P, chunk,
                              mask_mode, part_o, part_ml);
    else if (plan)
        launch_mla_t<2, true>(s, *plan, pool, table, rows, n_rows, work, n_work, qlat, H, P, chunk,
                              mask_mode, part_o, part_ml);
    else if (nqt == 1)
        launch_mla_t<1, false>(s, NoPlan{0}, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                               chunk, mask_mode, part_o, part_ml);
    else
        launch_mla_t<2, false>(s, NoPlan{0}, pool, table, rows, n_rows, work, n_work, qlat, H, P,
                               chunk, mask_mode, part_o, part_ml);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ev1) (void)hipEventRecord(ev1, s);
    if (plan)
        mla_combine_kernel<true><<<dim3(n_rows, max_nq * H), 256, 0, s>>>(*plan, rows, part_o,
                                                                          part_ml, H, 16 * nqt, olat);
    else
        mla_combine_kernel<false><<<dim3(n_rows, max_nq * H), 256, 0, s>>>(
            NoPlan{0}, rows, part_o, part_ml, H, 16 * nqt, olat);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    mla_proj_kernel<<<dim3(H, hd / 16, (total_q + 15) / 16), 256, 0, s>>>(olat, w_uv, H, hd,
                                                                         total_q, out, out_bf16);
    return hipGetLastError();
}

int mla_decode_wgs_per_cu(int nqt) {
    int n = 0;
    hipError_t e = hipErrorInvalidValue;
    if (nqt == 1) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mla_decode_kernel<1, true>, 64 * MlaShape<1>::NW, 0);
    if (nqt == 2) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mla_decode_kernel<2, true>, 64 * MlaShape<2>::NW, 0);
    return (e == hipSuccess && n > 0) ? n : 1;
}

}  // namespace rlx
