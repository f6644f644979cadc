// Chunked prefill / long verify: FA2-style attention of many query rows over
// the cache, causal with the cache offset (query i of n_q on a sequence of T
// live tokens sees keys <= T - n_q + i).
//
// Work item = (sequence, head group, query tile).  A head group is one kv
// head with its G = H/KVH query heads (GQA) or one head (MLA, decompressed).
// A tile holds 256 query rows, query-major: row r = (token r / G, head r % G),
// so the G heads that share a kv head share every K/V byte the tile loads
// (floor(256 / G) tokens; rows past them do nothing).
// 8 waves of 32 rows each.
//
// Keys stream in 64-key blocks through a multi-stage LDS ring filled
// straight from memory (16-byte global-to-LDS loads), and both products run
// on the 32x32 matrix instruction, so a wave pays the per-block bookkeeping
// (waits, barrier, page lookups, the running-max test) once per 64 keys:
//   S^T[32 keys][32 rows] = K . Q^T   (2 key tiles, DQK/16 k-steps each):
//       A = K rows from LDS (lane m%32 reads key row m, 8 dims per lane
//       half), B = Q^T in registers (8 dims of the lane's query row).
//   O^T[32 dims][32 rows] += V^T . P^T (DV/32 dim tiles, 4 k-steps of 16
//       keys): A = V^T rows from LDS, B = P^T straight from the score
//       registers.
//
// Sources (SRC):
//   kSrcPaged : GQA paged cache, K pages (k-step-major 16-token blocks) and
//               dim-major V pages, DQK = DV = D.
//   kSrcDense : MLA, per sequence decompressed K_c [H][Tp][128] and
//               V^T [H][128][Tp] (Tp = T rounded up to 128) plus the rope keys
//               k^R [Tp][64] gathered from the latent rows once per call
//               (shared by every head, addressed like K_c: no page-table
//               reads in the key loop); DQK = 192, DV = 128.
// Keys at or past the live length are masked; the K rows staged for them
// repeat the last live key and their V^T entries are zeroed in LDS, so
// nothing past the live length can reach the output.
#include "rlx_common.h"

namespace rlx {

constexpr int kWaves = 8;                // 512 threads, 32 query rows per wave
constexpr int kTileRows = 32 * kWaves;   // 256

__device__ __forceinline__ int pf_limit(int mask_mode, int len, int nq, int qi) {
    if (mask_mode == kMaskCausal) return len - nq + qi;
    if (mask_mode == kMaskRef) return (nq == len) ? qi : len - 1;
    return len - 1;
}

// A lane's 16 score values of a key tile are rows 8(i/4) + 4(lane/32) + i%4
// of S^T.  Row m of key tile kt holds key 32kt + pf_key(m), chosen so that
// value i of the lane is key 32kt + 8(lane/32) + 16(i/8) + i%8: values
// [8s', 8s'+8) are exactly the 8 consecutive keys the lane supplies to P.V
// k-step 2kt + s', and one 16-byte chunk of a V^T row.
// Softmax: the running max is only moved when a lane's weights of one key
// tile, computed with it, sum to more than kLazySum (a row max grew by about
// 2^6 or more), so the accumulators are rescaled about once per query tile
// instead of whenever some row's max grows; the weights exp2(s - m) stay
// below 2^10, which bf16 and the f32 sums hold with no loss of relative
// precision.  Numerator and denominator use the same m, so the normalised
// output is unchanged.
//
// LDS stage: K regions of [64 keys][8 chunks] (64 dims each: the paged K
// row split in DQK/64 regions; dense: K_c in two, then the rope keys) and
// the V^T region [DV][8 chunks].  Every region has a
// 128-byte row pitch and the same swizzle, chunk c of row r at c ^ ((r/2) & 7):
// the LDS serves a 16-byte read for 16 lanes per cycle from 64 banks, and
// any 16 consecutive rows -- two per 256-byte bank row -- then fill 16
// distinct slots, so the K (16 key rows) and V^T (16 dim rows) operand reads
// are free of bank conflicts.  Every wave loads 8 rows of each K region and
// DV/64 x 8 rows of V^T; a K load instruction's 64 chunks lie in one 16-key
// group (one page), so it takes a wave-uniform base plus a fixed lane offset.
constexpr int kKeyBlock = 64;            // keys per block
constexpr float kLazySum = 1024.f;  // bound of a lane's 16 weights of one key tile
constexpr int kPfD = 4;             // LDS operand reads in flight ahead of the products

typedef __attribute__((ext_vector_type(16))) float fl16;

__device__ __forceinline__ int pf_key(int m) {
    return ((m >> 4) << 4) | (((m >> 2) & 1) << 3) | (((m >> 3) & 1) << 2) | (m & 3);
}
__device__ __forceinline__ int pf_swz(int r) { return (r >> 1) & 7; }

template <int DQK, int DV, int SRC>
struct PfShape {
    static constexpr int KS = DQK / 16;                              // score k-steps
    static constexpr int NKR = DQK / 64;                             // K regions
    static constexpr int DP = SRC == kSrcDense ? DQK - 64 : DQK;     // dense: K_c row pitch
    static constexpr int ST = NKR * 512 + DV * 8;                    // chunks per stage
    static constexpr int LV = DV / 64;                               // V^T loads per wave
    static constexpr int LPW = NKR + LV;                             // ring loads per wave
    static constexpr int S = ST * 16 * 4 <= 131072 ? 4 : ST * 16 * 3 <= 163840 ? 3 : 2;  // blocks in flight + 1
    // Staggered waves (waves 4-7 run their P.V of block j - 1 in iteration
    // j) keep one more stage resident: the dense (MLA) shape, where it fits
    // the 160 KB and measured faster (config 4: 4.45-4.48 -> 4.36-4.39 ms;
    // the paged GQA shapes at D 64 / 128 were unchanged, so they keep the
    // plain schedule).
    static constexpr bool STAG = SRC == kSrcDense && ST * 16 * (S + 1) <= 163840;
    static constexpr int SR = S + (STAG ? 1 : 0);                    // ring stages
    static constexpr int MD = DV / 32;                               // output dim tiles
    static_assert(DQK % 64 == 0 && DV % 64 == 0, "whole 64-dim regions");
    static_assert(SRC == kSrcPaged || DV == 128, "dense: 128 value dims per launch");
};

// POW2: the page size is a power of two (page index and slot by shifts).
template <int DQK, int DV, int SRC, bool POW2>
__global__ __launch_bounds__(64 * kWaves) void prefill_kernel(const PrefillArgs a,
                                                          const int32_t *__restrict__ table) {
    using SH = PfShape<DQK, DV, SRC>;
    constexpr int KS = SH::KS, NKR = SH::NKR, S = SH::S, MD = SH::MD, LV = SH::LV, LPW = SH::LPW;
    constexpr int DP = SH::DP, SR = SH::SR;
    constexpr bool STAG = SH::STAG;
    __shared__ __attribute__((aligned(16))) uint16_t ring[SR * SH::ST * 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hh = lane >> 5;
    const int4 wk = a.work[blockIdx.x];
    if (wk.x < 0) return;  // padding item of the XCD-balanced work order
    const AttRow R = a.rows[wk.x];
    const int hg = wk.y;
    const int G = (SRC == kSrcPaged) ? a.H / a.KVH : 1;
    const int toks = kTileRows / G;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)ring;

    int kend;
    {
        const int jmax = min(R.nq - 1, wk.z * toks + toks - 1);
        kend = min(R.len, pf_limit(a.mask_mode, R.len, R.nq, jmax) + 1);
        if (a.mask_mode == kMaskRef && R.nq != R.len) kend = R.len;
    }
    const int nblk = (kend + kKeyBlock - 1) / kKeyBlock;

    // ---- per-lane ring load offsets (fixed for every block) ----------------
    // K regions: this wave's rows kr = 8 wave + lane / 8 (16-key group
    // wave / 2), logical chunk klc (dims 64 q + 8 klc of region q).
    const int kr = 8 * wave + (lane >> 3);
    const int klc = (lane & 7) ^ pf_swz(kr);
    uint32_t ko[NKR];
#pragma unroll
    for (int q = 0; q < NKR; q++) {
        if (SRC == kSrcPaged)
            ko[q] = (uint32_t)k_page_off(kr & 15, 64 * q + klc * 8, DQK) * 2;
        else if (q < NKR - 1)
            ko[q] = (uint32_t)(kr * DP + 64 * q + klc * 8) * 2;
        else
            ko[q] = (uint32_t)(kr * kMlaDr + klc * 8) * 2;
    }
    // V^T load i: row vd, logical chunk vlc (keys 8 vlc .. 8 vlc + 7).
    int vd[LV], vlc[LV];
    uint32_t ov[LV];
#pragma unroll
    for (int i = 0; i < LV; i++) {
        const int p = (8 * i + wave) * 64 + lane;
        vd[i] = p >> 3;
        vlc[i] = (p & 7) ^ pf_swz(vd[i]);
        ov[i] = (SRC == kSrcDense) ? (uint32_t)((int64_t)(a.dv0 + vd[i]) * R.nsplit + vlc[i] * 8) * 2 : 0u;
    }
    auto pdiv = [&](int t) { return POW2 ? t >> a.pshift : t / a.P; };
    auto pmod = [&](int t) { return POW2 ? t & (a.P - 1) : t % a.P; };
    const uint16_t *kc_seq = nullptr, *vt_seq = nullptr, *kr_seq = nullptr;
    if (SRC == kSrcDense) {
        kc_seq = a.kc + ((int64_t)R.part * a.H + (int64_t)hg * R.nsplit) * DP;
        vt_seq = a.vt + (int64_t)R.part * a.H * DP + (int64_t)hg * DP * R.nsplit;
        kr_seq = a.kr + (int64_t)R.part * kMlaDr;
    }
    // Blocks are issued in order, one per call: running K_c / V^T / rope-key
    // pointers and stage offset of the next block to issue.
    const uint16_t *kc_next = kc_seq, *vt_next = vt_seq, *kr_next = kr_seq;
    uint32_t st_next = 0;
    constexpr uint32_t kStageBytes = SH::ST * 16;

    // Page id of key t (t < len), a wave-uniform scalar load.
    auto page_of = [&](int t) { return table[R.tab + pdiv(t)]; };
    // V^T lanes of the paged cache read keys of 16-key group vlc / 2 of the
    // block: lane masks of the groups, for the per-lane page selection.
    bool vg1[LV], vg2[LV], vg3[LV];
#pragma unroll
    for (int i = 0; i < LV; i++) {
        vg1[i] = (vlc[i] >> 1) == 1;
        vg2[i] = (vlc[i] >> 1) == 2;
        vg3[i] = (vlc[i] >> 1) == 3;
    }

    auto issue_block = [&](int j) {
        const int k0 = j * kKeyBlock;
        const uint32_t stage = ring_lds + st_next;
        const uint32_t kdst = stage + (uint32_t)(wave * 64) * 16;  // + region q: q * 8 KB
        const uint16_t *kc_blk = kc_next, *vt_blk = vt_next, *kr_blk = kr_next;
        st_next = (st_next + kStageBytes == SR * kStageBytes) ? 0u : st_next + kStageBytes;
        if (SRC == kSrcDense) {
            kc_next += kKeyBlock * DP;
            vt_next += kKeyBlock;
            kr_next += kKeyBlock * kMlaDr;
        }
        if (k0 + kKeyBlock <= R.len) {
            // Every key of the block is live.  K: the wave's 8 rows lie in
            // 16-key group wave / 2.
            if (SRC == kSrcPaged) {
                const int tg = k0 + 16 * (wave >> 1);
                const uint16_t *b = a.kpool + (((int64_t)page_of(tg) * a.KVH + hg) * a.P + pmod(tg)) * DQK;
#pragma unroll
                for (int q = 0; q < NKR; q++) lds_dma16(b, ko[q], kdst + q * 8192);
            } else {
                // Dense K_c / V^T rows are re-read by every query tile of
                // the head (on one XCD, at consecutive positions): these
                // loads leave the lines in L2 (no non-temporal hint).
#pragma unroll
                for (int q = 0; q < NKR - 1; q++) lds_dma16_keep(kc_blk, ko[q], kdst + q * 8192);
                lds_dma16_keep(kr_blk, ko[NKR - 1], kdst + (NKR - 1) * 8192);
            }
            if (SRC == kSrcPaged) {
                int pg[4];
#pragma unroll
                for (int g = 0; g < 4; g++) pg[g] = page_of(k0 + 16 * g);
#pragma unroll
                for (int i = 0; i < LV; i++) {
                    const uint32_t dst = stage + (uint32_t)(NKR * 512 + (8 * i + wave) * 64) * 16;
                    const int pgl = vg1[i] ? pg[1] : vg2[i] ? pg[2] : vg3[i] ? pg[3] : pg[0];
                    const uint16_t *gp = a.vpool + (((int64_t)pgl * a.KVH + hg) * a.vd + a.dv0 + vd[i]) * a.P +
                                         pmod(k0 + 8 * vlc[i]);
                    lds_dma16(gp, dst);
                }
            } else {
#pragma unroll
                for (int i = 0; i < LV; i++)
                    lds_dma16_keep(vt_blk, ov[i], stage + (uint32_t)(NKR * 512 + (8 * i + wave) * 64) * 16);
            }
            return;
        }
        // Last block of the sequence: K rows past the live length repeat the
        // last live key; V^T chunks wholly past it load the block's first
        // chunk (their entries are zeroed in LDS before use).
        {
            const int t = min(k0 + kr, R.len - 1);
            const int pgt = SRC == kSrcPaged ? table[R.tab + pdiv(t)] : 0;
#pragma unroll
            for (int q = 0; q < NKR; q++) {
                const uint16_t *gp;
                if (SRC == kSrcPaged)
                    gp = a.kpool + ((int64_t)pgt * a.KVH + hg) * a.P * DQK + k_page_off(pmod(t), 64 * q + klc * 8, DQK);
                else if (q < NKR - 1)
                    gp = kc_seq + (int64_t)t * DP + 64 * q + klc * 8;
                else
                    gp = kr_seq + (int64_t)t * kMlaDr + klc * 8;
                lds_dma16(gp, __builtin_amdgcn_readfirstlane(kdst + q * 8192));
            }
        }
#pragma unroll
        for (int i = 0; i < LV; i++) {
            const uint32_t dst = __builtin_amdgcn_readfirstlane(
                stage + (uint32_t)(NKR * 512 + (8 * i + wave) * 64) * 16);
            int t = k0 + 8 * vlc[i];
            if (t >= R.len) t = k0;
            const uint16_t *gp;
            if (SRC == kSrcPaged) {
                const int pgt = table[R.tab + pdiv(t)];
                gp = a.vpool + (((int64_t)pgt * a.KVH + hg) * a.vd + a.dv0 + vd[i]) * a.P + pmod(t);
            } else {
                gp = vt_seq + (int64_t)(a.dv0 + vd[i]) * R.nsplit + t;
            }
            lds_dma16(gp, dst);
        }
    };
    // Wait until this wave's loads of block j landed: S - 2 blocks were
    // issued after it in the steady state, fewer at the end.
    auto wait_block = [&](int j) {
        if (j + S - 2 < nblk) {
            RLX_WAIT_VM((S - 2) * LPW);
        } else if (S >= 4 && j + 1 < nblk) {
            RLX_WAIT_VM(LPW);
        } else {
            RLX_WAIT_VM(0);
        }
    };
    static_assert(S <= 4, "wait_block covers at most two blocks ahead");

    for (int j = 0; j < S - 1 && j < nblk; j++) issue_block(j);

    // ---- query operand (B of S^T) and key limit of the lane's row ----------
    const int qrow_t = wave * 32 + l32;
    const int qj = wk.z * toks + qrow_t / G;
    const int qh = hg * G + qrow_t % G;
    // (rows past toks x G -- a group size that does not divide 256 -- belong
    // to no token of this tile: zero queries, every key masked, no store)
    const bool rvalid = qj < R.nq && qrow_t < toks * G;
    const int klim = rvalid ? pf_limit(a.mask_mode, R.len, R.nq, qj) : -1;
    bf16x8 qb[KS];
    {
        const int jc = min(qj, R.nq - 1);
        const float zs = rvalid ? a.qscale : 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            // q dims d .. d + 7 of a row of nd dims (zeros past nd: the K and V
            // rows hold zeros there too)
            const int d0 = ks * 16 + hh * 8;
            const void *src;
            int64_t off;
            int d, nd;
            if (SRC == kSrcPaged || d0 < DP) {
                src = a.q;
                d = d0;
                nd = a.qd;
                off = (a.layout == kLayoutSHD || SRC == kSrcDense)
                          ? ((int64_t)(R.qrow + jc) * a.HQ + a.h0 + qh) * nd + d
                          : ((int64_t)R.qrow * a.HQ + (int64_t)(a.h0 + qh) * R.nq + jc) * nd + d;
            } else {
                src = a.q2;
                d = d0 - DP;
                nd = a.qd2;
                off = ((int64_t)(R.qrow + jc) * a.HQ + a.h0 + qh) * nd + d;
            }
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (d + 8 <= nd && (nd & 7) == 0) {  // whole aligned chunk
                if (a.q_bf16) {
                    const u32x4 raw = *(const u32x4 *)((const uint16_t *)src + off);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[2 * i] = bf16_f32((uint16_t)(raw[i] & 0xFFFFu));
                        v[2 * i + 1] = bf16_f32((uint16_t)(raw[i] >> 16));
                    }
                } else {
                    const float4 *f = (const float4 *)((const float *)src + off);
                    const float4 x = f[0], y = f[1];
                    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
                    v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (d + i < nd)
                        v[i] = a.q_bf16 ? bf16_f32(((const uint16_t *)src)[off + i]) : ((const float *)src)[off + i];
            }
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = (uint32_t)bf16_rne(v[2 * i] * zs) | ((uint32_t)bf16_rne(v[2 * i + 1] * zs) << 16);
            qb[ks] = __builtin_bit_cast(bf16x8, w);
        }
    }
    int kmin = rvalid ? klim : 0x7fffffff;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) kmin = min(kmin, __shfl_xor(kmin, off));
    kmin = __builtin_amdgcn_readfirstlane(kmin);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) asm volatile("" ::"v"(qb[ks]));

    // LDS read offsets (bf16 elements within a stage).  K, k-step ks: region
    // ks / 4, row kt*32 + pf_key(l32), logical chunk 2 (ks % 4) + hh,
    // physical (2 (ks % 4)) ^ u with u = hh ^ swizzle(row); the region is an
    // immediate offset.  V^T, k-step s: row 32 md + l32 (md an immediate),
    // logical chunk 2s + hh, physical (2s) ^ (hh ^ swizzle(l32)).
    int krd[2][4], vrd[4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
        const int row = kt * 32 + pf_key(l32);
        const int u = hh ^ pf_swz(row);
#pragma unroll
        for (int e = 0; e < 4; e++) krd[kt][e] = row * 64 + ((2 * e) ^ u) * 8;
    }
#pragma unroll
    for (int s2 = 0; s2 < 4; s2++) vrd[s2] = NKR * 4096 + l32 * 64 + ((2 * s2) ^ (hh ^ pf_swz(l32))) * 8;

    float m_run = -INFINITY, l_part = 0.f;
    fl16 acc[MD];
#pragma unroll
    for (int md = 0; md < MD; md++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[md][i] = 0.f;
    // -m_use in every entry: the first score product of a key tile starts
    // its accumulation from it, so the scores come out as s - m_use and the
    // weights need no subtraction (rebuilt only when the running max moves).
    // The widest shape (<320,128>) keeps the subtraction: its 16 registers
    // would spill there.
    constexpr bool FOLD = DQK + DV <= 384;
    fl16 negm;
#pragma unroll
    for (int i = 0; i < 16; i++) negm[i] = 0.f;
    // P^T operands of the current block (the lagging waves keep them into
    // the next iteration).
    u32x4 pw[4];
    // P.V of the weights in pw over the V^T region of stage sv, operand
    // reads kPfD steps ahead (the lagging waves' form: no softmax work to
    // interleave).
    auto pv_plain = [&](const uint16_t *sv) {
        constexpr int NV = 4 * MD;
        auto vr = [&](int n) { return *(const u32x4 *)&sv[vrd[n / MD] + (n % MD) * 32 * 64]; };
        u32x4 va[kPfD + 1];
#pragma unroll
        for (int n = 0; n < kPfD; n++) va[n] = vr(n);
#pragma unroll
        for (int n = 0; n < NV; n++) {
            __builtin_amdgcn_sched_barrier(0);
            if (n + kPfD < NV) va[(n + kPfD) % (kPfD + 1)] = vr(n + kPfD);
            const int md = n % MD;
            acc[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, va[n % (kPfD + 1)]), __builtin_bit_cast(bf16x8, pw[n / MD]),
                acc[md], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // Staggered schedule: waves w and w + 4 share a SIMD.  Waves 0-3 run
    // block j's scores, softmax and P.V in iteration j; waves 4-7 first run
    // the P.V of block j - 1 (its weights kept in registers), then block j's
    // scores and softmax, so that one wave's softmax meets the other's
    // products instead of both waiting on the matrix unit's neighbour at
    // once.  Block j - 1 stays resident through iteration j: the refill of
    // iteration j goes to block j - 2's stage (SR = S + 1 stages).
    // The two schedules are separate loops (a compile-time flag each), so
    // that each gets its own register allocation; both pass the same
    // barriers.
    auto run = [&](auto lagc) {
    constexpr bool lag = decltype(lagc)::value;
    int st_prev = 0;
    for (int j = 0, st_read = 0; j < nblk;
         j++, st_prev = st_read, st_read = (st_read + SH::ST * 8 == SR * SH::ST * 8) ? 0 : st_read + SH::ST * 8) {
        wait_block(j);
        ring_barrier();
        if (SRC == kSrcPaged && j + S - 1 < nblk) issue_block(j + S - 1);
        const int k0 = j * kKeyBlock;
        const uint16_t *st = ring + st_read;
        if (k0 + kKeyBlock > R.len) {
            uint16_t *Vw = ring + st_read + NKR * 4096;
            const int live = R.len - k0;
            for (int e = tid; e < DV * kKeyBlock; e += 64 * kWaves) {
                const int d = e / kKeyBlock, kk = e - d * kKeyBlock;
                if (kk >= live) Vw[d * kKeyBlock + (((kk >> 3) ^ pf_swz(d)) << 3) + (kk & 7)] = 0;
            }
            ring_barrier();
        }
        // Weights of key tile 0 are computed with the current running max
        // while tile 1's score products execute, and those of tile 1 while
        // tile 0's P.V products execute.  A tile is redone after a rescale to
        // its max when some lane's weights of it sum to more than kLazySum
        // (or not to a finite value), or when a row gets its first unmasked
        // keys (no running max yet); rows with a stable maximum -- nearly
        // every block -- never need it.
        const bool need_mask = k0 + kKeyBlock - 1 > kmin;  // (also every block past the live length)

        // score operand reads run kPfD steps ahead of their products (a
        // rotating register set; the scheduling barriers keep the compiler
        // from sinking each read onto its product)
        auto kread = [&](int n) {
            const int kt = n / KS, ks = n % KS;
            return *(const u32x4 *)&st[(ks >> 2) * 4096 + krd[kt][ks & 3]];
        };
        auto vread = [&](int n) { return *(const u32x4 *)&st[vrd[n / MD] + (n % MD) * 32 * 64]; };
        // The lagging waves' P.V of the previous block (its stage stays
        // resident through this iteration).
        if constexpr (lag)
            if (j > 0) pv_plain(ring + st_prev);
        fl16 sc[2];
        float lt[2] = {0.f, 0.f};
        // With FOLD, sc holds s - m_use (m_use = the running max, 0 before a
        // row's first unmasked key); a rescale moves m_use and shifts the
        // tiles still to be weighed by the same amount.
        float m_use = (m_run == -INFINITY) ? 0.f : m_run;
        // P^T operands: word k (0..7) of key tile kt packs values 2k, 2k+1
        // (the B operand of k-step 2kt + k/4 is words 4(k/4) .. +3).
        // (The empty asm uses the word where it is computed: otherwise the
        // compiler sinks the work to its first use, out of the products it
        // is meant to overlap.)
        auto pword = [&](int kt, int k) {
            const float p0 = __builtin_amdgcn_exp2f(FOLD ? sc[kt][2 * k] : sc[kt][2 * k] - m_use);
            const float p1 = __builtin_amdgcn_exp2f(FOLD ? sc[kt][2 * k + 1] : sc[kt][2 * k + 1] - m_use);
            const uint32_t w = pack_bf16x2(p0, p1);
            pw[2 * kt + (k >> 2)][k & 3] = w;
            lt[kt] = add_bf16x2(w, lt[kt]);
            asm volatile("" ::"v"(w), "v"(lt[kt]));
        };
        // Causal mask of key tile kt (value i is masked when its key offset
        // exceeds t).  The empty asm keeps the caller's test a branch: as
        // selects it would run on every block.
        auto mask = [&](int kt) {
            asm volatile("");
            const int t = klim - k0 - 8 * hh;
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (32 * kt + 16 * (i >> 3) + (i & 7) > t) sc[kt][i] = -INFINITY;
        };
        // redo0 (the lagging waves at tile 1): tile 0's weights are not in
        // the accumulators yet, so a rescale recomputes them at the new max,
        // and l_part takes their new sum in place of the old one scaled.
        auto fixup = [&](int kt, bool redo0 = false) {
            if (__builtin_amdgcn_ballot_w64(!(lt[kt] <= kLazySum) || (m_run == -INFINITY && lt[kt] > 0.f))) {
                float mx = sc[kt][0];
#pragma unroll
                for (int i = 1; i < 16; i++) mx = fmaxf(mx, sc[kt][i]);
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                // (-inf + m_use stays -inf: a row with only masked keys)
                const float m_new = fmaxf(m_run, fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) + (FOLD ? m_use : 0.f));
                // A row that has seen only masked keys keeps m = -inf (factor
                // 1: its accumulators are zero).
                const float c = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
                l_part *= c;
#pragma unroll
                for (int md = 0; md < MD; md++) acc[md] *= c;
                m_run = m_new;
                const float m_use_new = (m_run == -INFINITY) ? 0.f : m_run;
                const float dlt = m_use_new - m_use;
                m_use = m_use_new;
                if constexpr (FOLD) {
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        negm[i] = -m_use;
                        sc[kt][i] -= dlt;
                        if (kt == 0 || redo0) sc[1 - kt][i] -= dlt;  // tile 1 is weighed after this
                    }
                }
                if (redo0) {
                    const float old0 = lt[0] * c;
                    lt[0] = 0.f;
#pragma unroll
                    for (int k = 0; k < 8; k++) pword(0, k);
                    l_part += lt[0] - old0;
                }
                lt[kt] = 0.f;
#pragma unroll
                for (int k = 0; k < 8; k++) pword(kt, k);
            }
            l_part += lt[kt];
        };
        // Scores of both key tiles; tile 0's weights during tile 1's
        // products (from its third, once tile 0's last product has landed).
        {
            constexpr int NS = 2 * KS;
            u32x4 ka[kPfD + 1];
#pragma unroll
            for (int n = 0; n < kPfD; n++) ka[n] = kread(n);
#pragma unroll
            for (int n = 0; n < NS; n++) {
                __builtin_amdgcn_sched_barrier(0);
                if (n + kPfD < NS) ka[(n + kPfD) % (kPfD + 1)] = kread(n + kPfD);
                const int kt = n / KS, ks = n % KS;
                const bf16x8 A = __builtin_bit_cast(bf16x8, ka[n % (kPfD + 1)]);
                if (ks == 0)
                    sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, qb[ks], FOLD ? negm : fl16{}, 0, 0, 0);
                else
                    sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, qb[ks], sc[kt], 0, 0, 0);
                if (n == KS + 1 && need_mask) mask(0);
                const int k = n - KS - 2;
                if (k >= 0 && k < 8) pword(0, k);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = KS - 2; k < 8; k++) pword(0, k);  // (what did not fit)
        // Dense sources refill the stage the barrier released with block
        // j + S - 1 here, between the score and the P.V products, so that a
        // load stalled by memory back-pressure does not hold up this block's
        // score reads (config 4: -0.5 %).  (The paged source issues right
        // after the barrier: its block loads wait on page-table reads.)
        if (SRC == kSrcDense && j + S - 1 < nblk) issue_block(j + S - 1);
        if (need_mask) mask(1);
        fixup(0);
        if constexpr (lag) {
            // tile 1's weights now; the products follow next iteration
#pragma unroll
            for (int k = 0; k < 8; k++) pword(1, k);
            fixup(1, true);
            continue;
        }
        // P.V with the V^T operands kPfD steps ahead; tile 1's weights during
        // tile 0's products.
        {
            constexpr int NV = 4 * MD, HALF = 2 * MD;
            u32x4 va[kPfD + 1];
#pragma unroll
            for (int n = 0; n < kPfD; n++) va[n] = vread(n);
#pragma unroll
            for (int n = 0; n < NV; n++) {
                __builtin_amdgcn_sched_barrier(0);
                if (n == HALF) {
                    fixup(1);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (n + kPfD < NV) va[(n + kPfD) % (kPfD + 1)] = vread(n + kPfD);
                const int md = n % MD;
                acc[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, va[n % (kPfD + 1)]), __builtin_bit_cast(bf16x8, pw[n / MD]),
                    acc[md], 0, 0, 0);
                if (n < HALF) {
#pragma unroll
                    for (int k = (n * 8) / HALF; k < ((n + 1) * 8) / HALF; k++) pword(1, k);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if constexpr (lag)
        if (nblk > 0) pv_plain(ring + st_prev);  // the last block's P.V
    };
    if (STAG && wave >= kWaves / 2)
        run(std::true_type{});
    else
        run(std::false_type{});

    // ---- normalise and write ----------------------------------------------
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_part), __float_as_uint(l_part), false, false);
        l_part = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (!rvalid) return;
    const float inv = (l_part > 0.f) ? 1.f / l_part : 0.f;
    const int64_t obase = ((a.layout == kLayoutSHD || SRC == kSrcDense)
                               ? ((int64_t)(R.qrow + qj) * a.HQ + a.h0 + qh) * a.od
                               : ((int64_t)R.qrow * a.HQ + (int64_t)(a.h0 + qh) * R.nq + qj) * a.od) + a.dv0;
#pragma unroll
    for (int md = 0; md < MD; md++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            if (a.dv0 + md * 32 + 8 * g4 + 4 * hh >= a.od) continue;  // (od is a multiple of 8)
            const int64_t off = obase + md * 32 + 8 * g4 + 4 * hh;
            const fl4 o = fl4{acc[md][4 * g4], acc[md][4 * g4 + 1], acc[md][4 * g4 + 2], acc[md][4 * g4 + 3]} * inv;
            if (a.out_bf16) {
                u32x2 w;
                w[0] = (uint32_t)bf16_rne(o[0]) | ((uint32_t)bf16_rne(o[1]) << 16);
                w[1] = (uint32_t)bf16_rne(o[2]) | ((uint32_t)bf16_rne(o[3]) << 16);
                *(u32x2 *)((uint16_t *)a.out + off) = w;
            } else {
                *(fl4 *)((float *)a.out + off) = o;
            }
        }
}

hipError_t launch_prefill(hipStream_t s, int src, int hd, const PrefillArgs &a, int n_work,
                          hipEvent_t ev0, hipEvent_t ev1) {
    if (n_work <= 0) return hipSuccess;
    const dim3 g(n_work), b(64 * kWaves);
    const bool p2 = a.pshift >= 0;
#define RLX_PF(DQK, DV, SRC, A, E0, E1)                                                              \
    (p2 ? launch_timed(prefill_kernel<DQK, DV, SRC, true>, g, b, s, E0, E1, A, A.table)            \
        : launch_timed(prefill_kernel<DQK, DV, SRC, false>, g, b, s, E0, E1, A, A.table))
    if (src == kSrcPaged && hd == 128) return RLX_PF(128, 128, kSrcPaged, a, ev0, ev1);
    if (src == kSrcPaged && hd == 64) return RLX_PF(64, 64, kSrcPaged, a, ev0, ev1);
    if (src == kSrcDense && hd == 128) return RLX_PF(192, 128, kSrcDense, a, ev0, ev1);
    if (hd == 256) {  // two launches, one per 128 value dims (the scores are computed in each)
        PrefillArgs a0 = a, a1 = a;
        a0.dv0 = 0;
        a1.dv0 = 128;
        hipError_t e = src == kSrcPaged ? RLX_PF(256, 128, kSrcPaged, a0, ev0, nullptr)
                                        : RLX_PF(320, 128, kSrcDense, a0, ev0, nullptr);
        if (e != hipSuccess) return e;
        return src == kSrcPaged ? RLX_PF(256, 128, kSrcPaged, a1, nullptr, ev1)
                                : RLX_PF(320, 128, kSrcDense, a1, nullptr, ev1);
    }
#undef RLX_PF
    return hipErrorInvalidValue;
}

}  // namespace rlx
