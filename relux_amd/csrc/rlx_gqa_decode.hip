// GQA flash-decoding over the paged bf16 cache (decode, speculative verify).
//
// Work item = (range, kv head); one 256-thread work-group (4 waves) per item,
// about one per CU.  The ranges cut the batch's tokens (rows laid end to
// end) into equal parts, so every work-group streams the same amount
// whatever the mix of lengths; a range holds one or more row segments, each
// processed in turn.  Each wave walks 16-token blocks of a segment:
//
//   S^T[16 tok][16 q-rows] = K_blk[16 x D] . Q^T          (D/32 MFMA 16x16x32 bf16)
//   online softmax per q-row column (lane-local state, exp2 domain)
//   O^T[D][16 q-rows]    += V_blk^T[D x 16 tok] . P^T     (D/16 MFMA 16x16x16 bf16)
//
// The K block is the A operand straight from its k-step-major page block
// (k_page_off: each 32-dim k-step of 16 tokens is 1 KB contiguous, 8
// consecutive dims per lane, 16-byte loads); the V^T tile is the A operand
// straight from a dim-major page (4 consecutive tokens per lane, 8-byte
// loads); the MFMA
// result layout of S^T is exactly the B-operand layout P^T needs, so no LDS
// and no shuffles sit between the two products.  The query rows of a kv head
// (H/KVH heads x n_q queries) fill the 16-wide N dimension; a second N tile
// covers up to 32 rows.  The 4 waves merge through LDS and write one
// unnormalised partial per segment; gqa_combine merges a row's segments
// (log-sum-exp).
//
// Reference restated: mha.go:291-348 (score = q.k * 1/sqrt(D), mask,
// softmaxRows, P.V); exact exp2 replaces fastexp32 (mha.go:823-833), f32
// accumulation throughout.
#include "rlx_common.h"

namespace rlx {


// Last key (inclusive, live index) query qi of a sequence may attend.
__device__ __forceinline__ int key_limit(int mask_mode, int len, int nq, int qi) {
    if (mask_mode == kMaskCausal) return len - nq + qi;
    if (mask_mode == kMaskRef) return (nq == len) ? qi : len - 1;
    return len - 1;
}

// head_dim 256 takes one 16-row query tile with the whole register file
// (its two block register sets alone are 128 VGPRs).
template <int D, int NQT>
constexpr int gqa_min_waves() { return D >= 256 ? 1 : (NQT == 1 ? 3 : 1); }

template <int D, int NQT, bool ARG>
__global__ __launch_bounds__(256, (gqa_min_waves<D, NQT>())) void gqa_decode_kernel(
    typename PlanSel<ARG>::T plan, const uint16_t *__restrict__ kpool,
    const uint16_t *__restrict__ vpool, const int32_t *__restrict__ table,
    const AttRow *__restrict__ rows, const int4 *__restrict__ ranges, int n_rows,
    const void *__restrict__ q, int q_bf16, int layout, int H, int KVH, int DQ, int P, int total64,
    int snap64, int ranges_off, float qscale, int mask_mode, float *__restrict__ part_o,
    float *__restrict__ part_ml) {
    // head_dim 16 holds only 4 dims per lane: its score step is one MFMA
    // 16x16x16 (4 bf16 per lane); wider heads use 16x16x32 k-steps.
    constexpr bool K16 = (D == 16);
    constexpr int KS = K16 ? 1 : D / 32;  // QK k-steps
    constexpr int KW = K16 ? 4 : 8;       // dims per lane per k-step
    constexpr int MT = D / 16;            // PV m-tiles
    constexpr int QRP = 16 * NQT;
    const int wave = threadIdx.x >> 6;
    // Work-group = (range, kv head); the kv heads of a range are consecutive
    // work-groups.  The rows' tokens, each row padded to a multiple of 64,
    // are laid end to end (total64 units of 64 positions) and cut into
    // n_ranges near-equal ranges; a cut closer than snap64 units to a row
    // boundary moves onto it (a sliver segment costs a start-up and a
    // partial).  Range wi covers [lo, hi) and every row segment inside it.
    // The host computes the same cuts (gqa_range_cuts).
    const int n_ranges = gridDim.x / KVH;
    const int kvh = blockIdx.x / n_ranges;
    const int wi = blockIdx.x - kvh * n_ranges;
    const int G = H / KVH;
    int r;
    int64_t Pr, lo, hi;  // padded start of row r; the range
    if (ARG && ranges_off >= 0) {
        // the host's ranges follow the rows in the arguments
        const __attribute__((address_space(4))) int32_t *p =
            (const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + ranges_off + wi * 16);
        r = p[0];
        Pr = (int64_t)p[1] * 64;
        lo = (int64_t)p[2] * 64;
        hi = (int64_t)p[3] * 64;
    } else if constexpr (ARG) {
        const int lane = threadIdx.x & 63;
        // <= 64 rows in the arguments: one lane per row, a wave-wide prefix
        // sum of the padded lengths (64-position units).
        const int len = lane < n_rows ? plan_row<ARG>(rows, lane).len : 0;
        const int pad = (len + 63) >> 6;
        int incl = pad;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(incl, off);
            if (lane >= off) incl += t;
        }
        const int excl = incl - pad;
        // floor(i * total64 / n_ranges) in 32-bit steps (i * rem < 2^31)
        const uint32_t qt = (uint32_t)total64 / (uint32_t)n_ranges;
        const uint32_t rem = (uint32_t)total64 - qt * (uint32_t)n_ranges;
        auto cut = [&](int i) -> int {
            const int b = (int)((uint32_t)i * qt + ((uint32_t)i * rem) / (uint32_t)n_ranges);
            if (b <= 0 || b >= total64) return b;
            const uint64_t at = __builtin_amdgcn_ballot_w64(lane < n_rows && excl <= b);
            const int rr = 63 - __builtin_clzll(at);
            const int p0 = __shfl(excl, rr), p1 = __shfl(incl, rr);
            const int d0 = b - p0, d1 = p1 - b;
            if (min(d0, d1) > snap64) return b;
            return d0 <= d1 ? p0 : p1;
        };
        const int lo64 = cut(wi), hi64 = cut(wi + 1);
        const uint64_t past = __builtin_amdgcn_ballot_w64(lane < n_rows && excl * 64 + len > lo64 * 64);
        r = past ? (int)__builtin_ctzll(past) : n_rows;
        Pr = (int64_t)__shfl(excl, r & 63) * 64;
        r = __builtin_amdgcn_readfirstlane(r);
        Pr = (int64_t)__builtin_amdgcn_readfirstlane((int)(Pr >> 6)) * 64;
        lo = (int64_t)__builtin_amdgcn_readfirstlane(lo64) * 64;
        hi = (int64_t)__builtin_amdgcn_readfirstlane(hi64) * 64;
    } else {
        // host-computed: first row, its start, the range (64-position units)
        const int4 rg = ranges[wi];
        r = rg.x;
        Pr = (int64_t)rg.y * 64;
        lo = (int64_t)rg.z * 64;
        hi = (int64_t)rg.w * 64;
    }

    __shared__ float sm[4][QRP], sl[4][QRP];
    __shared__ fl4 so[3][NQT][MT][64];
    const int64_t kstride = (int64_t)P * D;  // one kv head of one page
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    bool first = true;

    for (; r < n_rows && Pr < hi; r++) {
        // Lane-derived values are recomputed per segment from an opaque
        // lane index: hoisted out of the loop they would stay live across
        // it and spill.
        int lane = threadIdx.x & 63;
        asm volatile("" : "+v"(lane));
        const int col = lane & 15;
        const int grp = lane >> 4;
        // K blocks are k-step-major (k_page_off): k-step ks of row col sits
        // at ks * 512 + col * 32; head_dim 16 keeps plain rows.
        const int64_t k_lane = K16 ? (int64_t)col * D + grp * KW : (int64_t)col * 32 + grp * 8;
        const uint32_t v_off = (uint32_t)(col * P + grp * 4) * 2u;  // bytes
        const AttRow R = plan_row<ARG>(rows, r);
        const int64_t row_pos = Pr;
        Pr += (R.len + 63) & ~63;
        const int t_begin = (int)max(lo - row_pos, (int64_t)0);
        const int t_end = (int)min(hi - row_pos, (int64_t)R.len);
        if (t_begin >= t_end) continue;  // only the row's padding is in range
        // The previous segment's merge reads LDS until wave 0 gets here.
        if (!first) __syncthreads();
        first = false;
        const int QR = G * R.qn;  // query rows of this (tile of a) sequence

        // Wave w walks blocks t0 = tw0 + 64 j (j < nb) of 16 tokens.  Block
        // indices are wave-uniform (scalar), and the page ids of 64 blocks
        // are fetched at once, one per lane, and read back with readlane: no
        // table load sits between one block's K/V loads and the next's.
        const int tw0 = t_begin + 16 * wv;
        const int nb = (t_end > tw0) ? (t_end - tw0 + 63) / 64 : 0;
        auto fetch_pages = [&](int j0) {
            const int j = j0 + lane;
            return (j < nb) ? table[R.tab + (tw0 + 64 * j) / P] : 0;
        };
        // The first page ids are requested before the query loads so that
        // the two latencies overlap (the first block's loads wait for both).
        int pg = fetch_pages(0);

        // Q^T operand (B of the score product), pre-scaled by scale*log2(e);
        // KW consecutive dims per lane (the upper half stays zero when KW = 4).
        // Columns past the tile's query rows load row 0 (no branch around
        // the loads, so they are all in flight together) and are zeroed.
        u32x4 qb[NQT][KS];
        int klim[NQT];
        bool qv[NQT];
        int64_t qbase[NQT];
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            const int qr = nt * 16 + col;
            qv[nt] = qr < QR;
            const int qrc = qv[nt] ? qr : 0;
            const int ql = qrc / G;
            const int h = kvh * G + (qrc - ql * G);
            const int qi = R.q0 + ql;
            klim[nt] = qv[nt] ? key_limit(mask_mode, R.len, R.nq, qi) : R.len - 1;
            // q rows hold the caller's DQ dims (the pages may store more,
            // zero-padded): dims at or past DQ load nothing and stay zero.
            qbase[nt] = (layout == kLayoutSHD) ? ((int64_t)(R.qrow + qi) * H + h) * DQ
                                               : ((int64_t)R.qrow * H + (int64_t)h * R.nq + qi) * DQ;
        }
        bool dv[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) dv[ks] = ks * 32 + grp * KW < DQ;
        auto qoff = [&](int ks) { return dv[ks] ? ks * 32 + grp * KW : 0; };
        auto pack_q = [&](const float (&v)[8], bool valid) {
            u32x4 w = u32x4{0, 0, 0, 0};
            const float sc = valid ? qscale : 0.f;
#pragma unroll
            for (int i = 0; i < KW / 2; i++)
                w[i] = (uint32_t)bf16_rne(v[2 * i] * sc) | ((uint32_t)bf16_rne(v[2 * i + 1] * sc) << 16);
            return w;
        };
        if (q_bf16) {
            u32x4 raw[NQT][KS];
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const uint16_t *src = (const uint16_t *)q + qbase[nt] + qoff(ks);
                    if constexpr (K16) {
                        const u32x2 r2 = *(const u32x2 *)src;
                        raw[nt][ks] = u32x4{r2[0], r2[1], 0, 0};
                    } else {
                        raw[nt][ks] = *(const u32x4 *)src;
                    }
                }
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[2 * i] = bf16_lo(raw[nt][ks][i]);
                        v[2 * i + 1] = bf16_hi(raw[nt][ks][i]);
                    }
                    qb[nt][ks] = pack_q(v, qv[nt] && dv[ks]);
                }
        } else {
            float4 raw[NQT][KS][2];
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const float4 *src = (const float4 *)((const float *)q + qbase[nt] + qoff(ks));
                    raw[nt][ks][0] = src[0];
                    raw[nt][ks][1] = K16 ? float4{0.f, 0.f, 0.f, 0.f} : src[1];
                }
#pragma unroll
            for (int nt = 0; nt < NQT; nt++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const float4 x = raw[nt][ks][0], y = raw[nt][ks][1];
                    const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
                    qb[nt][ks] = pack_q(v, qv[nt] && dv[ks]);
                }
        }

        // Smallest key limit of the work-group's columns: blocks entirely
        // below it need no mask.
        int kmin = klim[0];
#pragma unroll
        for (int nt = 1; nt < NQT; nt++) kmin = min(kmin, klim[nt]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) kmin = min(kmin, __shfl_xor(kmin, off));
        kmin = __builtin_amdgcn_readfirstlane(kmin);

        float m_run[NQT], l_part[NQT];
        fl4 acc[NQT][MT];
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            m_run[nt] = -INFINITY;
            l_part[nt] = 0.f;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[nt][mt] = fl4{0.f, 0.f, 0.f, 0.f};
        }

        // The cache is streamed once: non-temporal loads keep it from
        // displacing reusable lines (measured ~12% more read bandwidth).
        auto load_block = [&](int j, int pg, u32x4(&kr)[KS], u32x2(&vr)[MT]) {
            const int t0 = tw0 + 64 * j;
            const int page = __builtin_amdgcn_readlane(pg, j & 63);
            const int slot0 = t0 % P;
            const int64_t pbase = ((int64_t)page * KVH + kvh) * kstride;
            const uint16_t *kp = kpool + pbase + (int64_t)slot0 * D + k_lane;
            if constexpr (K16) {
                const u32x2 k2 = __builtin_nontemporal_load((const u32x2 *)kp);
                kr[0] = u32x4{k2[0], k2[1], 0, 0};
            } else {
#pragma unroll
                for (int ks = 0; ks < KS; ks++) kr[ks] = __builtin_nontemporal_load((const u32x4 *)(kp + ks * 512));
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                // scalar base per m-tile + the lane's 32-bit byte offset
                const char *vb = (const char *)(vpool + pbase + slot0 + (int64_t)mt * 16 * P);
                vr[mt] = __builtin_nontemporal_load((const u32x2 *)(vb + v_off));
            }
        };

        auto consume = [&](int j, u32x4(&kr)[KS], u32x2(&vr)[MT]) {
            const int t0 = tw0 + 64 * j;
            // Tokens past the live length sit in the tail page's unused
            // slots: their V must contribute exact zeros whatever bytes they
            // hold.
            if (t0 + 16 > R.len) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (t0 + grp * 4 + jj >= R.len) {
                        const uint32_t keep = (jj & 1) ? 0x0000FFFFu : 0xFFFF0000u;
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) vr[mt][jj >> 1] &= keep;
                    }
                }
            }

            const bool need_mask = t0 + 15 > kmin;
            // Both query tiles step together (scores, softmax, one rescale
            // test, P.V), so the tiles' independent chains interleave.
            fl4 s[NQT];
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) s[nt] = fl4{0.f, 0.f, 0.f, 0.f};
            if constexpr (K16) {
#pragma unroll
                for (int nt = 0; nt < NQT; nt++)
                    s[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        __builtin_bit_cast(sh4, u32x2{kr[0][0], kr[0][1]}),
                        __builtin_bit_cast(sh4, u32x2{qb[nt][0][0], qb[nt][0][1]}), s[nt], 0, 0, 0);
            } else {
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
#pragma unroll
                    for (int nt = 0; nt < NQT; nt++)
                        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[ks]),
                                                                        __builtin_bit_cast(bf16x8, qb[nt][ks]),
                                                                        s[nt], 0, 0, 0);
            }
            float c[NQT];
            u32x2 pw[NQT];
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) {
                if (need_mask) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (t0 + grp * 4 + i > klim[nt]) s[nt][i] = -INFINITY;
                }
                float mx = fmaxf(fmaxf(s[nt][0], s[nt][1]), fmaxf(s[nt][2], s[nt][3]));
                mx = rows4_max(mx);
                const float m_new = fmaxf(m_run[nt], mx);
                // A column that has seen only masked keys keeps m = -inf: its
                // weights and factor come out as exact zeros (acc and l are
                // zero).
                const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
                float p[4];
                c[nt] = __builtin_amdgcn_exp2f(m_run[nt] - m_use);
#pragma unroll
                for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[nt][i] - m_use);
                // The P.V product consumes bf16 weights: normalise by the same
                // ones.
                pw[nt][0] = pack_bf16x2(p[0], p[1]);
                pw[nt][1] = pack_bf16x2(p[2], p[3]);
                l_part[nt] = add_bf16x2(pw[nt][1], add_bf16x2(pw[nt][0], l_part[nt] * c[nt]));
                m_run[nt] = m_new;
            }
            // Rescale only when some column's running max moved (c != 1).
            bool moved = false;
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) moved |= (c[nt] != 1.f);
            if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
                for (int nt = 0; nt < NQT; nt++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[nt][mt] *= c[nt];
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NQT; nt++)
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        __builtin_bit_cast(sh4, vr[mt]), __builtin_bit_cast(sh4, pw[nt]), acc[nt][mt], 0, 0, 0);
        };

        // Two register sets, A and B, alternate without copies so that the
        // next block's loads are always in flight while one block is
        // consumed; the loop is peeled so that every load it issues is
        // unconditional (the waits then count exactly one block of loads
        // still outstanding).
        asm volatile("" ::"v"(pg));
        auto load_next = [&](int j, u32x4(&kr)[KS], u32x2(&vr)[MT]) {
            if ((j & 63) == 0) {
                // Once per 64 blocks: wait for the new ids here, inside the
                // branch, so that no wait for them sits on the common path.
                pg = fetch_pages(j);
                asm volatile("" ::"v"(pg));
            }
            load_block(j, pg, kr, vr);
        };
        u32x4 ka[KS], kb[KS];
        u32x2 va[MT], vb[MT];
        if (nb > 0) load_block(0, pg, ka, va);
        int j = 0;
        for (; j + 2 < nb; j += 2) {
            load_next(j + 1, kb, vb);
            consume(j, ka, va);
            load_next(j + 2, ka, va);
            consume(j + 1, kb, vb);
        }
        if (j + 1 < nb) {
            load_next(j + 1, kb, vb);
            consume(j, ka, va);
            consume(j + 1, kb, vb);
        } else if (j < nb) {
            consume(j, ka, va);
        }

        // ---- merge the 4 waves; wave 0 writes the segment's partial ------
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            const float lt = rows4_sum(l_part[nt]);
            if (grp == 0) {
                sm[wave][nt * 16 + col] = m_run[nt];
                sl[wave][nt * 16 + col] = lt;
            }
            if (wave > 0) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) so[wave - 1][nt][mt][lane] = acc[nt][mt];
            }
        }
        __syncthreads();
        if (wave == 0) {
            // Partial slot of (row r, range wi): r + wi.  A row's ranges are
            // consecutive, so its slots are too (the host sets part and
            // nsplit to match).
            const int pidx = r + wi;
#pragma unroll
            for (int nt = 0; nt < NQT; nt++) {
                const int qr = nt * 16 + col;
                float M = -INFINITY;
#pragma unroll
                for (int w = 0; w < 4; w++) M = fmaxf(M, sm[w][qr]);
                float f[4], L = 0.f;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    f[w] = (sm[w][qr] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sm[w][qr] - M);
                    L += f[w] * sl[w][qr];
                }
                float *po = part_o + (((int64_t)pidx * KVH + kvh) * QRP + qr) * D;
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    fl4 o = acc[nt][mt] * f[0];
#pragma unroll
                    for (int w = 1; w < 4; w++) o += so[w - 1][nt][mt][lane] * f[w];
                    *(fl4 *)(po + mt * 16 + grp * 4) = o;
                }
                if (grp == 0) {
                    float *pm = part_ml + (((int64_t)pidx * KVH + kvh) * QRP + qr) * 2;
                    pm[0] = M;
                    pm[1] = L;
                }
            }
        }
    }
}

// Merge the partials (one per segment of the row) of a (row, kv head) for
// some of its query rows: O = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s,
// written in the caller's layout and dtype.  Work-group = 256 threads over
// TQ = 256 / (D/4) consecutive query rows (blockIdx.z), thread (row j,
// quad d4) owning dims 4 d4 .. 4 d4 + 3 of query row j: one float4 of each
// partial, so a verify call's 32 query rows take 4-8 work-groups instead of
// one each.  With at most kFewParts partials (the usual case) every load is
// issued at once -- one memory round trip -- and each thread computes its
// row's weights itself; with more, the partials are walked in batches of
// kFewParts after a first pass for the maximum.
constexpr int kFewParts = 8;  // partials merged in one round trip

template <bool ARG>
__global__ __launch_bounds__(256) void gqa_combine_kernel(
    typename PlanSel<ARG>::T plan, const AttRow *__restrict__ rows,
    const float *__restrict__ part_o, const float *__restrict__ part_ml, void *__restrict__ out,
    int out_bf16, int layout, int H, int KVH, int D, int DQ, int QRP) {
    const AttRow R = plan_row<ARG>(rows, blockIdx.x);
    const int kvh = blockIdx.y;
    const int Q4 = D >> 2;              // quads per query row
    const int TQ = 256 / Q4;            // query rows per work-group
    const int t = threadIdx.x;
    const int qr = blockIdx.z * TQ + t / Q4;
    const int d0 = (t - (t / Q4) * Q4) * 4;
    const int G = H / KVH;
    if (t >= TQ * Q4 || qr >= G * R.qn) return;
    const int64_t b0 = ((int64_t)R.part * KVH + kvh) * QRP + qr;  // first partial
    const int64_t sstride = (int64_t)KVH * QRP;                    // between partials
    const int n = R.nsplit;
    float M = -INFINITY, L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](float m, float l, const float4 &o) {
        const float f = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - M);
        L += f * l;
        O.x += f * o.x;
        O.y += f * o.y;
        O.z += f * o.z;
        O.w += f * o.w;
    };
    if (n <= kFewParts) {
        // partials past n re-read the last one and get weight 0
        float2 ml[kFewParts];
        float4 ov[kFewParts];
#pragma unroll
        for (int s = 0; s < kFewParts; s++) {
            const int64_t bs = b0 + (int64_t)min(s, n - 1) * sstride;
            ml[s] = *(const float2 *)(part_ml + bs * 2);
            ov[s] = *(const float4 *)(part_o + bs * D + d0);
        }
#pragma unroll
        for (int s = 0; s < kFewParts; s++)
            if (s < n) M = fmaxf(M, ml[s].x);
#pragma unroll
        for (int s = 0; s < kFewParts; s++)
            if (s < n) add(ml[s].x, ml[s].y, ov[s]);
    } else {
        for (int s = 0; s < n; s++) M = fmaxf(M, part_ml[(b0 + (int64_t)s * sstride) * 2]);
        for (int s0 = 0; s0 < n; s0 += kFewParts) {
            float2 ml[kFewParts];
            float4 ov[kFewParts];
#pragma unroll
            for (int s = 0; s < kFewParts; s++) {
                const int64_t bs = b0 + (int64_t)min(s0 + s, n - 1) * sstride;
                ml[s] = *(const float2 *)(part_ml + bs * 2);
                ov[s] = *(const float4 *)(part_o + bs * D + d0);
            }
#pragma unroll
            for (int s = 0; s < kFewParts; s++)
                if (s0 + s < n) add(ml[s].x, ml[s].y, ov[s]);
        }
    }
    if (d0 >= DQ) return;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const float v[4] = {O.x * inv, O.y * inv, O.z * inv, O.w * inv};
    const int ql = qr / G;
    const int h = kvh * G + (qr - ql * G);
    const int qi = R.q0 + ql;
    const int64_t o = (layout == kLayoutSHD) ? ((int64_t)(R.qrow + qi) * H + h) * DQ + d0
                                             : ((int64_t)R.qrow * H + (int64_t)h * R.nq + qi) * DQ + d0;
    // DQ is a multiple of 8: the 4 dims are all in or all out; one store
    // when the caller's buffer is aligned for it
    const bool vec = (((uintptr_t)out) & (out_bf16 ? 7 : 15)) == 0;
    if (out_bf16) {
        uint16_t *dst = (uint16_t *)out + o;
        if (vec) {
            const uint32_t lo = bf16_rne(v[0]) | ((uint32_t)bf16_rne(v[1]) << 16);
            const uint32_t hi = bf16_rne(v[2]) | ((uint32_t)bf16_rne(v[3]) << 16);
            *(uint2 *)dst = make_uint2(lo, hi);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = bf16_rne(v[i]);
        }
    } else {
        float *dst = (float *)out + o;
        if (vec) {
            *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = v[i];
        }
    }
}

template <int D, int NQT, bool ARG>
static hipError_t launch_gqa_t(hipStream_t s, typename PlanSel<ARG>::T plan,
                               const uint16_t *kpool, const uint16_t *vpool,
                               const int32_t *table, const AttRow *rows, int n_rows,
                               const int4 *ranges, int n_ranges, const void *q, int q_bf16,
                               int layout, int H, int KVH, int DQ, int P, int total64, int snap64,
                               int ranges_off, float qscale,
                               int mask_mode, float *part_o, float *part_ml, void *out,
                               int out_bf16, int max_qr, hipEvent_t ev0, hipEvent_t ev1) {
    hipError_t e = launch_timed(gqa_decode_kernel<D, NQT, ARG>, dim3(n_ranges * KVH), dim3(256), s,
                                ev0, ev1, plan, kpool, vpool, table, rows, ranges, n_rows, q, q_bf16,
                                layout, H, KVH, DQ, P, total64, snap64, ranges_off, qscale,
                                mask_mode, part_o, part_ml);
    if (e != hipSuccess) return e;
    constexpr int TQ = 256 / (D / 4);  // query rows per combine work-group
    gqa_combine_kernel<ARG><<<dim3(n_rows, KVH, (max_qr + TQ - 1) / TQ), 256, 0, s>>>(
        plan, rows, part_o, part_ml, out, out_bf16, layout, H, KVH, D, DQ, 16 * NQT);
    return hipGetLastError();
}

hipError_t launch_gqa_decode(hipStream_t s, const PlanArg *plan, const uint16_t *kpool,
                             const uint16_t *vpool, const int32_t *table, const AttRow *rows,
                             int n_rows, const int4 *ranges, int n_ranges, const void *q, int q_bf16,
                             int layout, int H, int KVH, int hd, int hdi, int P, int total64,
                             int snap64, int ranges_off, float qscale,
                             int mask_mode, int nqt, float *part_o, float *part_ml, void *out,
                             int out_bf16, int max_qr, hipEvent_t ev0, hipEvent_t ev1) {
    if (n_ranges <= 0) return hipSuccess;
#define RLX_GQA_CASE(DD, NN)                                                                    \
    if (hd == DD && nqt == NN)                                                                  \
        return plan ? launch_gqa_t<DD, NN, true>(s, *plan, kpool, vpool, table, rows, n_rows,   \
                                                 ranges, n_ranges, q, q_bf16, layout, H, KVH,   \
                                                 hdi, P, total64, snap64, ranges_off,           \
                                                 qscale, mask_mode, part_o, part_ml, out,       \
                                                 out_bf16, max_qr, ev0, ev1)                    \
                    : launch_gqa_t<DD, NN, false>(s, NoPlan{0}, kpool, vpool, table, rows,      \
                                                  n_rows, ranges, n_ranges, q, q_bf16, layout,  \
                                                  H, KVH, hdi, P, total64, snap64, -1, qscale,  \
                                                  mask_mode, part_o, part_ml, out, out_bf16,    \
                                                  max_qr, ev0, ev1);
    RLX_GQA_CASE(128, 1)
    RLX_GQA_CASE(128, 2)
    RLX_GQA_CASE(64, 1)
    RLX_GQA_CASE(64, 2)
    RLX_GQA_CASE(32, 1)
    RLX_GQA_CASE(32, 2)
    RLX_GQA_CASE(16, 1)
    RLX_GQA_CASE(16, 2)
    RLX_GQA_CASE(96, 1)
    RLX_GQA_CASE(96, 2)
    RLX_GQA_CASE(256, 1)
#undef RLX_GQA_CASE
    return hipErrorInvalidValue;
}

}  // namespace rlx
