// GQA flash-decoding over the paged bf16 cache (decode, speculative verify).
//
// Work item = (sequence, context split) x kv head; one 256-thread work-group
// (4 waves) per item.  Each wave walks 16-token blocks of the split:
//
//   S^T[16 tok][16 q-rows] = K_blk[16 x D] . Q^T          (D/32 MFMA 16x16x32 bf16)
//   online softmax per q-row column (lane-local state, exp2 domain)
//   O^T[D][16 q-rows]    += V_blk^T[D x 16 tok] . P^T     (D/16 MFMA 16x16x16 bf16)
//
// The K rows are the A operand straight from a row page (8 consecutive dims
// per lane, 16-byte loads); the V^T tile is the A operand straight from a
// dim-major page (4 consecutive tokens per lane, 8-byte loads); the MFMA
// result layout of S^T is exactly the B-operand layout P^T needs, so no LDS
// and no shuffles sit between the two products.  The query rows of a kv head
// (H/KVH heads x n_q queries) fill the 16-wide N dimension; a second N tile
// covers up to 32 rows.  The 4 waves merge through LDS and write one
// unnormalised partial per split; gqa_combine merges splits (log-sum-exp).
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

template <int D, int NQT, bool ARG>
__global__ __launch_bounds__(256, NQT == 1 ? 3 : 2) void gqa_decode_kernel(
    typename PlanSel<ARG>::T plan, const uint16_t *__restrict__ kpool,
    const uint16_t *__restrict__ vpool, const int32_t *__restrict__ table,
    const AttRow *__restrict__ rows, const int2 *__restrict__ work, int n_rows,
    const void *__restrict__ q, int q_bf16, int layout, int H, int KVH, int P, int chunk,
    float qscale, int mask_mode, float *__restrict__ part_o, float *__restrict__ part_ml) {
    // head_dim 16 holds only 4 dims per lane: its score step is one MFMA
    // 16x16x16 (4 bf16 per lane); wider heads use 16x16x32 k-steps.
    constexpr bool K16 = (D == 16);
    constexpr int KS = K16 ? 1 : D / 32;  // QK k-steps
    constexpr int KW = K16 ? 4 : 8;       // dims per lane per k-step
    constexpr int MT = D / 16;            // PV m-tiles
    constexpr int QRP = 16 * NQT;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int2 wk = plan_work<ARG>(work, n_rows);
    const AttRow R = plan_row<ARG>(rows, wk.x);
    const int kvh = blockIdx.y;
    const int G = H / KVH;
    const int QR = G * R.qn;  // query rows of this (tile of a) sequence
    const int t_begin = wk.y * chunk;
    const int t_end = min(R.len, t_begin + chunk);

    // Q^T operand (B of the score product), pre-scaled by scale*log2(e);
    // KW consecutive dims per lane (the upper half stays zero when KW = 4).
    u32x4 qb[NQT][KS];
    int klim[NQT];
#pragma unroll
    for (int nt = 0; nt < NQT; nt++) {
        const int qr = nt * 16 + col;
        klim[nt] = R.len - 1;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qb[nt][ks] = u32x4{0, 0, 0, 0};
        if (qr < QR) {
            const int ql = qr / G;
            const int h = kvh * G + (qr - ql * G);
            const int qi = R.q0 + ql;
            klim[nt] = key_limit(mask_mode, R.len, R.nq, qi);
            const int64_t base = (layout == kLayoutSHD)
                                     ? ((int64_t)(R.qrow + qi) * H + h) * D
                                     : ((int64_t)R.qrow * H + (int64_t)h * R.nq + qi) * D;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int64_t off = base + ks * 32 + grp * KW;
                float v[8];
                if (q_bf16) {
#pragma unroll
                    for (int i = 0; i < KW; i++) v[i] = bf16_f32(((const uint16_t *)q)[off + i]);
                } else {
#pragma unroll
                    for (int i = 0; i < KW; i += 4) {
                        const float4 f = *(const float4 *)((const float *)q + off + i);
                        v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
                    }
                }
#pragma unroll
                for (int i = 0; i < KW / 2; i++)
                    qb[nt][ks][i] = (uint32_t)bf16_rne(v[2 * i] * qscale) | ((uint32_t)bf16_rne(v[2 * i + 1] * qscale) << 16);
            }
        }
    }

    // Smallest key limit of the work-group's columns: blocks entirely below
    // it need no mask.
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

    const int64_t kstride = (int64_t)P * D;  // one kv head of one page
    // Wave w walks blocks t0 = tw0 + 64 j (j < nb) of 16 tokens.  Block
    // indices are wave-uniform (scalar), and the page ids of 64 blocks are
    // fetched at once, one per lane, and read back with readlane: no table
    // load sits between one block's K/V loads and the next's.
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int tw0 = t_begin + 16 * wv;
    const int nb = (t_end > tw0) ? (t_end - tw0 + 63) / 64 : 0;
    // K blocks are k-step-major (k_page_off): k-step ks of row col sits at
    // ks * 512 + col * 32; head_dim 16 keeps plain rows.
    const int64_t k_lane = K16 ? (int64_t)col * D + grp * KW : (int64_t)col * 32 + grp * 8;
    const int64_t v_lane = (int64_t)col * P + grp * 4;
    auto fetch_pages = [&](int j0) {
        const int j = j0 + lane;
        return (j < nb) ? table[R.tab + (tw0 + 64 * j) / P] : 0;
    };
    // The cache is streamed once: non-temporal loads keep it from
    // displacing reusable lines (measured ~12% more read bandwidth).
    auto load_block = [&](int j, int pg, u32x4(&kr)[KS], u32x2(&vr)[MT]) {
        const int t0 = tw0 + 64 * j;
        const int page = __builtin_amdgcn_readlane(pg, j & 63);
        const int slot0 = t0 % P;
        const int64_t pbase = ((int64_t)page * KVH + kvh) * kstride;
        const uint16_t *kp = kpool + pbase + (int64_t)slot0 * D + k_lane;
        const uint16_t *vp = vpool + pbase + slot0 + v_lane;
        if constexpr (K16) {
            const u32x2 k2 = __builtin_nontemporal_load((const u32x2 *)kp);
            kr[0] = u32x4{k2[0], k2[1], 0, 0};
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kr[ks] = __builtin_nontemporal_load((const u32x4 *)(kp + ks * 512));
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) vr[mt] = __builtin_nontemporal_load((const u32x2 *)(vp + (int64_t)mt * 16 * P));
    };

    auto consume = [&](int j, u32x4(&kr)[KS], u32x2(&vr)[MT]) {
        const int t0 = tw0 + 64 * j;
        // Tokens past the live length sit in the tail page's unused slots:
        // their V must contribute exact zeros whatever bytes they hold.
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
#pragma unroll
        for (int nt = 0; nt < NQT; nt++) {
            fl4 s = fl4{0.f, 0.f, 0.f, 0.f};
            if constexpr (K16) {
                s = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                    __builtin_bit_cast(sh4, u32x2{kr[0][0], kr[0][1]}),
                    __builtin_bit_cast(sh4, u32x2{qb[nt][0][0], qb[nt][0][1]}), s, 0, 0, 0);
            } else {
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[ks]),
                                                                __builtin_bit_cast(bf16x8, qb[nt][ks]), s, 0, 0, 0);
            }
            if (need_mask) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (t0 + grp * 4 + i > klim[nt]) s[i] = -INFINITY;
            }
            float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mx = rows4_max(mx);
            const float m_new = fmaxf(m_run[nt], mx);
            float c, p[4];
            if (m_new == -INFINITY) {
                c = 1.f;
                p[0] = p[1] = p[2] = p[3] = 0.f;
            } else {
                c = __builtin_amdgcn_exp2f(m_run[nt] - m_new);
#pragma unroll
                for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[i] - m_new);
            }
            // The P.V product consumes bf16 weights: normalise by the same ones.
            u32x2 pw;
            pw[0] = pack_bf16x2(p[0], p[1]);
            pw[1] = pack_bf16x2(p[2], p[3]);
            l_part[nt] = l_part[nt] * c + ((bf16_lo(pw[0]) + bf16_hi(pw[0])) + (bf16_lo(pw[1]) + bf16_hi(pw[1])));
            m_run[nt] = m_new;
            // Rescale only when some column's running max moved (c != 1).
            if (__builtin_amdgcn_ballot_w64(c != 1.f)) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) acc[nt][mt] *= c;
            }
            const sh4 pb = __builtin_bit_cast(sh4, pw);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(sh4, vr[mt]), pb, acc[nt][mt], 0, 0, 0);
        }
    };

    // Two register sets, A and B, alternate without copies so that the next
    // block's loads are always in flight while one block is consumed; the
    // loop is peeled so that every load it issues is unconditional (the
    // waits then count exactly one block of loads still outstanding).
    int pg = fetch_pages(0);
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

    // ---- merge the 4 waves of the work-group -------------------------------
    __shared__ float sm[4][QRP], sl[4][QRP];
    __shared__ fl4 so[3][NQT][MT][64];
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
    if (wave != 0) return;
    const int pidx = R.part + wk.y;
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

// Merge the splits of one (sequence, kv head, query row): O = sum_s
// 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s, written in the caller's layout and
// dtype.  One block of D threads per query row; the merge weights are
// computed once in LDS and every thread streams its dim across the splits.
template <bool ARG>
__global__ __launch_bounds__(128) void gqa_combine_kernel(
    typename PlanSel<ARG>::T plan, const AttRow *__restrict__ rows,
    const float *__restrict__ part_o, const float *__restrict__ part_ml, void *__restrict__ out,
    int out_bf16, int layout, int H, int KVH, int D, int QRP) {
    const AttRow R = plan_row<ARG>(rows, blockIdx.x);
    const int kvh = blockIdx.y;
    const int qr = blockIdx.z;
    const int G = H / KVH;
    if (qr >= G * R.qn) return;
    __shared__ float fac[kMaxSplits];
    __shared__ float inv_l;
    const int64_t b0 = ((int64_t)R.part * KVH + kvh) * QRP + qr;  // split 0
    const int64_t sstride = (int64_t)KVH * QRP;                    // between splits
    merge_weights(part_ml + b0 * 2, sstride, R.nsplit, fac, &inv_l);
    __syncthreads();
    const int ql = qr / G;
    const int h = kvh * G + (qr - ql * G);
    const int qi = R.q0 + ql;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float O = 0.f;
        for (int s = 0; s < R.nsplit; s++) O += fac[s] * part_o[(b0 + s * sstride) * D + d];
        const float v = O * inv_l;
        const int64_t o = (layout == kLayoutSHD)
                              ? ((int64_t)(R.qrow + qi) * H + h) * D + d
                              : ((int64_t)R.qrow * H + (int64_t)h * R.nq + qi) * D + d;
        if (out_bf16)
            ((uint16_t *)out)[o] = bf16_rne(v);
        else
            ((float *)out)[o] = v;
    }
}

template <int D, int NQT, bool ARG>
static hipError_t launch_gqa_t(hipStream_t s, typename PlanSel<ARG>::T plan,
                               const uint16_t *kpool, const uint16_t *vpool,
                               const int32_t *table, const AttRow *rows, int n_rows,
                               const int2 *work, int n_work, const void *q, int q_bf16,
                               int layout, int H, int KVH, int P, int chunk, float qscale,
                               int mask_mode, float *part_o, float *part_ml, void *out,
                               int out_bf16, int max_qr, hipEvent_t ev0, hipEvent_t ev1) {
    if (ev0) (void)hipEventRecord(ev0, s);
    gqa_decode_kernel<D, NQT, ARG><<<dim3(n_work, KVH), 256, 0, s>>>(
        plan, kpool, vpool, table, rows, work, n_rows, q, q_bf16, layout, H, KVH, P, chunk, qscale,
        mask_mode, part_o, part_ml);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ev1) (void)hipEventRecord(ev1, s);
    gqa_combine_kernel<ARG><<<dim3(n_rows, KVH, max_qr), (D < 64 ? 64 : D), 0, s>>>(
        plan, rows, part_o, part_ml, out, out_bf16, layout, H, KVH, D, 16 * NQT);
    return hipGetLastError();
}

hipError_t launch_gqa_decode(hipStream_t s, const PlanArg *plan, const uint16_t *kpool,
                             const uint16_t *vpool, const int32_t *table, const AttRow *rows,
                             int n_rows, const int2 *work, int n_work, const void *q, int q_bf16,
                             int layout, int H, int KVH, int hd, int P, int chunk, float qscale,
                             int mask_mode, int nqt, float *part_o, float *part_ml, void *out,
                             int out_bf16, int max_qr, hipEvent_t ev0, hipEvent_t ev1) {
    if (n_work <= 0) return hipSuccess;
#define RLX_GQA_CASE(DD, NN)                                                                    \
    if (hd == DD && nqt == NN)                                                                  \
        return plan ? launch_gqa_t<DD, NN, true>(s, *plan, kpool, vpool, table, rows, n_rows, work, \
                                                 n_work, q, q_bf16, layout, H, KVH, P, chunk,   \
                                                 qscale, mask_mode, part_o, part_ml, out,       \
                                                 out_bf16, max_qr, ev0, ev1)                    \
                    : launch_gqa_t<DD, NN, false>(s, NoPlan{0}, kpool, vpool, table, rows,      \
                                                  n_rows, work, n_work, q, q_bf16, layout, H,   \
                                                  KVH, P, chunk, qscale, mask_mode, part_o,     \
                                                  part_ml, out, out_bf16, max_qr, ev0, ev1);
    RLX_GQA_CASE(128, 1)
    RLX_GQA_CASE(128, 2)
    RLX_GQA_CASE(64, 1)
    RLX_GQA_CASE(64, 2)
    RLX_GQA_CASE(32, 1)
    RLX_GQA_CASE(32, 2)
    RLX_GQA_CASE(16, 1)
    RLX_GQA_CASE(16, 2)
#undef RLX_GQA_CASE
    return hipErrorInvalidValue;
}

}  // namespace rlx
