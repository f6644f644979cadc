// Chunked prefill / long verify: FA2-style attention of many query rows over
// the cache, causal with the cache offset (query i of n_q on a sequence of T
// live tokens sees keys <= T - n_q + i).
//
// Work item = (sequence, head group, query tile).  A head group is one kv
// head with its G = H/KVH query heads (GQA) or one head (MLA, decompressed).
// A tile holds 128 query rows, query-major: row r = (token r / G, head r % G),
// so the G heads that share a kv head share every K/V byte the tile loads.
// 4 waves, wave w owns rows [32w, 32w+32) as two 16-wide N tiles.
//
// Per 32-key block, staged in LDS (double buffered through registers):
//   S^T[32 keys][16 rows] = K . Q^T      MFMA 16x16x32 bf16, A = K rows (LDS),
//                                         B = Q^T in registers (pre-scaled)
//   online softmax per row, lane-local (the S^T result layout is the P^T
//   B-operand layout: the lane's 8 keys are {4g..4g+3, 16+4g..16+4g+3})
//   O^T[DV][16 rows] += V^T . P^T        MFMA 16x16x32 bf16, A = V^T rows (LDS,
//                                         the same 8 keys per lane)
//
// Sources (SRC):
//   kSrcPaged : GQA paged cache, K row pages and dim-major V pages, DQK = DV = D.
//   kSrcDense : MLA, per sequence decompressed K_c [H][Tp][128] and
//               V^T [H][128][Tp] (Tp = T rounded up to 128) plus the rope key
//               k^R read from the paged latent rows; DQK = 192, DV = 128.
// Keys at or past the live length are never read: their K rows and V columns
// are staged as zeros and their scores masked.
#include "rlx_common.h"

namespace rlx {

constexpr int kTileRows = 128;
constexpr int kKeyBlock = 32;

__device__ __forceinline__ float pf_max16(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float pf_sum16(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}
__device__ __forceinline__ int pf_limit(int mask_mode, int len, int nq, int qi) {
    if (mask_mode == kMaskCausal) return len - nq + qi;
    if (mask_mode == kMaskRef) return (nq == len) ? qi : len - 1;
    return len - 1;
}


template <int DQK, int DV, int SRC>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
    constexpr int KS = DQK / 32;          // score k-steps
    constexpr int MD = DV / 16;           // value m-tiles
    constexpr int KP = DQK + 8;           // K row pitch (bf16): 16-byte pad
    constexpr int VP = kKeyBlock + 4;     // V^T row pitch (bf16): 8-byte pad
    constexpr int KCH = kKeyBlock * DQK / 8;  // 16-byte chunks of a K block
    constexpr int VCH = DV * kKeyBlock / 8;   // 16-byte chunks of a V^T block
    constexpr int KPER = (KCH + 255) / 256;
    constexpr int VPER = (VCH + 255) / 256;
    __shared__ uint16_t Ks[2][kKeyBlock * KP];
    __shared__ uint16_t Vs[2][DV * VP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int4 wk = a.work[blockIdx.x];
    const AttRow R = a.rows[wk.x];
    const int hg = wk.y;
    const int G = (SRC == kSrcPaged) ? a.H / a.KVH : 1;
    const int toks = kTileRows / G;  // query tokens per tile

    // ---- query operand and per-row key limits -----------------------------
    bf16x8 qb[2][KS];
    int klim[2];
    bool rvalid[2];
    int rtok[2], rhead[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int r = wave * 32 + nt * 16 + col;
        const int j = wk.z * toks + r / G;
        const int h = hg * G + r % G;
        rtok[nt] = j;
        rhead[nt] = h;
        rvalid[nt] = j < R.nq;
        klim[nt] = rvalid[nt] ? pf_limit(a.mask_mode, R.len, R.nq, j) : -1;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int d0 = ks * 32 + grp * 8;
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (rvalid[nt]) {
                const void *src;
                int64_t off;
                if (SRC == kSrcPaged || d0 < 128) {
                    const int D = (SRC == kSrcPaged) ? DQK : 128;
                    src = a.q;
                    off = (a.layout == kLayoutSHD || SRC == kSrcDense)
                              ? ((int64_t)(R.qrow + j) * a.H + h) * D + d0
                              : ((int64_t)R.qrow * a.H + (int64_t)h * R.nq + j) * D + d0;
                } else {
                    src = a.q2;
                    off = ((int64_t)(R.qrow + j) * a.H + h) * kMlaDr + (d0 - 128);
                }
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
            }
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = (uint32_t)bf16_rne(v[2 * i] * a.qscale) | ((uint32_t)bf16_rne(v[2 * i + 1] * a.qscale) << 16);
            qb[nt][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }

    // Keys the tile needs: up to the largest limit of its rows.
    int kend;
    {
        const int jmax = min(R.nq - 1, wk.z * toks + toks - 1);
        kend = min(R.len, pf_limit(a.mask_mode, R.len, R.nq, jmax) + 1);
        if (a.mask_mode == kMaskRef && R.nq != R.len) kend = R.len;
    }

    // ---- staging of one 32-key block --------------------------------------
    u32x4 kreg[KPER], vreg[VPER];
    auto load_block = [&](int k0) {
#pragma unroll
        for (int u = 0; u < KPER; u++) {
            const int c = tid + 256 * u;
            kreg[u] = u32x4{0, 0, 0, 0};
            if (c < KCH) {
                const int r = c / (DQK / 8), cc = c % (DQK / 8);
                const int t = k0 + r;
                if (t < R.len) {
                    const uint16_t *src;
                    if (SRC == kSrcPaged) {
                        const int page = a.table[R.tab + t / a.P];
                        src = a.kpool + (((int64_t)page * a.KVH + hg) * a.P + (t % a.P)) * DQK + cc * 8;
                    } else if (cc < 16) {
                        src = a.kc + ((int64_t)R.part * a.H + (int64_t)hg * R.nsplit + t) * 128 + cc * 8;
                    } else {
                        const int page = a.table[R.tab + t / a.P];
                        src = a.kpool + ((int64_t)page * a.P + (t % a.P)) * kMlaRow + kMlaDc + (cc - 16) * 8;
                    }
                    kreg[u] = __builtin_nontemporal_load((const u32x4 *)src);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < VPER; u++) {
            const int c = tid + 256 * u;
            vreg[u] = u32x4{0, 0, 0, 0};
            if (c < VCH) {
                const int d = c / (kKeyBlock / 8), part = c % (kKeyBlock / 8);  // 8 keys per chunk
                const int t = k0 + part * 8;
                if (t < R.len) {
                    const uint16_t *src;
                    if (SRC == kSrcPaged) {
                        const int page = a.table[R.tab + t / a.P];
                        src = a.vpool + (((int64_t)page * a.KVH + hg) * DV + d) * a.P + (t % a.P);
                    } else {
                        src = a.vt + (int64_t)R.part * a.H * 128 + ((int64_t)hg * 128 + d) * R.nsplit + t;
                    }
                    u32x4 v = __builtin_nontemporal_load((const u32x4 *)src);
                    // zero the keys of this chunk that lie past the live length
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        if (t + i >= R.len) v[i >> 1] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                    vreg[u] = v;
                }
            }
        }
    };
    auto store_block = [&](int buf) {
#pragma unroll
        for (int u = 0; u < KPER; u++) {
            const int c = tid + 256 * u;
            if (c < KCH) {
                const int r = c / (DQK / 8), cc = c % (DQK / 8);
                *(u32x4 *)&Ks[buf][r * KP + cc * 8] = kreg[u];
            }
        }
#pragma unroll
        for (int u = 0; u < VPER; u++) {
            const int c = tid + 256 * u;
            if (c < VCH) {
                const int d = c / (kKeyBlock / 8), part = c % (kKeyBlock / 8);
                uint16_t *dst = &Vs[buf][d * VP + part * 8];
                *(u32x2 *)dst = u32x2{vreg[u][0], vreg[u][1]};
                *(u32x2 *)(dst + 4) = u32x2{vreg[u][2], vreg[u][3]};
            }
        }
    };

    float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};
    fl4 acc[2][MD];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int md = 0; md < MD; md++) acc[nt][md] = fl4{0.f, 0.f, 0.f, 0.f};

    int buf = 0;
    if (kend > 0) {
        load_block(0);
        store_block(0);
    }
    __syncthreads();
    for (int k0 = 0; k0 < kend; k0 += kKeyBlock) {
        const bool has_next = k0 + kKeyBlock < kend;
        if (has_next) load_block(k0 + kKeyBlock);
        const uint16_t *Kb = Ks[buf];
        const uint16_t *Vb = Vs[buf];
        fl4 s[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) s[mt][nt] = fl4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const bf16x8 ka = __builtin_bit_cast(bf16x8, *(const u32x4 *)&Kb[(mt * 16 + col) * KP + ks * 32 + grp * 8]);
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[nt][ks], s[mt][nt], 0, 0, 0);
            }
        }
        bf16x8 pb[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            float p[8];
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = k0 + mt * 16 + grp * 4 + i;
                    const float v = (t <= klim[nt]) ? s[mt][nt][i] : -INFINITY;
                    p[mt * 4 + i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = pf_max16(mx);
            const float m_new = fmaxf(m_run[nt], mx);
            float c = 1.f;
            if (m_new == -INFINITY) {
#pragma unroll
                for (int i = 0; i < 8; i++) p[i] = 0.f;
            } else {
                c = __builtin_amdgcn_exp2f(m_run[nt] - m_new);
#pragma unroll
                for (int i = 0; i < 8; i++) p[i] = __builtin_amdgcn_exp2f(p[i] - m_new);
            }
            // The P.V product consumes bf16 weights: normalise by the same ones.
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                p[i] = bf16_f32(bf16_rne(p[i]));
                ps += p[i];
            }
            l_part[nt] = l_part[nt] * c + ps;
            m_run[nt] = m_new;
#pragma unroll
            for (int md = 0; md < MD; md++) acc[nt][md] *= c;
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = (uint32_t)bf16_rne(p[2 * i]) | ((uint32_t)bf16_rne(p[2 * i + 1]) << 16);
            pb[nt] = __builtin_bit_cast(bf16x8, w);
        }
#pragma unroll
        for (int md = 0; md < MD; md++) {
            const uint16_t *vr = &Vb[(md * 16 + col) * VP + grp * 4];
            const u32x2 lo = *(const u32x2 *)vr;         // keys 4g .. 4g+3
            const u32x2 hi = *(const u32x2 *)(vr + 16);  // keys 16+4g .. 16+4g+3
            const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                acc[nt][md] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[nt], acc[nt][md], 0, 0, 0);
        }
        if (has_next) store_block(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // ---- normalise and write ----------------------------------------------
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const float lt = pf_sum16(l_part[nt]);
        if (!rvalid[nt]) continue;
        const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
        const int j = rtok[nt], h = rhead[nt];
        const int64_t obase = (a.layout == kLayoutSHD || SRC == kSrcDense)
                                  ? ((int64_t)(R.qrow + j) * a.H + h) * DV
                                  : ((int64_t)R.qrow * a.H + (int64_t)h * R.nq + j) * DV;
#pragma unroll
        for (int md = 0; md < MD; md++) {
            const fl4 o = acc[nt][md] * inv;
            const int64_t off = obase + md * 16 + grp * 4;
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
}

hipError_t launch_prefill(hipStream_t s, int src, int hd, const PrefillArgs &a, int n_work,
                          hipEvent_t ev0, hipEvent_t ev1) {
    if (n_work <= 0) return hipSuccess;
    if (ev0) (void)hipEventRecord(ev0, s);
    if (src == kSrcPaged && hd == 128)
        prefill_kernel<128, 128, kSrcPaged><<<n_work, 256, 0, s>>>(a);
    else if (src == kSrcPaged && hd == 64)
        prefill_kernel<64, 64, kSrcPaged><<<n_work, 256, 0, s>>>(a);
    else if (src == kSrcDense && hd == 128)
        prefill_kernel<192, 128, kSrcDense><<<n_work, 256, 0, s>>>(a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, s);
    return e;
}

}  // namespace rlx
