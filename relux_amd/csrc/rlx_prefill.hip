// Chunked prefill / long verify: FA2-style attention of many query rows over
// the cache, causal with the cache offset (query i of n_q on a sequence of T
// live tokens sees keys <= T - n_q + i).
//
// Work item = (sequence, head group, query tile).  A head group is one kv
// head with its G = H/KVH query heads (GQA) or one head (MLA, decompressed).
// A tile holds 256 query rows, query-major: row r = (token r / G, head r % G),
// so the G heads that share a kv head share every K/V byte the tile loads.
// 8 waves, wave w owns rows [32w, 32w+32) as two 16-wide N tiles.
//
// Keys stream in 32-key blocks through a 4-stage LDS ring filled straight
// from memory (16-byte global-to-LDS loads); each stage holds the block's K
// rows and its V^T rows, both swizzled in 16-byte chunks so that the MFMA
// operand reads are free of bank conflicts.  Per block and wave:
//   S^T[32 keys][16 rows] = K . Q^T    MFMA 16x16x32 bf16 (2 key tiles), A = K
//                                       rows from LDS, B = Q^T in registers
//   online softmax per row, lane-local.  Key tile mt's row m is key
//   8(m/4) + 4mt + m%4, so a lane's S^T values are the 8 consecutive keys
//   8g..8g+7: exactly the B operand P^T of the next product and one 16-byte
//   chunk of a V^T row.
//   O^T[DV][16 rows] += V^T . P^T       MFMA 16x16x32 bf16, A = V^T rows (LDS)
//
// Sources (SRC):
//   kSrcPaged : GQA paged cache, K pages (k-step-major 16-token blocks) and dim-major V pages, DQK = DV = D.
//   kSrcDense : MLA, per sequence decompressed K_c [H][Tp][128] and
//               V^T [H][128][Tp] (Tp = T rounded up to 128) plus the rope key
//               k^R read from the paged latent rows; DQK = 192, DV = 128.
// Keys at or past the live length are masked; the K rows staged for them
// repeat the last live key and their V^T entries are zeroed in LDS, so
// nothing past the live length can reach the output.
#include "rlx_common.h"

namespace rlx {

constexpr int kWaves = 8;                // 512 threads, 32 query rows per wave
constexpr int kTileRows = 32 * kWaves;   // 256
constexpr int kKeyBlock = 32;

__device__ __forceinline__ int pf_limit(int mask_mode, int len, int nq, int qi) {
    if (mask_mode == kMaskCausal) return len - nq + qi;
    if (mask_mode == kMaskRef) return (nq == len) ? qi : len - 1;
    return len - 1;
}


// Swizzles of the ring stages (16-byte chunk index XOR, within aligned
// groups of 8 chunks).  K: the 8 rows one pass of a b128 read touches
// ({0-3, 8-11} + 4mt, and +16) get 8 distinct chunk slots.  V^T (rows of 4
// chunks): 8 consecutive rows get 8 distinct slots.
__device__ __forceinline__ int pf_kswz(int row) { return (row & 3) | ((row >> 1) & 4); }
__device__ __forceinline__ int pf_vswz(int row) { return (row >> 1) & 3; }

template <int DQK, int DV, int SRC>
// The page table is a separate __restrict__ argument so that the compiler
// may read it through the scalar cache: a vector load would be ordered
// behind the in-flight ring loads by the waits the compiler inserts.
__global__ __launch_bounds__(64 * kWaves) void prefill_kernel(const PrefillArgs a,
                                                         const int32_t *__restrict__ table) {
    constexpr int KS = DQK / 32;             // score k-steps
    constexpr int MD = DV / 16;              // value m-tiles
    constexpr int KCH = DQK / 8;             // 16-byte chunks per K row
    constexpr int K_CH = kKeyBlock * KCH;    // K chunks per stage
    constexpr int V_CH = DV * kKeyBlock / 8; // V^T chunks per stage
    constexpr int ST_CH = K_CH + V_CH;
    // Waves 0-3 load the K rows of a block, waves 4-7 its V^T rows.
    constexpr int NK = K_CH / 256;           // K ring loads per K wave per block
    constexpr int NV = V_CH / 256;           // V^T ring loads per V wave per block
    constexpr int S = 4;                     // ring stages (one work-group per CU)
    static_assert(K_CH % 256 == 0 && V_CH % 256 == 0 && KCH % 8 == 0, "stage shape");
    __shared__ __attribute__((aligned(16))) uint16_t ring[S * ST_CH * 8];

    // wave is uniform: branches on it are scalar branches, not exec masks
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int4 wk = a.work[blockIdx.x];
    if (wk.x < 0) return;  // padding item of the XCD-balanced work order
    const AttRow R = a.rows[wk.x];
    const int hg = wk.y;
    const int G = (SRC == kSrcPaged) ? a.H / a.KVH : 1;
    const int toks = kTileRows / G;  // query tokens per tile
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)ring;

    // Keys the tile needs: up to the largest limit of its rows.
    int kend;
    {
        const int jmax = min(R.nq - 1, wk.z * toks + toks - 1);
        kend = min(R.len, pf_limit(a.mask_mode, R.len, R.nq, jmax) + 1);
        if (a.mask_mode == kMaskRef && R.nq != R.len) kend = R.len;
    }
    const int nblk = (kend + kKeyBlock - 1) / kKeyBlock;

    // ---- ring loads of key block j into stage j % S -------------------------
    // K wave w (0-3) fills K chunks (4i + w) * 64 + lane of a stage, V wave
    // w (4-7) fills V^T chunks (4i + w - 4) * 64 + lane.  The same lane
    // fetches the same (row, chunk) of every block, so its offsets are fixed
    // here and each block only adds wave-uniform page bases.
    const bool kwave = wave < 4;
    const int w4 = wave & 3;
    int k_row[NK], k_lc[NK];
    int v_d[NV], v_lc[NV];
    int64_t k_off[NK], v_off[NV];
#pragma unroll
    for (int i = 0; i < NK; i++) {
        const int p = (i * 4 + w4) * 64 + lane;
        k_row[i] = p / KCH;
        k_lc[i] = (p - k_row[i] * KCH) ^ pf_kswz(k_row[i]);
        const int r16 = k_row[i] & 15;
        if (SRC == kSrcPaged)
            k_off[i] = k_page_off(r16, k_lc[i] * 8, DQK);
        else if (k_lc[i] < 16)
            k_off[i] = (int64_t)k_row[i] * 128 + k_lc[i] * 8;
        else
            k_off[i] = (int64_t)r16 * kMlaRow + kMlaDc + (k_lc[i] - 16) * 8;
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int q = (i * 4 + w4) * 64 + lane;
        v_d[i] = q >> 2;
        v_lc[i] = (q & 3) ^ pf_vswz(v_d[i]);
        if (SRC == kSrcPaged)
            v_off[i] = (int64_t)v_d[i] * a.P + (v_lc[i] & 1) * 8;
        else
            v_off[i] = (int64_t)v_d[i] * R.nsplit + v_lc[i] * 8;
    }
    // Page index and slot of key t: shifts when the page size is a power of
    // two (a.pshift >= 0), else a division.
    auto pdiv = [&](int t) { return a.pshift >= 0 ? t >> a.pshift : t / a.P; };
    auto pmod = [&](int t) { return a.pshift >= 0 ? t & (a.P - 1) : t % a.P; };
    auto issue_block = [&](int j) {
        const int k0 = j * kKeyBlock;
        // Keys k0..k0+15 and k0+16..k0+31 each lie in one page (P is a
        // multiple of 16); both page ids are wave-uniform scalar loads.
        int pg0 = 0, pg1 = 0;
        if (SRC == kSrcPaged || DQK > 128) {  // dense: rope keys live in the pages
            pg0 = table[R.tab + pdiv(k0)];
            pg1 = (k0 + 16 < R.len) ? table[R.tab + pdiv(k0 + 16)] : pg0;
        }
        const int s0 = pmod(k0), s1 = pmod(k0 + 16);
        const uint32_t stage = ring_lds + (uint32_t)((j % S) * ST_CH * 16);
        if (k0 + kKeyBlock <= R.len) {
            // Every key of the block is live.
            if (kwave) {
#pragma unroll
            for (int i = 0; i < NK; i++) {
                const bool hi = k_row[i] >= 16;
                const uint16_t *g;
                if (SRC == kSrcPaged) {
                    const uint16_t *b0 = a.kpool + (((int64_t)pg0 * a.KVH + hg) * a.P + s0) * DQK;
                    const uint16_t *b1 = a.kpool + (((int64_t)pg1 * a.KVH + hg) * a.P + s1) * DQK;
                    g = (hi ? b1 : b0) + k_off[i];
                } else if (k_lc[i] < 16) {
                    g = a.kc + ((int64_t)R.part * a.H + (int64_t)hg * R.nsplit + k0) * 128 + k_off[i];
                } else {
                    const uint16_t *b0 = a.kpool + ((int64_t)pg0 * a.P + s0) * kMlaRow;
                    const uint16_t *b1 = a.kpool + ((int64_t)pg1 * a.P + s1) * kMlaRow;
                    g = (hi ? b1 : b0) + k_off[i];
                }
                lds_dma16(g, __builtin_amdgcn_readfirstlane(stage + (uint32_t)((i * 4 + w4) * 64) * 16));
            }
            } else {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const uint16_t *g;
                if (SRC == kSrcPaged) {
                    const bool hi = v_lc[i] >= 2;
                    const uint16_t *b0 = a.vpool + ((int64_t)pg0 * a.KVH + hg) * DV * a.P + s0;
                    const uint16_t *b1 = a.vpool + ((int64_t)pg1 * a.KVH + hg) * DV * a.P + s1;
                    g = (hi ? b1 : b0) + v_off[i];
                } else {
                    g = a.vt + (int64_t)R.part * a.H * 128 + (int64_t)hg * 128 * R.nsplit + k0 + v_off[i];
                }
                lds_dma16(g, __builtin_amdgcn_readfirstlane(stage + (uint32_t)(K_CH + (i * 4 + w4) * 64) * 16));
            }
            }
            return;
        }
        // Last block of the sequence: rows past the live length repeat the
        // last live key; V^T chunks wholly past it load chunk 0 (their
        // entries are zeroed in LDS before use).
        if (kwave) {
#pragma unroll
        for (int i = 0; i < NK; i++) {
            const int row = k_row[i], lc = k_lc[i];
            const int t = min(k0 + row, R.len - 1);
            const int pg = (t - k0 < 16) ? pg0 : pg1;
            const uint16_t *g;
            if (SRC == kSrcPaged)
                g = a.kpool + ((int64_t)pg * a.KVH + hg) * a.P * DQK + k_page_off(pmod(t), lc * 8, DQK);
            else if (lc < 16)
                g = a.kc + ((int64_t)R.part * a.H + (int64_t)hg * R.nsplit + t) * 128 + lc * 8;
            else
                g = a.kpool + ((int64_t)pg * a.P + pmod(t)) * kMlaRow + kMlaDc + (lc - 16) * 8;
            lds_dma16(g, __builtin_amdgcn_readfirstlane(stage + (uint32_t)((i * 4 + w4) * 64) * 16));
        }
        } else {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int d = v_d[i];
            int t = k0 + v_lc[i] * 8;
            if (t >= R.len) t = k0;
            const uint16_t *g;
            if (SRC == kSrcPaged) {
                const int pg = (t - k0 < 16) ? pg0 : pg1;
                g = a.vpool + (((int64_t)pg * a.KVH + hg) * DV + d) * a.P + pmod(t);
            } else {
                g = a.vt + (int64_t)R.part * a.H * 128 + ((int64_t)hg * 128 + d) * R.nsplit + t;
            }
            lds_dma16(g, __builtin_amdgcn_readfirstlane(stage + (uint32_t)(K_CH + (i * 4 + w4) * 64) * 16));
        }
        }
    };
    // Wait for this wave's loads of a block, given how many blocks it issued
    // after it (loads retire in issue order).
    auto wait_block = [&](int ahead) {
        const int n = ahead * (kwave ? NK : NV);
        switch (n) {
            case 0: RLX_WAIT_VM(0); break;
            case 1: RLX_WAIT_VM(1); break;
            case 2: RLX_WAIT_VM(2); break;
            case 3: RLX_WAIT_VM(3); break;
            case 4: RLX_WAIT_VM(4); break;
            case 6: RLX_WAIT_VM(6); break;
            case 8: RLX_WAIT_VM(8); break;
            default: RLX_WAIT_VM(0); break;
        }
    };
    static_assert((S - 2) * NK <= 6 && (S - 2) * NV <= 6, "wait table");

    for (int j = 0; j < S - 1 && j < nblk; j++) issue_block(j);

    // ---- query operand and per-row key limits -----------------------------
    // Rows past the tile's queries load a valid row (no divergent branch
    // around the loads) and are zeroed after.
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
        const int jc = min(j, R.nq - 1);
        const float zs = rvalid[nt] ? a.qscale : 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int d0 = ks * 32 + grp * 8;
            float v[8];
            const void *src;
            int64_t off;
            if (SRC == kSrcPaged || d0 < 128) {
                const int D = (SRC == kSrcPaged) ? DQK : 128;
                src = a.q;
                off = (a.layout == kLayoutSHD || SRC == kSrcDense)
                          ? ((int64_t)(R.qrow + jc) * a.HQ + a.h0 + h) * D + d0
                          : ((int64_t)R.qrow * a.HQ + (int64_t)(a.h0 + h) * R.nq + jc) * D + d0;
            } else {
                src = a.q2;
                off = ((int64_t)(R.qrow + jc) * a.HQ + a.h0 + h) * kMlaDr + (d0 - 128);
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
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = (uint32_t)bf16_rne(v[2 * i] * zs) | ((uint32_t)bf16_rne(v[2 * i + 1] * zs) << 16);
            qb[nt][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }
    // Smallest key limit over this wave's valid rows: blocks entirely below
    // it need no mask.
    int kmin = 0x7fffffff;
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
        if (rvalid[nt]) kmin = min(kmin, klim[nt]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) kmin = min(kmin, __shfl_xor(kmin, off));
    kmin = __builtin_amdgcn_readfirstlane(kmin);
    // Make the compiler complete the query loads here, once: the ring loads
    // are invisible to it, so a wait it placed inside the key loop would
    // also drain the ring on every block.
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) asm volatile("" ::"v"(qb[nt][ks]));

    float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.f, 0.f};
    fl4 acc[2][MD];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
#pragma unroll
        for (int md = 0; md < MD; md++) acc[nt][md] = fl4{0.f, 0.f, 0.f, 0.f};

    // LDS row of key tile mt's m-th row, and this lane's read offsets.
    int krow[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) krow[mt] = (col >> 2) * 8 + mt * 4 + (col & 3);

    for (int j = 0; j < nblk; j++) {
        wait_block(min(S - 2, nblk - 1 - j));
        // Block j is visible to every wave; stage (j-1) % S is no longer read.
        ring_barrier();
        if (j + S - 1 < nblk) issue_block(j + S - 1);
        const int k0 = j * kKeyBlock;
        const uint16_t *Kb = ring + (j % S) * ST_CH * 8;
        const uint16_t *Vb = Kb + K_CH * 8;
        if (k0 + kKeyBlock > R.len) {
            // Last block of the sequence: zero the V^T entries of keys past
            // the live length (they hold stale or repeated cache bytes).
            uint16_t *Vw = ring + (j % S) * ST_CH * 8 + K_CH * 8;
            const int live = R.len - k0;
            for (int e = tid; e < DV * kKeyBlock; e += 64 * kWaves) {
                const int d = e / kKeyBlock, kk = e - d * kKeyBlock;
                if (kk >= live) Vw[d * kKeyBlock + (((kk >> 3) ^ pf_vswz(d)) << 3) + (kk & 7)] = 0;
            }
            ring_barrier();
        }

        fl4 s[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) s[mt][nt] = fl4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const int row = krow[mt];
                const int pc = (ks * 4 + grp) ^ pf_kswz(row);
                const bf16x8 ka = __builtin_bit_cast(bf16x8, *(const u32x4 *)&Kb[row * DQK + pc * 8]);
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[nt][ks], s[mt][nt], 0, 0, 0);
            }
        }
        const bool need_mask = k0 + kKeyBlock - 1 > kmin;
        // V^T fragments of the block (issued early: their LDS latency hides
        // behind the softmax); each N tile's P.V follows its own softmax so
        // that tile 0's MFMAs overlap tile 1's softmax.
        bf16x8 va[MD];
#pragma unroll
        for (int md = 0; md < MD; md++) {
            const int d = md * 16 + col;
            va[md] = __builtin_bit_cast(bf16x8, *(const u32x4 *)&Vb[d * kKeyBlock + ((grp ^ pf_vswz(d)) << 3)]);
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            float p[8];  // keys k0 + 8*grp + i
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) p[mt * 4 + i] = s[mt][nt][i];
            if (need_mask) {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (k0 + grp * 8 + i > klim[nt]) p[i] = -INFINITY;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, p[i]);
            mx = rows4_max(mx);
            const float m_new = fmaxf(m_run[nt], mx);
            // A row that has seen only masked keys keeps m = -inf: its
            // weights and factor come out as exact zeros (acc and l are zero).
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float c = __builtin_amdgcn_exp2f(m_run[nt] - m_use);
#pragma unroll
            for (int i = 0; i < 8; i++) p[i] = __builtin_amdgcn_exp2f(p[i] - m_use);
            // The P.V product consumes bf16 weights: normalise by the same ones.
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
            float lsum = l_part[nt] * c;
#pragma unroll
            for (int i = 0; i < 4; i++) lsum = add_bf16x2(w[i], lsum);
            l_part[nt] = lsum;
            m_run[nt] = m_new;
            // Rescale only when some row's running max moved (c != 1).
            if (__builtin_amdgcn_ballot_w64(c != 1.f)) {
#pragma unroll
                for (int md = 0; md < MD; md++) acc[nt][md] *= c;
            }
            const bf16x8 pbt = __builtin_bit_cast(bf16x8, w);
#pragma unroll
            for (int md = 0; md < MD; md++)
                acc[nt][md] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[md], pbt, acc[nt][md], 0, 0, 0);
        }
    }

    // ---- normalise and write ----------------------------------------------
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const float lt = rows4_sum(l_part[nt]);
        if (!rvalid[nt]) continue;
        const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
        const int j = rtok[nt], h = rhead[nt];
        const int64_t obase = (a.layout == kLayoutSHD || SRC == kSrcDense)
                                  ? ((int64_t)(R.qrow + j) * a.HQ + a.h0 + h) * DV
                                  : ((int64_t)R.qrow * a.HQ + (int64_t)(a.h0 + h) * R.nq + j) * DV;
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
    const dim3 g(n_work), b(64 * kWaves);
    if (src == kSrcPaged && hd == 128)
        return launch_timed(prefill_kernel<128, 128, kSrcPaged>, g, b, s, ev0, ev1, a, a.table);
    if (src == kSrcPaged && hd == 64)
        return launch_timed(prefill_kernel<64, 64, kSrcPaged>, g, b, s, ev0, ev1, a, a.table);
    if (src == kSrcDense && hd == 128)
        return launch_timed(prefill_kernel<192, 128, kSrcDense>, g, b, s, ev0, ev1, a, a.table);
    return hipErrorInvalidValue;
}

}  // namespace rlx
