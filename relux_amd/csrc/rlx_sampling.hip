// Token selection on the device: Sampler.Greedy, Sampler.Sample and the
// speculative decoder's acceptPhase / resampleRejected, with 512-thread
// work-groups.
//
// Launch shapes:
//   * Greedy, and Sample without top-k, with top-k above kPartMaxK, or on a
//     vocabulary of at most kPartChunk entries: one work-group per row
//     (the whole-row path below).
//   * Sample with top-k on a larger vocabulary (the split path):
//     sample_part_kernel, one work-group per (row, chunk of at most
//     kPartChunk entries), holds its chunk in registers, applies the
//     penalties and writes, in index order, the entries at or above a
//     lower bound of the chunk's k-th largest undivided logit (with a
//     16-key margin for the temperature division still to come) plus a
//     record {count, lower bound, largest key}; sample_kernel then merges a
//     row's lists in one load round trip, divides by the temperature, finds
//     the exact k-th largest by radix select over the key range the records
//     leave open, and finishes the short list.  A list past its slots or a
//     merge past kCandCap sends the row down the whole-row path.
//   * acceptPhase + resampleRejected: spec_stat_kernel (per row, draft
//     position and side: softmaxAlloc's max, sum and the draft token's
//     probability, all drafts at once; further work-groups cut the next
//     target row into the split path's chunk lists), spec_mass_kernel (per
//     row and chunk: the first rejection, then that position's chunk sums
//     of max(0, p_t - p_d) and of p_t) and spec_final_kernel (the draw).
//
// Reference: sampler.go:56-68 (Greedy), 73-210 (Sample: penalties ->
// temperature -> top-k -> fastexp32 softmax -> top-p -> min-p -> categorical
// draw), 213-262 (penalties); speculative.go:203-290 (acceptance test
// r < min(1, p_t/p_d), resample from norm(max(0, p_t - p_d))), 344-368
// (softmaxAlloc).  Each rng.Float32() draw is an input.
//
// Whole-row working set.  Sample first brings the row's scratch values (logits after
// penalties and temperature, sampler.go:80-97) into LDS when the vocabulary
// fits (<= 32768 entries: 128 KB), applying the penalties in place on the
// row's distinct window tokens; larger vocabularies are re-read from memory
// each pass, with the penalised tokens found through an LDS bitmap.  With
// top-k on, the tokens at or above the k-th largest value are compacted, in
// index order, into an LDS candidate list (<= 2048 entries) and every later
// stage runs over that list only (its top-p search by one wave, with the
// probabilities in registers).  Once the softmax is known the working set
// holds probabilities in place.
//
// The reference sorts (argsortDescF32, kthLargest: selection sorts) and sums
// the vocabulary sequentially.  Here:
//   * the top-k threshold (k-th largest value) is found one key bit at a
//     time on the float's order-preserving key: first a lower bound, the
//     k-th largest of the per-thread maxima to 16 key bits, then the exact
//     value (32 counting steps) on the short list of entries at or above
//     that bound; the single-wave searches are instantiated for the
//     64-entry register groups in use, so a list of 100 entries costs one
//     ballot per step;
//   * the top-p cutoff is the key tau of the item where the descending
//     cumulative probability first reaches p, i.e. the largest tau whose
//     tail sum still reaches p: 31 bisection steps over probabilities kept
//     in LDS; every item with key >= tau is kept (the reference keeps only
//     as many items tied at tau as its sort order reaches: the one place
//     the results can differ besides rounding);
//   * sums are per-thread sequential partials combined in a fixed order
//     (64-lane trees, then the 8 wave results in order), so a call is
//     deterministic; they round differently from a sequential sum by a few
//     ulp, which moves a draw only when r lies within that of a cumulative
//     boundary;
//   * the categorical draw: per-thread chunk sums, an ordered exclusive
//     scan, then each thread walks its chunk; the lowest hit wins.
// Arithmetic follows the reference's f32 order with explicitly rounded
// operations (no fused multiply-add): s/temp, fastexp32(x - max) with one
// multiply and one add (mha.go:823-833), p * f32(1/sum).
#include <type_traits>

#include "rlx_common.h"

namespace rlx {

constexpr int kST = 512;            // threads per row
constexpr int kSW = kST / 64;       // waves per row
constexpr int kRowCap = 32768;      // LDS row region (floats)
constexpr int kCandCap = 2048;      // compacted top-k candidates
constexpr int kSeenOff = 8192;      // region words: bitmap [0, 8192), seen tokens, values
constexpr int kTileOff = 16384;     // region words: tile counts of a memory-resident row
static_assert(kSampMaxVocab / 32 <= kSeenOff, "bitmap must fit before the seen list");
static_assert(kSeenOff + 2 * kSampMaxSeen <= kTileOff, "seen list must fit before the tile counts");
static_assert(kTileOff + kSampMaxVocab / 64 <= kRowCap, "tile counts must fit in the region");
static_assert(kRowCap / 64 <= kST, "LDS-row tile counts use one slot per thread");

__device__ __forceinline__ float fastexp32_dev(float x) {
    if (x < -87.f) return 0.f;
    if (x > 87.f) return __uint_as_float(0x7F800000u);
    const float factor = 12102203.0f;  // f32(2^23 / ln 2)
    const float bias = 1064948224.0f;  // f32(127 * 2^23 - 405000)
    return __int_as_float((int)__fadd_rn(__fmul_rn(factor, x), bias));
}

// Order-preserving map of a float to uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// Lanes below this one whose bit is set in m.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

struct SampLds {
    float red[2][kSW];
    int cnt[kST];
    uint32_t key[kST];
    int tiles[kRowCap / 64];
    int sel_i[2];
    float sel_f;
    int best;
    union {
        struct {
            float cv[kCandCap];
            int ci[kCandCap];
        };
        // a device-counted repetition window until the row is loaded:
        // id | count << 18 per distinct id, ascending
        uint32_t win[2 * kCandCap];
    };
    float region[kRowCap];
};
static_assert(2 * kCandCap == kSampMaxSeen, "the window list fills the candidate arrays");
static_assert(kSampMaxVocab <= (1 << 18) && kSampMaxSeen < (1 << 13), "id | count << 18 fits 31 bits");

// ---- block-wide reductions and scans: fixed combination order, every
// thread gets the same result --------------------------------------------
// Wave reductions in the VALU pipeline: DPP row shifts 1, 2, 4, 8 leave each
// 16-lane row's total in its lane 15, row_bcast 15 / 31 carry them up; lane
// 63 ends with the wave's total.
#define RLX_DPP(v, ctrl, rmask, ident)                                                              \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, (float)(ident)),   \
                                                          __builtin_bit_cast(int, v), ctrl, rmask, 0xF, false))
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += RLX_DPP(v, 0x111, 0xF, 0.f);
    v += RLX_DPP(v, 0x112, 0xF, 0.f);
    v += RLX_DPP(v, 0x114, 0xF, 0.f);
    v += RLX_DPP(v, 0x118, 0xF, 0.f);
    v += RLX_DPP(v, 0x142, 0xA, 0.f);
    v += RLX_DPP(v, 0x143, 0xC, 0.f);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, RLX_DPP(v, 0x111, 0xF, -INFINITY));
    v = fmaxf(v, RLX_DPP(v, 0x112, 0xF, -INFINITY));
    v = fmaxf(v, RLX_DPP(v, 0x114, 0xF, -INFINITY));
    v = fmaxf(v, RLX_DPP(v, 0x118, 0xF, -INFINITY));
    v = fmaxf(v, RLX_DPP(v, 0x142, 0xA, -INFINITY));
    v = fmaxf(v, RLX_DPP(v, 0x143, 0xC, -INFINITY));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
template <class L>
__device__ __forceinline__ void blk_sum2(float &a, float &b, L &s) {
    a = wave_sum_dpp(a);
    b = wave_sum_dpp(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        s.red[0][threadIdx.x >> 6] = a;
        s.red[1][threadIdx.x >> 6] = b;
    }
    __syncthreads();
    a = s.red[0][0];
    b = s.red[1][0];
#pragma unroll
    for (int w = 1; w < kSW; w++) {
        a += s.red[0][w];
        b += s.red[1][w];
    }
}
template <class L>
__device__ __forceinline__ void blk_max2(float &a, float &b, L &s) {
    a = wave_max_dpp(a);
    b = wave_max_dpp(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        s.red[0][threadIdx.x >> 6] = a;
        s.red[1][threadIdx.x >> 6] = b;
    }
    __syncthreads();
    a = s.red[0][0];
    b = s.red[1][0];
#pragma unroll
    for (int w = 1; w < kSW; w++) {
        a = fmaxf(a, s.red[0][w]);
        b = fmaxf(b, s.red[1][w]);
    }
}
template <class L>
__device__ __forceinline__ float blk_sum(float v, L &s) {
    float z = 0.f;
    blk_sum2(v, z, s);
    return v;
}
template <class L>
__device__ __forceinline__ float blk_max(float v, L &s) {
    float z = -INFINITY;
    blk_max2(v, z, s);
    return v;
}
// The same DPP sequence leaves every lane with its inclusive prefix.
__device__ __forceinline__ float wave_scan_dpp(float v) {
    v += RLX_DPP(v, 0x111, 0xF, 0.f);
    v += RLX_DPP(v, 0x112, 0xF, 0.f);
    v += RLX_DPP(v, 0x114, 0xF, 0.f);
    v += RLX_DPP(v, 0x118, 0xF, 0.f);
    v += RLX_DPP(v, 0x142, 0xA, 0.f);
    v += RLX_DPP(v, 0x143, 0xC, 0.f);
    return v;
}
#define RLX_DPPI(v, ctrl, rmask) __builtin_amdgcn_update_dpp(0, v, ctrl, rmask, 0xF, false)
__device__ __forceinline__ int wave_iscan_dpp(int v) {
    v += RLX_DPPI(v, 0x111, 0xF);
    v += RLX_DPPI(v, 0x112, 0xF);
    v += RLX_DPPI(v, 0x114, 0xF);
    v += RLX_DPPI(v, 0x118, 0xF);
    v += RLX_DPPI(v, 0x142, 0xA);
    v += RLX_DPPI(v, 0x143, 0xC);
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x111, 0xF));
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x112, 0xF));
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x114, 0xF));
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x118, 0xF));
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x142, 0xA));
    v = max(v, (uint32_t)RLX_DPPI((int)v, 0x143, 0xC));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
template <class L>
__device__ __forceinline__ float blk_scan_excl(float v, L &s, float *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float inc = wave_scan_dpp(v);
    const float exc = RLX_DPP(inc, 0x138, 0xF, 0.f);  // wave_shr:1, lane 0 gets 0
    __syncthreads();
    if (lane == 63) s.red[0][w] = inc;
    __syncthreads();
    float base = 0.f, tot = 0.f;
    for (int i = 0; i < kSW; i++) {
        if (i < w) base += s.red[0][i];
        tot += s.red[0][i];
    }
    *total = tot;
    return base + exc;
}
template <class L>
__device__ __forceinline__ int blk_iscan_excl(int v, L &s, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int inc = wave_iscan_dpp(v);
    __syncthreads();
    if (lane == 63) s.cnt[w] = inc;
    __syncthreads();
    int base = 0, tot = 0;
    for (int i = 0; i < kSW; i++) {
        if (i < w) base += s.cnt[i];
        tot += s.cnt[i];
    }
    __syncthreads();
    *total = tot;
    return base + inc - v;
}
template <class L>
__device__ __forceinline__ int blk_isum(int v, L &s) {
    int t;
    blk_iscan_excl(v, s, &t);
    return t;
}

// ---- the working set ------------------------------------------------------
struct Src {
    int mode;  // 0: LDS row region, 1: LDS candidate list, 2: memory
    int n;     // entries
    const float *row;
    int V;
    int nseen;  // mode 2: penalised tokens (bitmap + list in the region)
    float temp;
    bool div;
    bool topk;  // mode 2 without compaction: mask below kthr
    float kthr;
    float m;
    bool n1;
    float i1;
    bool topp;
    uint32_t tau;
    bool n2;
    float i2;
    bool minp;
    float thr3;
    bool n3;
    float i3;
};

// Scratch value of working-set entry i (sampler.go:80-114).  M is the
// storage mode as a template parameter, so each pass compiles to plain LDS
// reads (modes 0, 1) or to the memory path (mode 2) alone.
template <int M>
__device__ __forceinline__ float wval(const Src &c, const SampLds &s, int i) {
    if constexpr (M == 0) return s.region[i];
    if constexpr (M == 1) return s.cv[i];
    float x;
    const uint32_t *bits = (const uint32_t *)s.region;
    if (c.nseen > 0 && ((bits[i >> 5] >> (i & 31)) & 1u)) {
        const int *stok = (const int *)(s.region + kSeenOff);
        const float *sv = s.region + kSeenOff + kSampMaxSeen;
        int lo = 0, hi = c.nseen - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (stok[mid] < i)
                lo = mid + 1;
            else
                hi = mid;
        }
        x = sv[lo];
    } else {
        x = c.row[i];
    }
    if (c.div) x = __fdiv_rn(x, c.temp);
    if (c.topk && x < c.kthr) x = -INFINITY;
    return x;
}
template <int M>
__device__ __forceinline__ int widx(const SampLds &s, int i) {
    if constexpr (M == 1) return s.ci[i];
    return i;
}
// Stage-1 probability of entry i: stored in place once the softmax is known
// (modes 0 and 1), recomputed from the value in mode 2.
template <int M>
__device__ __forceinline__ float wp1(const Src &c, const SampLds &s, int i) {
    if constexpr (M == 0) return s.region[i];
    if constexpr (M == 1) return s.cv[i];
    const float x = wval<2>(c, s, i);
    const float p = (x == -INFINITY) ? 0.f : fastexp32_dev(__fsub_rn(x, c.m));
    return c.n1 ? __fmul_rn(p, c.i1) : p;
}
// Probability after stage `stage` (1 softmax, 2 top-p, 3 min-p).
template <int M>
__device__ __forceinline__ float wprob(const Src &c, const SampLds &s, int i, int stage) {
    float p = wp1<M>(c, s, i);
    if (stage >= 2 && c.topp) {
        p = (fkey(p) >= c.tau) ? p : 0.f;
        if (c.n2) p = __fmul_rn(p, c.i2);
    }
    if (stage >= 3 && c.minp) {
        p = (p < c.thr3) ? 0.f : p;
        if (c.n3) p = __fmul_rn(p, c.i3);
    }
    return p;
}

// ---- selection building blocks --------------------------------------------

// Largest key t with #{i < n : key(i) >= t} >= k (the k-th largest key),
// one bit per step, by wave 0 with the n <= kCandCap keys in registers.
// Calls f(std::integral_constant<int, G>) with G the power of two >= the
// number of 64-entry register groups that n entries need (at most R), so
// the group loops are unrolled to exactly the groups in use.
template <int R, class F>
__device__ __forceinline__ void with_groups(int n, F f) {
    const int g = __builtin_amdgcn_readfirstlane((n + 63) >> 6);
    if (g <= 1) f(std::integral_constant<int, 1>{});
    else if (g <= 2) f(std::integral_constant<int, 2>{});
    else if (g <= 4) f(std::integral_constant<int, 4>{});
    else if (g <= 8 || R <= 8) f(std::integral_constant<int, (R < 8 ? R : 8)>{});
    else if (g <= 16 || R <= 16) f(std::integral_constant<int, (R < 16 ? R : 16)>{});
    else f(std::integral_constant<int, R>{});
}

// With lo_bit > 0 only the key bits above lo_bit are searched: the result
// is then a lower bound of the k-th largest key (its low bits zero).
template <class L, class K>
__device__ uint32_t kth_key_w0(int n, int k, L &s, K key, int lo_bit = 0) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        with_groups<kCandCap / 64>(n, [&](auto gc) {
            constexpr int G = decltype(gc)::value;
            uint32_t kk[G];
#pragma unroll
            for (int j = 0; j < G; j++) kk[j] = (lane + 64 * j < n) ? key(lane + 64 * j) : 0u;
            uint32_t res = 0;
            for (int bit = 31; bit >= lo_bit; bit--) {
                const uint32_t cand = res | (1u << bit);
                int cnt = 0;  // per-key ballots, counted on the scalar unit
#pragma unroll
                for (int j = 0; j < G; j++) cnt += (int)__popcll(__ballot(kk[j] >= cand));
                if (cnt >= k) res = cand;
            }
            if (lane == 0) s.sel_i[0] = (int)res;
        });
    }
    __syncthreads();
    const uint32_t r = (uint32_t)s.sel_i[0];
    __syncthreads();
    return r;
}
// The same over the whole working set with every thread (n entries).
template <class L, class K>
__device__ uint32_t kth_key_blk(int n, int k, L &s, K key) {
    uint32_t res = 0;
    for (int bit = 31; bit >= 0; bit--) {
        const uint32_t cand = res | (1u << bit);
        int cnt = 0;
        for (int i = threadIdx.x; i < n; i += kST) cnt += key(i) >= cand;
        if (blk_isum(cnt, s) >= k) res = cand;
    }
    return res;
}

// Entries i < n with keep(i), in index order, into the candidate list
// (value val(i), index idx(i)); returns their count and writes nothing if
// it exceeds kCandCap.  64-entry tiles: a ballot per tile, an ordered scan
// of the tile counts, then each kept entry's slot is its tile's offset plus
// the kept lanes below it.
template <class L, class P, class Vf, class If>
__device__ int compact_blk(int n, int *tc, L &s, P keep, Vf val, If idx) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T = (n + 63) / 64;
#pragma unroll 8
    for (int t = wave; t < T; t += kSW) {
        const int i = 64 * t + lane;
        const uint64_t m = __ballot(i < n && keep(i));
        if (lane == 0) tc[t] = (int)__popcll(m);
    }
    __syncthreads();
    const int TP = (T + kST - 1) / kST;
    const int t0 = min(T, (int)threadIdx.x * TP), t1 = min(T, t0 + TP);
    int mine = 0;
    for (int t = t0; t < t1; t++) mine += tc[t];
    int total;
    int off = blk_iscan_excl(mine, s, &total);
    for (int t = t0; t < t1; t++) {
        const int c = tc[t];
        tc[t] = off;
        off += c;
    }
    __syncthreads();
    if (total > kCandCap) return total;
#pragma unroll 8
    for (int t = wave; t < T; t += kSW) {
        const int i = 64 * t + lane;
        const bool k = i < n && keep(i);
        const uint64_t m = __ballot(k);
        if (k) {
            const int pos = tc[t] + lanes_below(m);
            s.cv[pos] = val(i);
            s.ci[pos] = idx(i);
        }
    }
    __syncthreads();
    return total;
}

// compact_blk for n <= 64 * kST entries (the LDS row): thread t owns the
// contiguous entries [t C, t C + C), C = ceil(n / kST) <= 64, marks the kept
// ones in a 64-bit mask and an ordered exclusive scan of the counts gives
// its first slot.  One pass over the entries; index order is kept.  (With C
// odd the lanes of a wave read distinct banks; C = 64, a 32768 row, reads
// one bank per step.)
template <class L, class P, class Vf>
__device__ int compact_chunks(int n, L &s, P keep, Vf val) {
    const int tid = threadIdx.x;
    const int C = (n + kST - 1) / kST;
    const int i0 = tid * C;
    uint64_t m = 0;
    for (int j = 0; j < C; j++) {
        const int i = i0 + j;
        if (i < n && keep(i)) m |= 1ull << j;
    }
    int total;
    int off = blk_iscan_excl((int)__popcll(m), s, &total);
    if (total > kCandCap) return total;
    while (m) {
        const int j = __builtin_ctzll(m);
        m &= m - 1;
        s.cv[off] = val(i0 + j);
        s.ci[off] = i0 + j;
        off++;
    }
    __syncthreads();
    return total;
}

// Filter the candidate list in place, in order (wave 0, one 64-entry tile
// after another: a tile is read before any slot at or below it is written).
template <class L, class P>
__device__ int filter_w0(int n, L &s, P keep) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        int out = 0;
        for (int t = 0; t < n; t += 64) {
            const int i = t + lane;
            const bool in = i < n;
            const float v = in ? s.cv[i] : 0.f;
            const int x = in ? s.ci[i] : 0;
            const bool k = in && keep(v);
            const uint64_t m = __ballot(k);
            if (k) {
                s.cv[out + lanes_below(m)] = v;
                s.ci[out + lanes_below(m)] = x;
            }
            out += (int)__popcll(m);
        }
        if (lane == 0) s.sel_i[0] = out;
    }
    __syncthreads();
    const int r = s.sel_i[0];
    __syncthreads();
    return r;
}

// First entry (in order) at which the running sum of w, started at `base`,
// exceeds r, or -1 when none does; *tot: the sum of the n weights.  Chunk
// sums per thread (contiguous chunks), an ordered exclusive scan, then only
// the thread whose chunk holds r walks it; should rounding leave that walk
// without a hit, every later chunk is walked.
template <class L, class W>
__device__ int samp_draw_from(int n, float r, float base, L &s, W w, float *tot) {
    const int tid = threadIdx.x;
    const int C = (n + kST - 1) / kST;
    const int i0 = min(n, tid * C), i1 = min(n, i0 + C);
    float cs = 0.f;
#pragma unroll 8
    for (int i = i0; i < i1; i++) cs += w(i);
    const float start = base + blk_scan_excl(cs, s, tot);
    if (tid == 0) s.best = INT_MAX;
    __syncthreads();
    auto walk = [&]() {
        float cum = start;
        for (int i = i0; i < i1; i++) {
            cum += w(i);
            if (r < cum) {
                atomicMin(&s.best, i);
                break;
            }
        }
    };
    if (!(r < start) && r < start + cs) walk();
    __syncthreads();
    if (s.best == INT_MAX) {
        if (r < start + cs) walk();
        __syncthreads();
    }
    const int b = s.best;
    __syncthreads();
    return b == INT_MAX ? -1 : b;
}
// The same over a whole set: the hit mapped through idx, `dflt` when r is
// never reached.
template <class L, class W, class I>
__device__ int samp_draw(int n, float r, int dflt, L &s, W w, I idx) {
    float tot;
    const int b = samp_draw_from(n, r, 0.f, s, w, &tot);
    return b < 0 ? dflt : idx(b);
}

// ---- Sampler.Sample ---------------------------------------------------------

// Top-k (sampler.go:100-114) on a row in mode M (0 or 2): keep the values >=
// the k-th largest.  Lower bound: the k-th largest of the per-thread maxima
// (k distinct entries, so <= the k-th largest of all); the entries at or
// above it are compacted in index order and the exact threshold is found
// within that list, which then becomes the working set (mode 1).  If the
// list would not fit, the threshold is searched over the whole row.
template <int M>
__device__ __forceinline__ void topk_select(Src &c, int top_k, SampLds &s) {
    const int tid = threadIdx.x;
    auto vkey = [&](int i) { return fkey(wval<M>(c, s, i)); };
    if (top_k <= kST) {
        uint32_t mk = 0;
#pragma unroll 8
        for (int i = tid; i < c.n; i += kST) mk = max(mk, vkey(i));
        s.key[tid] = mk;
        __syncthreads();
        // a lower bound of the k-th largest maximum is enough here (the
        // exact threshold is searched in the list): 16 key bits
        const uint32_t lb = kth_key_w0(kST, top_k, s, [&](int i) { return s.key[i]; }, 16);
        int total;
        if constexpr (M == 0) {
            static_assert(kRowCap <= 64 * kST, "an LDS row is at most 64 entries per thread");
            total = compact_chunks(
                c.n, s, [&](int i) { return vkey(i) >= lb; }, [&](int i) { return wval<M>(c, s, i); });
        } else {
            total = compact_blk(
                c.n, (int *)(s.region + kTileOff), s, [&](int i) { return vkey(i) >= lb; },
                [&](int i) { return wval<M>(c, s, i); }, [&](int i) { return i; });
        }
        if (total <= kCandCap) {
            c.mode = 1;
            c.n = total;
            c.div = false;
            c.topk = false;
            const uint32_t tk = kth_key_w0(c.n, top_k, s, [&](int i) { return fkey(s.cv[i]); });
            c.n = filter_w0(c.n, s, [&](float v) { return fkey(v) >= tk; });
            return;
        }
    }
    const float thr = funkey(kth_key_blk(c.n, top_k, s, vkey));
    if (M == 0) {
        for (int i = tid; i < c.n; i += kST)
            if (s.region[i] < thr) s.region[i] = -INFINITY;
        __syncthreads();
    } else {
        c.topk = true;
        c.kthr = thr;
    }
}

// Softmax, top-p, min-p and the draw (sampler.go:117-206) over a working
// set in mode M.
template <int M>
__device__ __forceinline__ int sample_finish(Src &c, float top_p, float min_p, float r, SampLds &s) {
    const int tid = threadIdx.x;
    // Softmax with fastexp32 (sampler.go:117-138).
    float mx = -INFINITY;
#pragma unroll 8
    for (int i = tid; i < c.n; i += kST) mx = fmaxf(mx, wval<M>(c, s, i));
    c.m = blk_max(mx, s);
    float sm = 0.f;
#pragma unroll 8
    for (int i = tid; i < c.n; i += kST) {
        const float x = wval<M>(c, s, i);
        sm += (x == -INFINITY) ? 0.f : fastexp32_dev(__fsub_rn(x, c.m));
    }
    const float S1 = blk_sum(sm, s);
    c.n1 = S1 > 0.f;
    c.i1 = c.n1 ? __fdiv_rn(1.f, S1) : 1.f;
    if constexpr (M != 2) {  // values -> stage-1 probabilities, in place
        float *lw = M == 0 ? s.region : s.cv;
#pragma unroll 8
        for (int i = tid; i < c.n; i += kST) {
            const float x = lw[i];
            const float p = (x == -INFINITY) ? 0.f : fastexp32_dev(__fsub_rn(x, c.m));
            lw[i] = c.n1 ? __fmul_rn(p, c.i1) : p;
        }
        __syncthreads();
    }
    // Top-p (sampler.go:141-165): the cutoff is the item where the
    // descending cumulative probability first reaches p, i.e. the largest
    // key tau whose tail sum sum(p : key(p) >= tau) still reaches p.
    if (top_p > 0.f && top_p < 1.f) {
        uint32_t res;
        if constexpr (M == 1) {  // short list: wave 0, probabilities in registers
            constexpr int R = kCandCap / 64;
            const int lane = tid & 63;
            if (tid < 64) {
                with_groups<R>(c.n, [&](auto gc) {
                    constexpr int G = decltype(gc)::value;
                    float pv[G];
#pragma unroll
                    for (int j = 0; j < G; j++) pv[j] = (lane + 64 * j < c.n) ? s.cv[lane + 64 * j] : 0.f;
                    auto tail = [&](uint32_t t) {
                        float a = 0.f;
#pragma unroll
                        for (int j = 0; j < G; j++) a += (fkey(pv[j]) >= t) ? pv[j] : 0.f;
                        return wave_sum_dpp(a);
                    };
                    uint32_t rr = 0x80000000u;  // key of +0: the whole set
                    if (tail(rr) >= top_p) {
                        for (int bit = 30; bit >= 0; bit--) {
                            const uint32_t cand = rr | (1u << bit);
                            if (tail(cand) >= top_p) rr = cand;
                        }
                    } else {
                        rr = 0;  // never reached: keep everything
                    }
                    if (lane == 0) s.sel_i[0] = (int)rr;
                });
            }
            __syncthreads();
            res = (uint32_t)s.sel_i[0];
            __syncthreads();
        } else {
            auto tail = [&](uint32_t t) {
                float a = 0.f;
#pragma unroll 8
                for (int i = tid; i < c.n; i += kST) {
                    const float p = wp1<M>(c, s, i);
                    a += (fkey(p) >= t) ? p : 0.f;
                }
                return blk_sum(a, s);
            };
            res = 0x80000000u;
            if (tail(res) >= top_p) {
                for (int bit = 30; bit >= 0; bit--) {
                    const uint32_t cand = res | (1u << bit);
                    if (tail(cand) >= top_p) res = cand;
                }
            } else {
                res = 0;
            }
        }
        c.tau = res;
        c.topp = true;
        c.n2 = false;
        float k2 = 0.f;
#pragma unroll 8
        for (int i = tid; i < c.n; i += kST) k2 += wprob<M>(c, s, i, 2);
        const float S2 = blk_sum(k2, s);
        c.n2 = S2 > 0.f;
        c.i2 = c.n2 ? __fdiv_rn(1.f, S2) : 1.f;
    }
    // Min-p (sampler.go:168-191).
    if (min_p > 0.f) {
        float mp = 0.f;
#pragma unroll 8
        for (int i = tid; i < c.n; i += kST) mp = fmaxf(mp, wprob<M>(c, s, i, 2));
        mp = blk_max(mp, s);
        c.thr3 = __fmul_rn(mp, min_p);
        c.minp = true;
        c.n3 = false;
        float k3 = 0.f;
#pragma unroll 8
        for (int i = tid; i < c.n; i += kST) k3 += wprob<M>(c, s, i, 3);
        const float S3 = blk_sum(k3, s);
        c.n3 = S3 > 0.f;
        c.i3 = c.n3 ? __fdiv_rn(1.f, S3) : 1.f;
    }
    // Categorical draw (sampler.go:194-206), vocab - 1 if r is never reached.
    return samp_draw(
        c.n, r, c.V - 1, s, [&](int i) { return wprob<M>(c, s, i, 3); }, [&](int i) { return widx<M>(s, i); });
}

__device__ __forceinline__ int sample_set(Src &c, int top_k, float top_p, float min_p, float r, SampLds &s) {
    if (top_k > 0 && top_k < c.n) {
        if (c.mode == 0)
            topk_select<0>(c, top_k, s);
        else
            topk_select<2>(c, top_k, s);
    }
    if (c.mode == 0) return sample_finish<0>(c, top_p, min_p, r, s);
    if (c.mode == 1) return sample_finish<1>(c, top_p, min_p, r, s);
    return sample_finish<2>(c, top_p, min_p, r, s);
}

// Penalties of a window token seen f times (sampler.go:213-262): repeat
// (divide a positive logit, multiply a negative one), frequency, presence.
__device__ __forceinline__ float pen_value(float x, int f, float rp, float fp, float pp) {
    if (rp != 1.f && rp != 0.f) x = (x > 0.f) ? __fdiv_rn(x, rp) : __fmul_rn(x, rp);
    if (fp != 0.f) x = __fsub_rn(x, __fmul_rn(fp, (float)f));
    if (pp != 0.f) x = __fsub_rn(x, pp);
    return x;
}

// Bring a row into the working set: LDS values (penalties applied in place,
// then divided by the temperature) when it fits, else memory reads with the
// penalised tokens in an LDS bitmap and list.  seen(i) / freq(i): the row's
// distinct window tokens (ascending) and counts; ns of them.
template <class SeenF, class FreqF>
__device__ __forceinline__ void load_row(Src &c, SampLds &s, const float *row, int V, float temperature,
                         SeenF seen, FreqF freq, int ns, float rp, float fp, float pp) {
    const int tid = threadIdx.x;
    c.row = row;
    c.V = V;
    c.n = V;
    c.nseen = 0;
    float t = temperature;
    if (t <= 0.f) t = 1e-5f;
    c.temp = t;
    c.div = (t != 1.f);
    c.topk = c.topp = c.minp = false;
    c.n1 = c.n2 = c.n3 = false;
    auto pen = [&](float x, int f) { return pen_value(x, f, rp, fp, pp); };
    if (V <= kRowCap) {
        // scratch value = pen(x) / temperature (sampler.go:80-97), the
        // division applied as the row is stored; the penalised entries are
        // then rewritten from their logits
        c.mode = 0;
        const bool div = c.div;
        auto dv = [&](float x) { return div ? __fdiv_rn(x, t) : x; };
        if ((((uintptr_t)row) & 15) == 0 && (V & 3) == 0) {
            const float4 *r4 = (const float4 *)row;
#pragma unroll 8
            for (int v = tid; v < V / 4; v += kST) {
                const float4 x = r4[v];
                ((float4 *)s.region)[v] = make_float4(dv(x.x), dv(x.y), dv(x.z), dv(x.w));
            }
        } else {
#pragma unroll 8
            for (int v = tid; v < V; v += kST) s.region[v] = dv(row[v]);
        }
        __syncthreads();
        if (ns > 0) {
            for (int i = tid; i < ns; i += kST) {
                const int k = seen(i);
                s.region[k] = dv(pen(row[k], freq(i)));
            }
            __syncthreads();
        }
        c.div = false;
        return;
    }
    c.mode = 2;
    if (ns > 0) {
        uint32_t *bits = (uint32_t *)s.region;
        int *stok = (int *)(s.region + kSeenOff);
        float *sv = s.region + kSeenOff + kSampMaxSeen;
        for (int i = tid; i < (V + 31) >> 5; i += kST) bits[i] = 0u;
        __syncthreads();
        for (int i = tid; i < ns; i += kST) {
            const int t = seen(i);
            stok[i] = t;
            sv[i] = pen(row[t], freq(i));
            atomicOr(&bits[t >> 5], 1u << (t & 31));
        }
        __syncthreads();
        c.nseen = ns;
    }
}

// top_k / top_p clamped as sampler.go:100-106, 141-144.
__device__ __forceinline__ int clamp_topk(int k, int V) { return (k < 0 || k >= V) ? 0 : k; }
__device__ __forceinline__ float clamp_topp(float p) { return (p <= 0.f || p > 1.f) ? 1.f : p; }

// Row b's repetition window counted in LDS (sampler.go:213-262 counts each
// window token's occurrences; ids outside [0, V) are skipped): the window's
// ids are set in a bitmap over the vocabulary, an exclusive scan of the
// bitmap words' popcounts ranks the distinct ids in ascending order, and
// every window entry adds one to its id's rank.  Leaves s.win[r] = id |
// count << 18 for ranks r < the returned number of distinct ids; the window
// holds at most kSampMaxSeen entries (the host checks the bound).
__device__ __forceinline__ int count_window(const SampleArgs &a, int b, SampLds &s) {
    constexpr int WPT = kSampMaxVocab / 32 / kST;  // bitmap words per thread
    const int tid = threadIdx.x;
    const int V = a.V;
    const int n = (int)max((int64_t)0, min((int64_t)a.hist_len[b], a.hist_stride));
    const int lo = (a.window > 0 && n > a.window) ? n - a.window : 0;
    const int w = n - lo;
    const int32_t *h = a.hist + (int64_t)b * a.hist_stride + lo;
    const int nw = (V + 31) >> 5;
    uint32_t *bits = (uint32_t *)s.region;                  // [kSampMaxVocab / 32]
    int *wpre = (int *)(s.region + kSampMaxVocab / 32);     // rank of each word's first id
    int *ids = (int *)(s.region + kSampMaxVocab / 16);      // window ids (-1: skipped)
    int *cnt = ids + kSampMaxSeen;                          // count per rank
    static_assert(kSampMaxVocab / 16 + 2 * kSampMaxSeen <= kRowCap, "window scratch fits the region");
    for (int i = tid; i < nw; i += kST) bits[i] = 0u;
    __syncthreads();
    for (int i = tid; i < w; i += kST) {
        const int t = h[i];
        const bool ok = t >= 0 && t < V;
        ids[i] = ok ? t : -1;
        if (ok) atomicOr(&bits[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    const int w0 = tid * WPT;
    int local = 0;
#pragma unroll
    for (int j = 0; j < WPT; j++)
        if (w0 + j < nw) local += __popc(bits[w0 + j]);
    int nd;
    int base = blk_iscan_excl(local, s, &nd);
#pragma unroll
    for (int j = 0; j < WPT; j++)
        if (w0 + j < nw) {
            wpre[w0 + j] = base;
            base += __popc(bits[w0 + j]);
        }
    for (int i = tid; i < nd; i += kST) cnt[i] = 0;
    __syncthreads();
    for (int i = tid; i < w; i += kST) {
        const int t = ids[i];
        if (t >= 0) atomicAdd(&cnt[wpre[t >> 5] + __popc(bits[t >> 5] & ((1u << (t & 31)) - 1u))], 1);
    }
    __syncthreads();
    for (int j = 0; j < WPT; j++) {
        if (w0 + j >= nw) break;
        uint32_t m = bits[w0 + j];
        int r = wpre[w0 + j];
        while (m) {
            const int k = __builtin_ctz(m);
            m &= m - 1u;
            s.win[r] = (uint32_t)((w0 + j) * 32 + k) | ((uint32_t)cnt[r] << 18);
            r++;
        }
    }
    __syncthreads();
    return nd;
}

// ---- the vocabulary split ----------------------------------------------------
// One work-group per row leaves most of the chip idle for a decode batch, so
// rows are cut into vocabulary chunks of at most kPartChunk entries, one
// work-group each.  For top-k sampling a chunk keeps its own candidates: the
// entries at or above its k-th largest value.  The row's k-th largest is at
// least any chunk's (that chunk holds k entries at or above its own), so
// every entry the row keeps is among them, and the k-th largest of the
// merged lists is the row's.  The row's work-group merges the lists in
// chunk order, which is index order, and continues at Sample's
// candidate-list stage (the exact k-th largest, softmax, top-p, min-p, the
// draw), as a whole-row work-group does after its own compaction.  A chunk
// list past its slots (ties) or a merge past kCandCap sends the row down the
// whole-row path instead.
constexpr int kPartChunk = 8192;  // entries of a top-k chunk
constexpr int kPartMaxK = 256;    // largest top-k the split serves
constexpr int kRegRow = 16;       // float4 rounds a thread holds: rows of up to 32768 entries

struct PartLds {
    float red[2][kSW];
    int cnt[kST];
    uint32_t key[kST];
    int sel_i[2];
    float sel_f;
    int best;
    union {
        struct {
            float cv[kCandCap];
            int ci[kCandCap];
        };
        // one 16-bit slot per chunk entry until the penalties are applied:
        // its window count, or its position + 1 in a host-counted list
        uint32_t pcw[kPartChunk / 2];
    };
};
static_assert(kPartChunk / 2 <= 2 * kCandCap, "window slots alias the candidate arrays");
static_assert(kSampMaxSeen < (1 << 16), "a window count or list position fits 16 bits");
static_assert(kRegRow * kSW <= 128, "reg_topk scans the tile totals 2 per lane of a wave");

struct RedLds {
    float red[2][kSW];
};

// ---- rows held in registers ---------------------------------------------------
// Entry e of a segment [0, n) sits in thread (e / 4) % kST, float4 round
// e / (4 kST), component e % 4 (x[4 round + component]): the loads
// coalesce, and (round, thread, component) is index order.  Entries past n
// read as -inf.
template <int R>
__device__ __forceinline__ void reg_load(const float *src, int n, float (&x)[4 * R]) {
    const int tid = threadIdx.x;
    const bool vec = (((uintptr_t)src) & 15) == 0;
#pragma unroll
    for (int j = 0; j < R; j++) {
        const int e = 4 * (tid + kST * j);
        if (vec && e + 3 < n) {
            const float4 v = *(const float4 *)(src + e);
            x[4 * j] = v.x;
            x[4 * j + 1] = v.y;
            x[4 * j + 2] = v.z;
            x[4 * j + 3] = v.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) x[4 * j + q] = (e + q < n) ? src[e + q] : -INFINITY;
        }
    }
}
__device__ __forceinline__ int reg_idx(int j, int q) { return 4 * ((int)threadIdx.x + kST * j) + q; }

// Calls f(std::integral_constant<int, R>) with the fewest float4 rounds R
// (2, 4, 8 or 16) that hold n <= 4 kST kRegRow entries.
template <class F>
__device__ __forceinline__ void with_rounds(int n, F f) {
    if (n <= 8 * kST) f(std::integral_constant<int, 2>{});
    else if (n <= 16 * kST) f(std::integral_constant<int, 4>{});
    else if (n <= 32 * kST) f(std::integral_constant<int, 8>{});
    else f(std::integral_constant<int, kRegRow>{});
}

// A row's window tokens for the penalties (sampler.go:213-262), loaded with
// the chunk's logits: rlx_sample_async's device history (the last `window`
// ids of the row's history; the caller bounds it by kSampMaxSeen) or
// rlx_sample's host-counted distinct tokens.  ids[r] is entry tid + kST r,
// -1 past the end.
struct WinIds {
    int ids[kSampMaxSeen / kST];
    int n0;  // host lists: the row's first list position
};
__device__ __forceinline__ void win_load(const SampleArgs &a, int b, WinIds &w) {
    const int tid = threadIdx.x;
    int nw = 0;
    const int32_t *h = nullptr;
    w.n0 = 0;
    if (a.hist && a.hist_stride <= kSampMaxSeen) {
        // a short history row is read whole, with its length, then cut to
        // the window
        const int32_t *row = a.hist + (int64_t)b * a.hist_stride;
        const int S = (int)a.hist_stride;
#pragma unroll
        for (int r = 0; r < kSampMaxSeen / kST; r++) {
            const int i = tid + kST * r;
            w.ids[r] = i < S ? row[i] : -1;
        }
        const int hn = (int)max((int64_t)0, min((int64_t)a.hist_len[b], a.hist_stride));
        const int h0 = (a.window > 0 && hn > a.window) ? hn - a.window : 0;
#pragma unroll
        for (int r = 0; r < kSampMaxSeen / kST; r++) {
            const int i = tid + kST * r;
            if (i < h0 || i >= hn) w.ids[r] = -1;
        }
        return;
    }
    if (a.hist) {
        const int hn = (int)max((int64_t)0, min((int64_t)a.hist_len[b], a.hist_stride));
        const int h0 = (a.window > 0 && hn > a.window) ? hn - a.window : 0;
        nw = hn - h0;
        h = a.hist + (int64_t)b * a.hist_stride + h0;
    } else if (a.seen_off) {
        w.n0 = a.seen_off[b];
        nw = a.seen_off[b + 1] - w.n0;
        h = a.seen_tok + w.n0;
    }
#pragma unroll
    for (int r = 0; r < kSampMaxSeen / kST; r++) {
        const int i = tid + kST * r;
        w.ids[r] = i < nw ? h[i] : -1;
    }
}

// The penalties applied to the chunk's raw logits in registers: each window
// token in [lo, lo + n) marks its entry's 16-bit LDS slot -- with its
// occurrence count (device history; ids outside [0, V) fall in no chunk) or
// its list position + 1 (host lists, whose counts are read back).
template <int R>
__device__ __forceinline__ void reg_penalties(const SampleArgs &a, const WinIds &w, int lo, int n,
                                              float (&x)[4 * R], uint32_t *slots) {
    const int tid = threadIdx.x;
    for (int i = tid; i < (n + 1) >> 1; i += kST) slots[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kSampMaxSeen / kST; r++) {
        const int id = w.ids[r];
        if (id >= lo && id < lo + n) {
            const uint32_t sh = 16 * ((id - lo) & 1);
            if (a.hist)
                atomicAdd(&slots[(id - lo) >> 1], 1u << sh);
            else
                atomicOr(&slots[(id - lo) >> 1], (uint32_t)(tid + kST * r + 1) << sh);
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < R; j++) {
        const int e = reg_idx(j, 0);
        if (e >= n) continue;
        const uint2 v = *(const uint2 *)&slots[e >> 1];  // the round's 4 slots
        const uint32_t sl[4] = {v.x & 0xFFFFu, v.x >> 16, v.y & 0xFFFFu, v.y >> 16};
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (sl[q] != 0u && e + q < n) {
                const int f = a.hist ? (int)sl[q] : a.seen_freq[w.n0 + (int)sl[q] - 1];
                x[4 * j + q] = pen_value(x[4 * j + q], f, a.rp, a.fp, a.pp);
            }
    }
    __syncthreads();  // the slots alias the candidate list or the row region
}

// Chunks select on the logits before their division by the temperature t
// (> 0): fl(x / t) does not decrease as x grows, so the order is the same,
// and only the candidates are divided.  Entries whose quotient rounds to a
// bound's quotient lie within a few floats of the bound (in the normal
// range dividing scales the float spacing by 1/t up to a factor 2 either
// way, so at most about 6 consecutive floats share a quotient): selecting
// 16 keys below the raw bound keeps every entry whose quotient reaches the
// bound's.  Near zero, overflow or underflow every entry is kept instead.
__device__ __forceinline__ uint32_t div_margin(uint32_t lb, float t) {
    if (t == 1.f || lb == 0u) return 0u;
    const float f = fabsf(funkey(lb)), q = fabsf(__fdiv_rn(funkey(lb), t));
    if (!(f >= 0x1p-60f && f <= 0x1p100f && q >= 0x1p-100f && q <= 0x1p100f)) return lb;
    return 16u;
}
// The key of fl(funkey(k) / t) (k = 0, no bound, stays 0).
__device__ __forceinline__ uint32_t div_key(uint32_t k, float t) {
    return (t == 1.f || k == 0u) ? k : fkey(__fdiv_rn(funkey(k), t));
}

// Candidates from n register-held values (0 < k): the entries at or above a
// lower bound of their k-th largest, placed in index order.
//   reg_bound: lb = each wave's ceil(k / kSW)-th largest lane maximum, to 16
//     key bits, the smallest over the waves (every wave holds that many
//     entries at or above it: kSW ceil(k / kSW) >= k in all); ub = the
//     largest key; the entries kept (at or above lb, less div_margin for
//     the division by t still to come); their lane offsets within their
//     (round, wave) tile and, in s.cnt, the tiles' first slots (an ordered
//     scan); returns their count (every thread).
//   reg_place: the kept entries written to dv / di (indices + ioff).
template <int R, class L>
__device__ __forceinline__ int reg_bound(const float (&x)[4 * R], int n, int k, float t, L &s, uint32_t (&keep)[R],
                                         int (&off)[R], uint32_t &lb, uint32_t &ub) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t mk = 0;
#pragma unroll
    for (int j = 0; j < 4 * R; j++)
        if (reg_idx(j >> 2, j & 3) < n) mk = max(mk, fkey(x[j]));
    const int kw = (k + kSW - 1) / kSW;
    uint32_t lbw = 0;
    for (int bit = 31; bit >= 16; bit--) {
        const uint32_t cand = lbw | (1u << bit);
        if ((int)__popcll(__ballot(mk >= cand)) >= kw) lbw = cand;
    }
    const uint32_t ubw = wave_max_u32(mk);
    if (lane == 0) {
        s.key[wave] = lbw;
        s.key[kSW + wave] = ubw;
    }
    __syncthreads();
    lb = s.key[0];
    ub = s.key[kSW];
#pragma unroll
    for (int w = 1; w < kSW; w++) {
        lb = min(lb, s.key[w]);
        ub = max(ub, s.key[kSW + w]);
    }
    const uint32_t th = lb - div_margin(lb, t);
#pragma unroll
    for (int j = 0; j < R; j++) {
        keep[j] = 0u;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (reg_idx(j, q) < n && fkey(x[4 * j + q]) >= th) keep[j] |= 1u << q;
        const int c = __popc(keep[j]);
        const int inc = wave_iscan_dpp(c);
        off[j] = inc - c;
        if (lane == 63) s.cnt[j * kSW + wave] = inc;
    }
    __syncthreads();
    if (tid < 64) {  // ordered exclusive scan of the R kSW tile totals, 2 per lane
        const int t0 = 2 * lane, t1 = 2 * lane + 1;
        const int c0 = t0 < R * kSW ? s.cnt[t0] : 0, c1 = t1 < R * kSW ? s.cnt[t1] : 0;
        const int inc = wave_iscan_dpp(c0 + c1);
        if (t0 < R * kSW) s.cnt[t0] = inc - c0 - c1;
        if (t1 < R * kSW) s.cnt[t1] = inc - c1;
        if (lane == 63) s.sel_i[0] = inc;
    }
    __syncthreads();
    return s.sel_i[0];
}
template <int R>
__device__ __forceinline__ void reg_place(const float (&x)[4 * R], const uint32_t (&keep)[R], const int (&off)[R],
                                          const int *base, float *dv, int32_t *di, int ioff) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < R; j++) {
        int o = base[j * kSW + wave] + off[j];
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (keep[j] & (1u << q)) {
                dv[o] = x[4 * j + q];
                di[o] = ioff + reg_idx(j, q);
                o++;
            }
    }
}

// A chunk's top-k candidates (logits not yet divided by t) written out in
// index order (indices offset by lo) with the chunk record on = {count,
// lower bound key, largest key} (count -1: overflow; keys of the divided
// values): the reg_bound entries straight from registers when they fit the
// cap slots; otherwise compacted in LDS, cut to the exact k-th largest
// (wave 0, one key bit per step; it becomes the lower bound) and written
// from there.
template <int R>
__device__ __forceinline__ void reg_topk(const float (&x)[4 * R], int n, int k, float t, int lo, int cap,
                                         PartLds &s, float *ov, int32_t *oi, int32_t *on) {
    const int tid = threadIdx.x;
    uint32_t keep[R], lb, ub;
    int off[R];
    const int total = reg_bound<R>(x, n, k, t, s, keep, off, lb, ub);
    if (total <= cap) {
        reg_place<R>(x, keep, off, s.cnt, ov, oi, lo);
        if (tid == 0) *(int4 *)on = make_int4(total, (int)div_key(lb, t), (int)div_key(ub, t), 0);
        return;
    }
    int m = -1;
    uint32_t tk = 0;
    if (total <= kCandCap) {
        reg_place<R>(x, keep, off, s.cnt, s.cv, s.ci, 0);
        __syncthreads();
        tk = kth_key_w0(total, k, s, [&](int i) { return fkey(s.cv[i]); });
        const uint32_t th = tk - div_margin(tk, t);
        m = filter_w0(total, s, [&](float v) { return fkey(v) >= th; });
        if (m > cap) m = -1;
        for (int j = tid; j < m; j += kST) {
            ov[j] = s.cv[j];
            oi[j] = lo + s.ci[j];
        }
    }
    if (tid == 0) *(int4 *)on = make_int4(m, (int)div_key(tk, t), (int)div_key(ub, t), 0);
}

// k-th largest of n keys (0 when n < k), given that it lies in [lo, hi]
// and no key exceeds hi: the bits above the highest one in which lo and hi
// differ are known; the rest is found 8 bits per step (the first step
// takes the odd bits), by an LDS histogram of the next digit over the keys
// matching the digits so far, then wave 0 finds the digit from the top
// (lane l holds digits 255 - 4l down to 252 - 4l; an ordered scan of the
// lanes' totals).  Keys below lo that match the known bits only add to the
// counts below the answer.
template <class L, class K>
__device__ uint32_t kth_key_radix(int n, int k, uint32_t lo, uint32_t hi, L &s, K key) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (n < k) return 0u;
    if (lo >= hi) return hi;
    const int top = 31 - __builtin_clz(lo ^ hi);  // highest differing bit
    const int steps = (top + 8) / 8;
    const uint32_t known = top == 31 ? 0u : (0xFFFFFFFFu << (top + 1));
    uint32_t prefix = lo & known;
    int kk = k;
    for (int st = 0; st < steps; st++) {
        const int shift = 8 * (steps - 1 - st);
        const uint32_t fixed = st == 0 ? known : (0xFFFFFFFFu << (shift + 8));
        if (tid < 256) s.cnt[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kST) {
            const uint32_t kv = key(i);
            if ((kv & fixed) == prefix) atomicAdd(&s.cnt[(kv >> shift) & 255u], 1);
        }
        __syncthreads();
        if (tid < 64) {
            int h[4];
#pragma unroll
            for (int q = 0; q < 4; q++) h[q] = s.cnt[255 - 4 * lane - q];
            const int loc = h[0] + h[1] + h[2] + h[3];
            const int inc = wave_iscan_dpp(loc);
            const uint64_t hit = __ballot(inc >= kk);  // the last lane's total is >= kk
            if (lane == (int)__builtin_ctzll(hit)) {
                int before = inc - loc, d = 255 - 4 * lane;
                bool found = false;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (!found) {
                        if (before + h[q] >= kk) {
                            found = true;
                            d = 255 - 4 * lane - q;
                        } else {
                            before += h[q];
                        }
                    }
                s.sel_i[0] = d;
                s.sel_i[1] = kk - before;
            }
        }
        __syncthreads();
        prefix |= (uint32_t)s.sel_i[0] << shift;
        kk = s.sel_i[1];
    }
    __syncthreads();
    return prefix;
}

// Keep the candidate-list entries with keep(v), in order, in place: each
// thread reads its contiguous run (at most 4 entries: n <= kCandCap), an
// ordered scan gives its first slot, the writes follow every read.
template <class P>
__device__ __forceinline__ int filter_blk(int n, SampLds &s, P keep) {
    static_assert(kCandCap <= 4 * kST, "at most 4 entries per thread");
    const int C = (n + kST - 1) / kST;
    const int i0 = min(n, (int)threadIdx.x * C);
    float v[4];
    int ix[4];
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (q < C && i0 + q < n) {
            v[q] = s.cv[i0 + q];
            ix[q] = s.ci[i0 + q];
            if (keep(v[q])) m |= 1u << q;
        }
    int total;
    int o = blk_iscan_excl(__popc(m), s, &total);  // (its barriers follow every read)
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (m & (1u << q)) {
            s.cv[o] = v[q];
            s.ci[o] = ix[q];
            o++;
        }
    __syncthreads();
    return total;
}


// Softmax, top-p, min-p and the draw (sampler.go:117-206) over a candidate
// list of n <= 64 entries, one per lane of wave 0 (lane order = list order
// = index order), with wave-level sums: the arithmetic of sample_finish.
// The top-p cutoff is the largest key whose tail sum reaches p; every
// entry's tail is summed by the 8 waves at once, over 8 entries each, then
// the 8 partials in order.
__device__ __forceinline__ int finish_list64(int n, int V, float top_p, float min_p, float r, SampLds &s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool in = lane < n;
    float p = 0.f;
    uint32_t kp = 0u;
    if (tid < 64) {
        const float x = in ? s.cv[lane] : -INFINITY;
        const float m = wave_max_dpp(x);
        p = (x == -INFINITY) ? 0.f : fastexp32_dev(__fsub_rn(x, m));
        const float S1 = wave_sum_dpp(p);
        if (S1 > 0.f) p = __fmul_rn(p, __fdiv_rn(1.f, S1));
        kp = fkey(p);
    }
    if (top_p > 0.f && top_p < 1.f) {
        if (tid < 64) {
            s.cv[lane] = p;  // the values are no longer needed
            s.key[lane] = kp;
        }
        __syncthreads();
        const uint32_t kj = s.key[lane];
        float part = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int i = 8 * wave + q;
            if (i < n && s.key[i] >= kj) part += s.cv[i];
        }
        s.cnt[tid] = __float_as_int(part);
        __syncthreads();
        if (tid < 64) {
            float T = 0.f;
#pragma unroll
            for (int w = 0; w < kSW; w++) T += __int_as_float(s.cnt[64 * w + lane]);
            const uint32_t tau = wave_max_u32((in && T >= top_p) ? kp : 0u);  // 0: keep all
            p = (kp >= tau) ? p : 0.f;
            const float S2 = wave_sum_dpp(p);
            if (S2 > 0.f) p = __fmul_rn(p, __fdiv_rn(1.f, S2));
        }
    }
    if (tid < 64) {
        if (min_p > 0.f) {
            const float thr = __fmul_rn(wave_max_dpp(p), min_p);
            p = (p < thr) ? 0.f : p;
            const float S3 = wave_sum_dpp(p);
            if (S3 > 0.f) p = __fmul_rn(p, __fdiv_rn(1.f, S3));
        }
        const float cum = wave_scan_dpp(p);
        const uint64_t hit = __ballot(in && r < cum);
        if (lane == 0) s.sel_i[0] = hit ? s.ci[__builtin_ctzll(hit)] : V - 1;
    }
    __syncthreads();
    const int res = s.sel_i[0];
    __syncthreads();
    return res;
}

// Row b's chunk lists merged, in chunk order, into the working set's
// candidate list (mode 1), each value divided by the temperature t here
// (sampler.go:94-97): every thread loads its slots while wave 0 scans the
// chunk records {count, lower bound key, largest key}; lb / ub: the largest
// lower bound and the largest key (the row's k-th largest lies between
// them); false, for the whole work-group, when a chunk overflowed or the
// lists pass kCandCap.
__device__ __forceinline__ bool part_merge(const float *pv, const int32_t *pi, const int32_t *pn, int nch,
                                           int cap, int V, float t, Src &c, uint32_t &lb, uint32_t &ub,
                                           SampLds &s) {
    constexpr int kSlots = 8;  // nch * cap <= kSlots * kST
    const int tid = threadIdx.x;
    const int ns = nch * cap;
    float v[kSlots];
    int ix[kSlots];
#pragma unroll
    for (int r = 0; r < kSlots; r++) {
        const int j = tid + kST * r;
        if (j < ns) {
            v[r] = pv[j];
            ix[r] = pi[j];
        }
    }
    if (tid < 64) {  // nch <= 64
        const int4 r = tid < nch ? ((const int4 *)pn)[tid] : make_int4(0, 0, 0, 0);
        const bool bad = __ballot(r.x < 0) != 0;
        const int m0 = max(r.x, 0);
        const int inc = wave_iscan_dpp(m0);
        s.key[tid] = (uint32_t)(inc - m0);
        s.cnt[tid] = m0;
        const uint32_t l = wave_max_u32((uint32_t)r.y), u = wave_max_u32((uint32_t)r.z);
        if (tid == 63) {
            s.sel_i[0] = bad ? -1 : inc;
            s.key[64] = l;
            s.key[65] = u;
        }
    }
    __syncthreads();
    const int total = s.sel_i[0];
    lb = s.key[64];
    ub = s.key[65];
    if (total < 0 || total > kCandCap) {
        __syncthreads();
        return false;
    }
#pragma unroll
    for (int r = 0; r < kSlots; r++) {
        const int j = tid + kST * r;
        if (j < ns) {
            const int ch = j / cap, e = j - ch * cap;
            if (e < s.cnt[ch]) {
                s.cv[(int)s.key[ch] + e] = t == 1.f ? v[r] : __fdiv_rn(v[r], t);
                s.ci[(int)s.key[ch] + e] = ix[r];
            }
        }
    }
    __syncthreads();
    c.mode = 1;
    c.n = total;
    c.row = nullptr;
    c.V = V;
    c.nseen = 0;
    c.temp = 1.f;
    c.div = false;
    c.topk = c.topp = c.minp = false;
    c.n1 = c.n2 = c.n3 = false;
    return true;
}

// Top-k completed on the merged list (the row's exact k-th largest, then
// the entries at or above it), then Sample's remaining stages.
__device__ __forceinline__ int part_finish(Src &c, uint32_t lb, uint32_t ub, int top_k, float top_p, float min_p,
                                           float r, SampLds &s) {
    const uint32_t tk = kth_key_radix(c.n, top_k, lb, ub, s, [&](int i) { return fkey(s.cv[i]); });
    c.n = filter_blk(c.n, s, [&](float v) { return fkey(v) >= tk; });
    if (c.n <= 64) return finish_list64(c.n, c.V, top_p, min_p, r, s);
    return sample_finish<1>(c, top_p, min_p, r, s);
}

// One chunk [lo, lo + n) of a row: its logits (with the penalties of
// Sample's arguments a when PEN), its candidates written out; the merge
// divides them by the temperature t.
template <int R, bool PEN, class A>
__device__ __forceinline__ void part_chunk(const A &a, const float *row, int lo, int n, float t, int k, int cap,
                                           PartLds &s, float *ov, int32_t *oi, int32_t *on) {
    float x[4 * R];
    reg_load<R>(row + lo, n, x);
    if constexpr (PEN) {
        WinIds w;
        win_load(a, blockIdx.x, w);
        reg_penalties<R>(a, w, lo, n, x, s.pcw);
    }
    reg_topk<R>(x, n, k, t, lo, cap, s, ov, oi, on);
}

// Phase one of the split Sample: chunk blockIdx.y of row blockIdx.x.
__global__ __launch_bounds__(kST) void sample_part_kernel(const SampleArgs a) {
    __shared__ PartLds s;
    const int b = blockIdx.x, ch = blockIdx.y;
    const int lo = ch * a.pch, n = min(a.V - lo, a.pch);
    float t = a.temperature;
    if (t <= 0.f) t = 1e-5f;
    const int64_t q = (int64_t)b * a.nch + ch;
    const float *row = a.logits + (int64_t)b * a.stride;
    float *ov = a.part_v + q * a.pcap;
    int32_t *oi = a.part_i + q * a.pcap;
    const int k = clamp_topk(a.top_k, a.V);
    const bool pen = a.hist || a.seen_off;
    if (n <= 8 * kST) {
        if (pen)
            part_chunk<2, true>(a, row, lo, n, t, k, a.pcap, s, ov, oi, a.part_n + 4 * q);
        else
            part_chunk<2, false>(a, row, lo, n, t, k, a.pcap, s, ov, oi, a.part_n + 4 * q);
    } else {
        if (pen)
            part_chunk<4, true>(a, row, lo, n, t, k, a.pcap, s, ov, oi, a.part_n + 4 * q);
        else
            part_chunk<4, false>(a, row, lo, n, t, k, a.pcap, s, ov, oi, a.part_n + 4 * q);
    }
}

// Sample, one work-group per row: phase two of the split path when the
// chunk lists are there, else the whole row.
__global__ __launch_bounds__(kST) void sample_kernel(const SampleArgs a) {
    __shared__ SampLds s;
    const int b = blockIdx.x;
    Src c;
    if (a.nch > 0) {
        const int64_t q = (int64_t)b * a.nch;
        uint32_t lb, ub;
        float t = a.temperature;
        if (t <= 0.f) t = 1e-5f;
        if (part_merge(a.part_v + q * a.pcap, a.part_i + q * a.pcap, a.part_n + 4 * q, a.nch, a.pcap, a.V, t, c,
                       lb, ub, s)) {
            const int t =
                part_finish(c, lb, ub, clamp_topk(a.top_k, a.V), clamp_topp(a.top_p), a.min_p, a.u[b], s);
            if (threadIdx.x == 0) a.out[b] = t;
            return;
        }
    }
    const float *row = a.logits + (int64_t)b * a.stride;
    if (a.hist) {
        const int ns = count_window(a, b, s);
        load_row(
            c, s, row, a.V, a.temperature, [&](int i) { return (int)(s.win[i] & 0x3FFFFu); },
            [&](int i) { return (int)(s.win[i] >> 18); }, ns, a.rp, a.fp, a.pp);
    } else {
        const int n0 = a.seen_off ? a.seen_off[b] : 0;
        const int ns = a.seen_off ? a.seen_off[b + 1] - n0 : 0;
        const int32_t *st = a.seen_tok + n0, *sf = a.seen_freq + n0;
        load_row(
            c, s, row, a.V, a.temperature, [&](int i) { return st[i]; }, [&](int i) { return sf[i]; }, ns,
            a.rp, a.fp, a.pp);
    }
    const int t = sample_set(c, clamp_topk(a.top_k, a.V), clamp_topp(a.top_p), a.min_p, a.u[b], s);
    if (threadIdx.x == 0) a.out[b] = t;
}

// First index of the largest value (sampler.go:56-68).
__global__ __launch_bounds__(kST) void greedy_kernel(const float *__restrict__ logits, int64_t stride,
                                                      int V, int32_t *__restrict__ out) {
    __shared__ float bv[kST];
    __shared__ int bi[kST];
    const float *row = logits + (int64_t)blockIdx.x * stride;
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int idx = INT_MAX;
    for (int v = tid; v < V; v += kST) {
        const float x = row[v];
        if (idx == INT_MAX || x > best) {
            best = x;
            idx = v;
        }
    }
    bv[tid] = best;
    bi[tid] = idx;
    __syncthreads();
    for (int o = kST / 2; o > 0; o >>= 1) {
        if (tid < o) {
            const float x = bv[tid + o];
            const int j = bi[tid + o];
            if (j != INT_MAX && (bi[tid] == INT_MAX || x > bv[tid] || (x == bv[tid] && j < bi[tid]))) {
                bv[tid] = x;
                bi[tid] = j;
            }
        }
        __syncthreads();
    }
    if (tid == 0) out[blockIdx.x] = bi[0];
}

// ---- speculative acceptance -------------------------------------------------
// acceptPhase for a batch of sequences (speculative.go:203-244): accept
// draft i while u_i < min(1, p_t/max(p_d, 1e-10)); on the first rejection
// draw the replacement from norm(max(0, p_t - p_d)) (resampleRejected
// 247-290; the target distribution if that is empty); all accepted: Sample
// the target's next row without penalties.  Three launches:
//   1. spec_stat_kernel: one work-group per (row, position, side) holds the
//      draft or target row in registers (up to 4 kST kRegRow entries, else
//      it reads the row twice) and gives softmaxAlloc's figures
//      (speculative.go:344-368: the max, the sum of fastexp32 weights
//      against it) and the draft token's probability, for every draft at
//      once; further work-groups cut the next target row into top-k chunk
//      lists (as the split Sample);
//   2. spec_mass_kernel, per (row, chunk of kStatChunk entries): the first
//      rejection from those figures (all drafts at once, by ballot), then
//      that position's chunk sums of the resample weights max(0, p_t - p_d)
//      and of p_t;
//   3. spec_final_kernel, one work-group per row: the chunk whose running
//      mass passes the draw, then the draw within it; or, all accepted, the
//      next row's Sample from the merged lists.
constexpr int kStatChunk = 8 * kST;  // entries of a resample chunk (2 float4 rounds)

struct SpecLds {
    float red[2][kSW];
    int cnt[kST];
    int sel_i[2];
};

__device__ __forceinline__ float spec_pv(float x, float m, bool norm, float inv) {
    const float e = fastexp32_dev(__fsub_rn(x, m));
    return norm ? __fmul_rn(e, inv) : e;
}

// Draft count of row b: clamped to [0, max_k] (rlx_spec_accept_async takes
// it from the device; rlx_spec_accept checks it on the host).
__device__ __forceinline__ int spec_count(const SpecArgs &a, int b) { return min(max(a.n_draft[b], 0), a.max_k); }

// The first rejected draft of row b (k: none), every thread of the
// work-group getting it: wave 0 tests 64 drafts per ballot; an id outside
// [0, V) is a rejection.
template <class L>
__device__ __forceinline__ int spec_first_reject(const SpecArgs &a, int b, int k, L &s) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        const float4 *rec = (const float4 *)a.rec + (int64_t)b * a.max_k * 2;
        const float *u = a.u + (int64_t)b * (a.max_k + 1);
        int first = k;
        for (int i0 = 0; i0 < k; i0 += 64) {
            const int i = i0 + lane;
            bool rej = false;
            if (i < k) {
                const int tok = a.d_tok[(int64_t)b * a.max_k + i];
                rej = true;
                if (tok >= 0 && tok < a.V) {
                    const float dP = rec[2 * i].z, tP = rec[2 * i + 1].z;
                    float q = __fdiv_rn(tP, dP > 1e-10f ? dP : 1e-10f);
                    if (q > 1.f) q = 1.f;
                    rej = !(u[i] < q);
                }
            }
            const uint64_t m = __ballot(rej);
            if (m) {
                first = i0 + (int)__builtin_ctzll(m);
                break;
            }
        }
        if (tid == 0) s.sel_i[0] = first;
    }
    __syncthreads();
    const int i = s.sel_i[0];
    __syncthreads();
    return i;
}

// Position i's figures: maxima, whether each sum is positive, and 1/sum.
struct SpecFig {
    float dm, tm, di, ti;
    bool dn, tn;
};
__device__ __forceinline__ SpecFig spec_fig(const SpecArgs &a, int b, int i) {
    const float4 *rec = (const float4 *)a.rec + ((int64_t)b * a.max_k + i) * 2;
    const float4 d = rec[0], t = rec[1];
    SpecFig f;
    f.dm = d.x;
    f.tm = t.x;
    f.dn = d.y > 0.f;
    f.tn = t.y > 0.f;
    f.di = f.dn ? __fdiv_rn(1.f, d.y) : 1.f;
    f.ti = f.tn ? __fdiv_rn(1.f, t.y) : 1.f;
    return f;
}
// max(0, p_t - p_d) of one entry (resampleRejected, speculative.go:256-262)
__device__ __forceinline__ float spec_resid(const SpecFig &f, float d, float t) {
    const float x = __fsub_rn(spec_pv(t, f.tm, f.tn, f.ti), spec_pv(d, f.dm, f.dn, f.di));
    return x < 0.f ? 0.f : x;
}

__global__ __launch_bounds__(kST) void spec_stat_kernel(const SpecArgs a) {
    __shared__ PartLds s;
    const int b = blockIdx.x, y = blockIdx.y;
    const int V = a.V, k = spec_count(a, b);
    if (y >= 2 * a.max_k) {  // chunk y - 2 max_k of the target's row k
        const int ch = y - 2 * a.max_k;
        const int lo = ch * a.pch, n = min(V - lo, a.pch);
        const float *row = a.t_logits + ((int64_t)b * (a.max_k + 1) + k) * V;
        float t = a.temperature;
        if (t <= 0.f) t = 1e-5f;
        const int64_t q = (int64_t)b * a.nch + ch;
        const int kk = clamp_topk(a.top_k, V);
        if (n <= 8 * kST)
            part_chunk<2, false>(a, row, lo, n, t, kk, a.pcap, s, a.part_v + q * a.pcap, a.part_i + q * a.pcap,
                                 a.part_n + 4 * q);
        else
            part_chunk<4, false>(a, row, lo, n, t, kk, a.pcap, s, a.part_v + q * a.pcap, a.part_i + q * a.pcap,
                                 a.part_n + 4 * q);
        return;
    }
    const int i = y >> 1, side = y & 1;
    if (i >= k) return;
    const float *row = side ? a.t_logits + ((int64_t)b * (a.max_k + 1) + i) * V
                            : a.d_logits + ((int64_t)b * a.max_k + i) * V;
    float m, S;
    if (V <= 4 * kST * kRegRow) {
        with_rounds(V, [&](auto rc) {
            constexpr int R = decltype(rc)::value;
            float x[4 * R];
            reg_load<R>(row, V, x);  // entries past V read as -inf
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4 * R; j++) mx = fmaxf(mx, x[j]);
            m = blk_max(mx, s);
            float sm = 0.f;
#pragma unroll
            for (int j = 0; j < 4 * R; j++)
                if (reg_idx(j >> 2, j & 3) < V) sm += fastexp32_dev(__fsub_rn(x[j], m));
            S = blk_sum(sm, s);
        });
    } else {
        float mx = -INFINITY;
#pragma unroll 8
        for (int v = threadIdx.x; v < V; v += kST) mx = fmaxf(mx, row[v]);
        m = blk_max(mx, s);
        float sm = 0.f;
#pragma unroll 8
        for (int v = threadIdx.x; v < V; v += kST) sm += fastexp32_dev(__fsub_rn(row[v], m));
        S = blk_sum(sm, s);
    }
    const int tok = a.d_tok[(int64_t)b * a.max_k + i];
    const bool norm = S > 0.f;
    const float p = (tok >= 0 && tok < V) ? spec_pv(row[tok], m, norm, norm ? __fdiv_rn(1.f, S) : 1.f) : 0.f;
    if (threadIdx.x == 0) ((float4 *)a.rec)[((int64_t)b * a.max_k + i) * 2 + side] = make_float4(m, S, p, 0.f);
}

__global__ __launch_bounds__(kST) void spec_mass_kernel(const SpecArgs a) {
    __shared__ SpecLds s;
    const int b = blockIdx.x, c = blockIdx.y;
    const int V = a.V, k = spec_count(a, b);
    const int i = spec_first_reject(a, b, k, s);
    if (i >= k) return;
    const SpecFig f = spec_fig(a, b, i);
    const int lo = c * kStatChunk, n = min(V - lo, kStatChunk);
    float xd[8], xt[8];
    reg_load<2>(a.d_logits + ((int64_t)b * a.max_k + i) * V + lo, n, xd);
    reg_load<2>(a.t_logits + ((int64_t)b * (a.max_k + 1) + i) * V + lo, n, xt);
    float sa = 0.f, st = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (reg_idx(j >> 2, j & 3) < n) {
            sa += spec_resid(f, xd[j], xt[j]);
            st += spec_pv(xt[j], f.tm, f.tn, f.ti);
        }
    blk_sum2(sa, st, s);
    if (threadIdx.x == 0) ((float2 *)a.st_mass)[(int64_t)b * a.sch + c] = make_float2(sa, st);
}

__global__ __launch_bounds__(kST) void spec_final_kernel(const SpecArgs a) {
    __shared__ SampLds s;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int V = a.V, k = spec_count(a, b);
    const float *u = a.u + (int64_t)b * (a.max_k + 1);
    const float *tl = a.t_logits + (int64_t)b * (a.max_k + 1) * V;
    const int i = spec_first_reject(a, b, k, s);
    if (i < k) {
        const SpecFig f = spec_fig(a, b, i);
        const float *dr = a.d_logits + ((int64_t)b * a.max_k + i) * V, *tr = tl + (int64_t)i * V;
        const float2 *ms = (const float2 *)a.st_mass + (int64_t)b * a.sch;
        float SA = 0.f;
        for (int c = 0; c < a.sch; c++) SA += ms[c].x;
        // norm(max(0, p_t - p_d)), or p_t when that is empty
        const bool resid = SA > 0.f;
        const float inv = resid ? __fdiv_rn(1.f, SA) : 1.f;
        const float rr = u[i + 1];
        // the chunk whose running mass passes the draw, then the draw within
        // it (on through later chunks should rounding leave it no hit)
        int c0 = 0;
        float base = 0.f;
        for (; c0 < a.sch - 1; c0++) {
            const float m = resid ? __fmul_rn(ms[c0].x, inv) : ms[c0].y;
            if (rr < base + m) break;
            base += m;
        }
        int res = -1;
        for (int c = c0; c < a.sch && res < 0; c++) {
            const int lo = c * kStatChunk, n = min(V - lo, kStatChunk);
            float xd[8], xt[8];
            reg_load<2>(dr + lo, n, xd);
            reg_load<2>(tr + lo, n, xt);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int e = reg_idx(j >> 2, j & 3);
                if (e < n)
                    s.region[e] = resid ? __fmul_rn(spec_resid(f, xd[j], xt[j]), inv)
                                        : spec_pv(xt[j], f.tm, f.tn, f.ti);
            }
            __syncthreads();
            float tot;
            const int hit = samp_draw_from(n, rr, base, s, [&](int v) { return s.region[v]; }, &tot);
            if (hit >= 0) res = lo + hit;
            base += tot;
        }
        if (tid == 0) {
            a.n_acc[b] = i;
            a.next[b] = res < 0 ? 0 : res;
        }
        return;
    }
    int t;
    Src c;
    uint32_t lb, ub;
    float tt = a.temperature;
    if (tt <= 0.f) tt = 1e-5f;
    if (a.nch > 0 &&
        part_merge(a.part_v + (int64_t)b * a.nch * a.pcap, a.part_i + (int64_t)b * a.nch * a.pcap,
                   a.part_n + (int64_t)b * a.nch * 4, a.nch, a.pcap, V, tt, c, lb, ub, s)) {
        t = part_finish(c, lb, ub, clamp_topk(a.top_k, V), clamp_topp(a.top_p), a.min_p, u[k], s);
    } else {
        load_row(
            c, s, tl + (int64_t)k * V, V, a.temperature, [](int) { return 0; }, [](int) { return 0; }, 0, 0.f,
            0.f, 0.f);
        t = sample_set(c, clamp_topk(a.top_k, V), clamp_topp(a.top_p), a.min_p, u[k], s);
    }
    if (tid == 0) {
        a.n_acc[b] = k;
        a.next[b] = t;
    }
}

hipError_t launch_sample(hipStream_t st, const SampleArgs &a, int n_rows, hipEvent_t e0,
                         hipEvent_t e1) {
    if (e0) (void)hipEventRecord(e0, st);
    if (a.nch > 0) {
        sample_part_kernel<<<dim3(n_rows, a.nch), dim3(kST), 0, st>>>(a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    sample_kernel<<<dim3(n_rows), dim3(kST), 0, st>>>(a);
    const hipError_t e = hipGetLastError();
    if (e1) (void)hipEventRecord(e1, st);
    return e;
}

hipError_t launch_greedy(hipStream_t st, const float *logits, int64_t stride, int V, int n_rows,
                         int32_t *out, hipEvent_t e0, hipEvent_t e1) {
    return launch_timed(greedy_kernel, dim3(n_rows), dim3(kST), st, e0, e1, logits, stride, V, out);
}

hipError_t launch_spec_accept(hipStream_t st, const SpecArgs &a, int n_rows, hipEvent_t e0,
                              hipEvent_t e1) {
    if (e0) (void)hipEventRecord(e0, st);
    hipError_t e = hipSuccess;
    const int ny = 2 * a.max_k + a.nch;
    if (ny > 0) {
        spec_stat_kernel<<<dim3(n_rows, ny), dim3(kST), 0, st>>>(a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (a.max_k > 0) {
        spec_mass_kernel<<<dim3(n_rows, a.sch), dim3(kST), 0, st>>>(a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    spec_final_kernel<<<dim3(n_rows), dim3(kST), 0, st>>>(a);
    e = hipGetLastError();
    if (e1) (void)hipEventRecord(e1, st);
    return e;
}

namespace {
constexpr int kGridY = 65535;  // grid y extent limit

// Top-k chunking of a vocabulary V for top-k k (clamped as Sample does):
// chunks of up to kPartChunk entries (measured faster than 4096 or 16384:
// fewer, larger chunks shorten the merge), fewer when their lists could
// pass kCandCap (or their slots the merge's 8 per thread); none (nch 0)
// when top-k is off, larger than kPartMaxK, or a single chunk would do.
void topk_split(int V, int top_k, int &nch, int &pch, int &pcap) {
    nch = pch = pcap = 0;
    const int k = (top_k < 0 || top_k >= V) ? 0 : top_k;
    if (k <= 0 || k > kPartMaxK) return;
    int n = (V + kPartChunk - 1) / kPartChunk;
    if (n * k > kCandCap) n = kCandCap / k;
    if (n < 2) return;
    const int len = ((V + n - 1) / n + 3) & ~3;
    const int nc = (V + len - 1) / len;
    if (len > kPartChunk || nc > 64 || nc < 2) return;
    // slots for a chunk's lower-bound list (about 2k entries on typical
    // rows), within the merge's 8 slots per thread
    const int cap = min(min(kCandCap, max(128, 4 * k)), 8 * kST / nc);
    if (cap < k) return;
    nch = nc;
    pch = len;
    pcap = cap;
}

int64_t carve(int64_t &off, int64_t bytes) {
    const int64_t at = off;
    off += (bytes + 255) & ~(int64_t)255;
    return at;
}
}  // namespace

int64_t plan_sample_split(SampleArgs &a, int n_rows, char *base) {
    topk_split(a.V, a.top_k, a.nch, a.pch, a.pcap);
    a.part_v = nullptr;
    a.part_i = a.part_n = nullptr;
    if (a.nch == 0) return 0;
    int64_t off = 0;
    const int64_t slots = (int64_t)n_rows * a.nch * a.pcap;
    const int64_t o_n = carve(off, (int64_t)n_rows * a.nch * 16);
    const int64_t o_v = carve(off, slots * 4);
    const int64_t o_i = carve(off, slots * 4);
    if (base) {
        a.part_n = (int32_t *)(base + o_n);
        a.part_v = (float *)(base + o_v);
        a.part_i = (int32_t *)(base + o_i);
    }
    return off;
}

int64_t plan_spec_split(SpecArgs &a, int n_rows, char *base) {
    topk_split(a.V, a.top_k, a.nch, a.pch, a.pcap);
    a.sch = (a.V + kStatChunk - 1) / kStatChunk;
    if ((int64_t)2 * a.max_k + a.nch > kGridY || a.sch > kGridY) return -1;
    a.rec = a.st_mass = a.part_v = nullptr;
    a.part_i = a.part_n = nullptr;
    int64_t off = 0;
    const int64_t o_r = carve(off, (int64_t)n_rows * a.max_k * 2 * 16);
    const int64_t o_m = carve(off, (int64_t)n_rows * a.sch * 8);
    const int64_t slots = (int64_t)n_rows * a.nch * a.pcap;
    const int64_t o_n = carve(off, (int64_t)n_rows * a.nch * 16);
    const int64_t o_v = carve(off, slots * 4);
    const int64_t o_i = carve(off, slots * 4);
    if (base) {
        a.rec = (float *)(base + o_r);
        a.st_mass = (float *)(base + o_m);
        if (a.nch) {
            a.part_n = (int32_t *)(base + o_n);
            a.part_v = (float *)(base + o_v);
            a.part_i = (int32_t *)(base + o_i);
        }
    }
    return off;
}

}  // namespace rlx
