// Token selection on the device: Sampler.Greedy, Sampler.Sample and the
// speculative decoder's acceptPhase / resampleRejected, one 512-thread
// work-group per row of logits.
//
// Reference: sampler.go:56-68 (Greedy), 73-210 (Sample: penalties ->
// temperature -> top-k -> fastexp32 softmax -> top-p -> min-p -> categorical
// draw), 213-262 (penalties); speculative.go:203-290 (acceptance test
// r < min(1, p_t/p_d), resample from norm(max(0, p_t - p_d))), 344-368
// (softmaxAlloc).  Each rng.Float32() draw is an input.
//
// Working set.  Sample first brings the row's scratch values (logits after
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
__device__ __forceinline__ void blk_sum2(float &a, float &b, SampLds &s) {
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
__device__ __forceinline__ void blk_max2(float &a, float &b, SampLds &s) {
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
__device__ __forceinline__ float blk_sum(float v, SampLds &s) {
    float z = 0.f;
    blk_sum2(v, z, s);
    return v;
}
__device__ __forceinline__ float blk_max(float v, SampLds &s) {
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
__device__ __forceinline__ float blk_scan_excl(float v, SampLds &s, float *total) {
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
__device__ __forceinline__ int blk_iscan_excl(int v, SampLds &s, int *total) {
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
__device__ __forceinline__ int blk_isum(int v, SampLds &s) {
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
template <class K>
__device__ uint32_t kth_key_w0(int n, int k, SampLds &s, K key, int lo_bit = 0) {
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
template <class K>
__device__ uint32_t kth_key_blk(int n, int k, SampLds &s, K key) {
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
template <class P, class Vf, class If>
__device__ int compact_blk(int n, int *tc, SampLds &s, P keep, Vf val, If idx) {
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
template <class P, class Vf>
__device__ int compact_chunks(int n, SampLds &s, P keep, Vf val) {
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
template <class P>
__device__ int filter_w0(int n, SampLds &s, P keep) {
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

// First entry (in order) at which the running sum of w exceeds r, mapped
// through idx; `dflt` when none does.  Chunk sums per thread (contiguous
// chunks), an ordered exclusive scan, then only the thread whose chunk
// holds r walks it; should rounding leave that walk without a hit, every
// later chunk is walked.
template <class W, class I>
__device__ int samp_draw(int n, float r, int dflt, SampLds &s, W w, I idx) {
    const int tid = threadIdx.x;
    const int C = (n + kST - 1) / kST;
    const int i0 = min(n, tid * C), i1 = min(n, i0 + C);
    float cs = 0.f;
#pragma unroll 8
    for (int i = i0; i < i1; i++) cs += w(i);
    float tot;
    const float start = blk_scan_excl(cs, s, &tot);
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
    return b == INT_MAX ? dflt : idx(b);
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
    auto pen = [&](float x, int f) {
        if (rp != 1.f && rp != 0.f) x = (x > 0.f) ? __fdiv_rn(x, rp) : __fmul_rn(x, rp);
        if (fp != 0.f) x = __fsub_rn(x, __fmul_rn(fp, (float)f));
        if (pp != 0.f) x = __fsub_rn(x, pp);
        return x;
    };
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

__global__ __launch_bounds__(kST) void sample_kernel(const SampleArgs a) {
    __shared__ SampLds s;
    const int b = blockIdx.x;
    Src c;
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

// ---- speculative acceptance ---------------------------------------------------
__device__ __forceinline__ float spec_p(const float *row, int v, float m, bool norm, float inv) {
    const float e = fastexp32_dev(__fsub_rn(row[v], m));
    return norm ? __fmul_rn(e, inv) : e;
}

// acceptPhase for one sequence (speculative.go:203-244): accept draft i
// while u_i < min(1, p_t/max(p_d, 1e-10)); on the first rejection draw the
// replacement from norm(max(0, p_t - p_d)) (resampleRejected 247-290, the
// target distribution if that is empty); all accepted: Sample the target's
// next row without penalties.  The draft and target rows of a position are
// reduced together (softmaxAlloc, speculative.go:344-368: max, then the sum
// of fastexp32 weights) with 16-byte loads; the resample weights are staged
// in LDS for the draw when the vocabulary fits.
__global__ __launch_bounds__(kST) void spec_accept_kernel(const SpecArgs a) {
    __shared__ SampLds s;
    const int b = blockIdx.x, tid = threadIdx.x;
    // draft counts and ids come from the device in rlx_spec_accept_async:
    // the count is clamped to [0, max_k], an id outside [0, V) is rejected
    // (rlx_spec_accept checks both on the host)
    const int V = a.V;
    const int k = min(max(a.n_draft[b], 0), a.max_k);
    const float *u = a.u + (int64_t)b * (a.max_k + 1);
    const float *dl = a.d_logits + (int64_t)b * a.max_k * V;
    const float *tl = a.t_logits + (int64_t)b * (a.max_k + 1) * V;
    for (int i = 0; i < k; i++) {
        const float *dr = dl + (int64_t)i * V, *tr = tl + (int64_t)i * V;
        const bool vec = ((((uintptr_t)dr) | ((uintptr_t)tr)) & 15) == 0 && (V & 3) == 0;
        float dm = -INFINITY, tm = -INFINITY;
        if (vec) {
            const float4 *d4 = (const float4 *)dr, *t4 = (const float4 *)tr;
#pragma unroll 8
            for (int v = tid; v < V / 4; v += kST) {
                const float4 x = d4[v], y = t4[v];
                dm = fmaxf(dm, fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)));
                tm = fmaxf(tm, fmaxf(fmaxf(y.x, y.y), fmaxf(y.z, y.w)));
            }
        } else {
#pragma unroll 8
            for (int v = tid; v < V; v += kST) {
                dm = fmaxf(dm, dr[v]);
                tm = fmaxf(tm, tr[v]);
            }
        }
        blk_max2(dm, tm, s);
        float ds = 0.f, ts = 0.f;
        if (vec) {
            const float4 *d4 = (const float4 *)dr, *t4 = (const float4 *)tr;
#pragma unroll 8
            for (int v = tid; v < V / 4; v += kST) {
                const float4 x = d4[v], y = t4[v];
                ds += fastexp32_dev(__fsub_rn(x.x, dm));
                ds += fastexp32_dev(__fsub_rn(x.y, dm));
                ds += fastexp32_dev(__fsub_rn(x.z, dm));
                ds += fastexp32_dev(__fsub_rn(x.w, dm));
                ts += fastexp32_dev(__fsub_rn(y.x, tm));
                ts += fastexp32_dev(__fsub_rn(y.y, tm));
                ts += fastexp32_dev(__fsub_rn(y.z, tm));
                ts += fastexp32_dev(__fsub_rn(y.w, tm));
            }
        } else {
#pragma unroll 8
            for (int v = tid; v < V; v += kST) {
                ds += fastexp32_dev(__fsub_rn(dr[v], dm));
                ts += fastexp32_dev(__fsub_rn(tr[v], tm));
            }
        }
        blk_sum2(ds, ts, s);
        const bool dn = ds > 0.f, tn = ts > 0.f;
        const float di = dn ? __fdiv_rn(1.f, ds) : 1.f, ti = tn ? __fdiv_rn(1.f, ts) : 1.f;
        const int tok = a.d_tok[(int64_t)b * a.max_k + i];
        if (tok >= 0 && tok < V) {
            const float dP = spec_p(dr, tok, dm, dn, di), tP = spec_p(tr, tok, tm, tn, ti);
            float acc = __fdiv_rn(tP, dP > 1e-10f ? dP : 1e-10f);
            if (acc > 1.f) acc = 1.f;
            if (u[i] < acc) continue;
        }
        auto adj = [&](int v) {
            const float d = __fsub_rn(spec_p(tr, v, tm, tn, ti), spec_p(dr, v, dm, dn, di));
            return d < 0.f ? 0.f : d;
        };
        const bool lds = V <= kRowCap;
        float sa = 0.f;
#pragma unroll 4
        for (int v = tid; v < V; v += kST) {
            const float x = adj(v);
            if (lds) s.region[v] = x;
            sa += x;
        }
        const float SA = blk_sum(sa, s);  // (its barriers also publish the region)
        auto ident = [](int v) { return v; };
        int res;
        if (SA > 0.f) {
            const float inv = __fdiv_rn(1.f, SA);
            if (lds)
                res = samp_draw(V, u[i + 1], 0, s, [&](int v) { return __fmul_rn(s.region[v], inv); }, ident);
            else
                res = samp_draw(V, u[i + 1], 0, s, [&](int v) { return __fmul_rn(adj(v), inv); }, ident);
        } else {
            res = samp_draw(V, u[i + 1], 0, s, [&](int v) { return spec_p(tr, v, tm, tn, ti); }, ident);
        }
        if (tid == 0) {
            a.n_acc[b] = i;
            a.next[b] = res;
        }
        return;
    }
    Src c;
    load_row(
        c, s, tl + (int64_t)k * V, V, a.temperature, [](int) { return 0; }, [](int) { return 0; }, 0, 0.f,
        0.f, 0.f);
    const int t = sample_set(c, clamp_topk(a.top_k, V), clamp_topp(a.top_p), a.min_p, u[k], s);
    if (tid == 0) {
        a.n_acc[b] = k;
        a.next[b] = t;
    }
}

hipError_t launch_sample(hipStream_t st, const SampleArgs &a, int n_rows, hipEvent_t e0,
                         hipEvent_t e1) {
    return launch_timed(sample_kernel, dim3(n_rows), dim3(kST), st, e0, e1, a);
}

hipError_t launch_greedy(hipStream_t st, const float *logits, int64_t stride, int V, int n_rows,
                         int32_t *out, hipEvent_t e0, hipEvent_t e1) {
    return launch_timed(greedy_kernel, dim3(n_rows), dim3(kST), st, e0, e1, logits, stride, V, out);
}

hipError_t launch_spec_accept(hipStream_t st, const SpecArgs &a, int n_rows, hipEvent_t e0,
                              hipEvent_t e1) {
    return launch_timed(spec_accept_kernel, dim3(n_rows), dim3(kST), st, e0, e1, a);
}

}  // namespace rlx
