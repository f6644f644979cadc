// Token selection on the device: Sampler.Greedy, Sampler.Sample and the
// speculative decoder's acceptPhase / resampleRejected, one 256-thread
// work-group per row of logits.
//
// Reference: sampler.go:56-68 (Greedy), 73-210 (Sample: penalties ->
// temperature -> top-k -> fastexp32 softmax -> top-p -> min-p -> categorical
// draw), 213-262 (penalties); speculative.go:203-290 (acceptance test
// r < min(1, p_t/p_d), resample from norm(max(0, p_t - p_d))), 344-368
// (softmaxAlloc).  Each rng.Float32() draw is an input.
//
// The reference sorts (argsortDescF32, kthLargest: selection sorts) and sums
// the vocabulary sequentially.  Here every stage is a pass over the row:
//   * the top-k threshold (k-th largest value) is a radix select on the
//     float's order-preserving key, 8 bits per pass, integer counts;
//   * the top-p cutoff is the key tau of the item where the descending
//     cumulative probability first reaches p: a radix walk, 4 bits per
//     pass, over per-bin probability sums; every item with key >= tau is
//     kept (the reference keeps only as many items tied at tau as its sort
//     order reaches: the one place the results can differ besides rounding);
//   * sums are per-thread sequential partials combined in a fixed order, so
//     a call is deterministic; they round differently from a sequential sum
//     by a few ulp, which moves a draw only when r lies within that of a
//     cumulative boundary;
//   * the categorical draw: per-thread chunk sums, an ordered exclusive
//     prefix, then each thread walks its chunk; the lowest hit wins.
// Arithmetic follows the reference's f32 order with explicitly rounded
// operations (no fused multiply-add): s/temp, fastexp32(x - max) with one
// multiply and one add (mha.go:823-833), p * f32(1/sum).
#include "rlx_common.h"

namespace rlx {

constexpr int kSampThreads = 256;

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

struct SampLds {
    float red[4];
    int hist[256];
    float bins[16][kSampThreads];
    float tot[16];
    float pre[kSampThreads];
    int sel_i[2];
    float sel_f;
    int best;
    int stok[kSampMaxSeen];
    float sval[kSampMaxSeen];
};

// Block reductions: per-thread values, 64-lane tree, then the 4 wave
// results in a fixed order; every thread returns the same value.
__device__ __forceinline__ float blk_sum(float v, SampLds &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s.red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((s.red[0] + s.red[1]) + s.red[2]) + s.red[3];
}
__device__ __forceinline__ float blk_max(float v, SampLds &s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_down(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s.red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(s.red[0], s.red[1]), fmaxf(s.red[2], s.red[3]));
}

// One row's sampling state: the value function (penalties, temperature,
// top-k mask) and the normalisation factors of each enabled stage.
struct RowCtx {
    const float *row;
    int V;
    const uint32_t *bits;  // seen-token bitmap (nseen > 0)
    int nseen;
    float temp;
    bool div;
    bool topk;
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

// scratch[v] after penalties and temperature, -inf if top-k drops it.
__device__ __forceinline__ float samp_val(const RowCtx &c, const SampLds &s, int v) {
    float x;
    if (c.nseen > 0 && ((c.bits[v >> 5] >> (v & 31)) & 1u)) {
        int lo = 0, hi = c.nseen - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s.stok[mid] < v)
                lo = mid + 1;
            else
                hi = mid;
        }
        x = s.sval[lo];
    } else {
        x = c.row[v];
    }
    if (c.div) x = __fdiv_rn(x, c.temp);
    if (c.topk && x < c.kthr) x = -INFINITY;
    return x;
}

// Probability of v after stage `stage` (1 softmax, 2 top-p, 3 min-p).
__device__ __forceinline__ float samp_prob(const RowCtx &c, const SampLds &s, int v, int stage) {
    const float x = samp_val(c, s, v);
    float p = (x == -INFINITY) ? 0.f : fastexp32_dev(__fsub_rn(x, c.m));
    if (c.n1) p = __fmul_rn(p, c.i1);
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

// First index v (in index order) at which the running sum of w(v) exceeds
// r; `dflt` when none does.
template <class W>
__device__ int samp_draw(int V, float r, int dflt, SampLds &s, W w) {
    const int tid = threadIdx.x;
    const int C = (V + kSampThreads - 1) / kSampThreads;
    const int v0 = min(V, tid * C), v1 = min(V, v0 + C);
    float cs = 0.f;
    for (int v = v0; v < v1; v++) cs += w(v);
    __syncthreads();
    s.pre[tid] = cs;
    if (tid == 0) s.best = INT_MAX;
    __syncthreads();
    if (tid == 0) {
        float a = 0.f;
        for (int i = 0; i < kSampThreads; i++) {
            const float t = s.pre[i];
            s.pre[i] = a;
            a += t;
        }
    }
    __syncthreads();
    float cum = s.pre[tid];
    for (int v = v0; v < v1; v++) {
        cum += w(v);
        if (r < cum) {
            atomicMin(&s.best, v);
            break;
        }
    }
    __syncthreads();
    const int b = s.best;
    return b == INT_MAX ? dflt : b;
}

// Sampler.Sample for one row (the row context's value function set up).
__device__ int sample_row(RowCtx &c, int top_k, float top_p, float min_p, float r, SampLds &s) {
    const int tid = threadIdx.x, V = c.V;
    c.topk = false;
    c.topp = false;
    c.minp = false;
    // Top-k threshold: the k-th largest value (sampler.go:100-114).
    if (top_k > 0) {
        uint32_t prefix = 0, mask = 0;
        int kk = top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += kSampThreads) s.hist[i] = 0;
            __syncthreads();
            for (int v = tid; v < V; v += kSampThreads) {
                const uint32_t key = fkey(samp_val(c, s, v));
                if ((key & mask) == prefix) atomicAdd(&s.hist[(key >> shift) & 255], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, d = 255;
                for (; d > 0; d--) {
                    if (cum + s.hist[d] >= kk) break;
                    cum += s.hist[d];
                }
                s.sel_i[0] = d;
                s.sel_i[1] = kk - cum;
            }
            __syncthreads();
            prefix |= (uint32_t)s.sel_i[0] << shift;
            mask |= 0xFFu << shift;
            kk = s.sel_i[1];
        }
        c.kthr = funkey(prefix);
        c.topk = true;
    }
    // Softmax with fastexp32 (sampler.go:117-138).
    float mx = -INFINITY;
    for (int v = tid; v < V; v += kSampThreads) mx = fmaxf(mx, samp_val(c, s, v));
    c.m = blk_max(mx, s);
    float sm = 0.f;
    for (int v = tid; v < V; v += kSampThreads) {
        const float x = samp_val(c, s, v);
        if (x != -INFINITY) sm += fastexp32_dev(__fsub_rn(x, c.m));
    }
    const float S1 = blk_sum(sm, s);
    c.n1 = S1 > 0.f;
    c.i1 = c.n1 ? __fdiv_rn(1.f, S1) : 1.f;
    // Top-p (sampler.go:141-165): radix walk for the cutoff key.
    if (top_p > 0.f && top_p < 1.f) {
        uint32_t prefix = 0, mask = 0;
        float above = 0.f;
        bool all = false;
        for (int shift = 28; shift >= 0 && !all; shift -= 4) {
#pragma unroll
            for (int j = 0; j < 16; j++) s.bins[j][tid] = 0.f;
            for (int v = tid; v < V; v += kSampThreads) {
                const float p = samp_prob(c, s, v, 1);
                const uint32_t key = fkey(p);
                if ((key & mask) == prefix) s.bins[(key >> shift) & 15][tid] += p;
            }
            __syncthreads();
            if (tid < 16) {
                float t = 0.f;
                for (int i = 0; i < kSampThreads; i++) t += s.bins[tid][i];
                s.tot[tid] = t;
            }
            __syncthreads();
            if (tid == 0) {
                float acc = above;
                int d = 15;
                for (; d >= 0; d--) {
                    if (acc + s.tot[d] >= top_p) break;
                    acc += s.tot[d];
                }
                // Nothing reaches p: on the first pass the whole row is kept
                // (the reference's cutoff stays n); deeper, rounding of the
                // sub-bin sums: keep the whole bin.
                s.sel_i[0] = (d < 0) ? 0 : d;
                s.sel_i[1] = (d < 0 && shift == 28) ? 1 : 0;
                s.sel_f = (d < 0) ? above : acc;
            }
            __syncthreads();
            if (s.sel_i[1]) {
                all = true;
                prefix = 0;
            } else {
                prefix |= (uint32_t)s.sel_i[0] << shift;
                mask |= 0xFu << shift;
                above = s.sel_f;
            }
            __syncthreads();
        }
        c.tau = prefix;
        c.topp = true;
        c.n2 = false;
        float k2 = 0.f;
        for (int v = tid; v < V; v += kSampThreads) k2 += samp_prob(c, s, v, 2);
        const float S2 = blk_sum(k2, s);
        c.n2 = S2 > 0.f;
        c.i2 = c.n2 ? __fdiv_rn(1.f, S2) : 1.f;
    }
    // Min-p (sampler.go:168-191).
    if (min_p > 0.f) {
        float mp = 0.f;
        for (int v = tid; v < V; v += kSampThreads) mp = fmaxf(mp, samp_prob(c, s, v, 2));
        mp = blk_max(mp, s);
        c.thr3 = __fmul_rn(mp, min_p);
        c.minp = true;
        c.n3 = false;
        float k3 = 0.f;
        for (int v = tid; v < V; v += kSampThreads) k3 += samp_prob(c, s, v, 3);
        const float S3 = blk_sum(k3, s);
        c.n3 = S3 > 0.f;
        c.i3 = c.n3 ? __fdiv_rn(1.f, S3) : 1.f;
    }
    // Categorical draw (sampler.go:194-206), n-1 if r is never reached.
    return samp_draw(V, r, V - 1, s, [&](int v) { return samp_prob(c, s, v, 3); });
}

__device__ void row_init(RowCtx &c, const float *row, int V, float temperature) {
    c.row = row;
    c.V = V;
    c.bits = nullptr;
    c.nseen = 0;
    float t = temperature;
    if (t <= 0.f) t = 1e-5f;
    c.temp = t;
    c.div = (t != 1.f);
    c.topk = c.topp = c.minp = false;
    c.n1 = c.n2 = c.n3 = false;
}

// top_k / top_p clamped as sampler.go:100-106, 141-144.
__device__ __forceinline__ int clamp_topk(int k, int V) { return (k < 0 || k >= V) ? 0 : k; }
__device__ __forceinline__ float clamp_topp(float p) { return (p <= 0.f || p > 1.f) ? 1.f : p; }

__global__ __launch_bounds__(kSampThreads) void sample_kernel(const SampleArgs a) {
    __shared__ SampLds s;
    extern __shared__ uint32_t seen_bits[];
    const int b = blockIdx.x, tid = threadIdx.x;
    RowCtx c;
    row_init(c, a.logits + (int64_t)b * a.stride, a.V, a.temperature);
    // Penalties (sampler.go:213-262) on the row's distinct window tokens,
    // given sorted with their counts; looked up through a bitmap.
    const int n0 = a.seen_off ? a.seen_off[b] : 0;
    const int ns = a.seen_off ? a.seen_off[b + 1] - n0 : 0;
    if (ns > 0) {
        const int words = (a.V + 31) >> 5;
        for (int i = tid; i < words; i += kSampThreads) seen_bits[i] = 0u;
        __syncthreads();
        for (int i = tid; i < ns; i += kSampThreads) {
            const int tok = a.seen_tok[n0 + i];
            float x = c.row[tok];
            if (a.rp != 1.f && a.rp != 0.f) x = (x > 0.f) ? __fdiv_rn(x, a.rp) : __fmul_rn(x, a.rp);
            if (a.fp != 0.f) x = __fsub_rn(x, __fmul_rn(a.fp, (float)a.seen_freq[n0 + i]));
            if (a.pp != 0.f) x = __fsub_rn(x, a.pp);
            s.stok[i] = tok;
            s.sval[i] = x;
            atomicOr(&seen_bits[tok >> 5], 1u << (tok & 31));
        }
        __syncthreads();
        c.bits = seen_bits;
        c.nseen = ns;
    }
    const int t = sample_row(c, clamp_topk(a.top_k, a.V), clamp_topp(a.top_p), a.min_p, a.u[b], s);
    if (tid == 0) a.out[b] = t;
}

// First index of the largest value (sampler.go:56-68).
__global__ __launch_bounds__(kSampThreads) void greedy_kernel(const float *__restrict__ logits,
                                                               int64_t stride, int V,
                                                               int32_t *__restrict__ out) {
    __shared__ float bv[kSampThreads];
    __shared__ int bi[kSampThreads];
    const float *row = logits + (int64_t)blockIdx.x * stride;
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int idx = INT_MAX;
    for (int v = tid; v < V; v += kSampThreads) {
        const float x = row[v];
        if (idx == INT_MAX || x > best) {
            best = x;
            idx = v;
        }
    }
    bv[tid] = best;
    bi[tid] = idx;
    __syncthreads();
    for (int o = kSampThreads / 2; o > 0; o >>= 1) {
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

// softmaxAlloc of one row (speculative.go:344-368): max and f32(1/sum).
__device__ void spec_softmax(const float *row, int V, SampLds &s, float *m, bool *norm, float *inv) {
    float mx = -INFINITY;
    for (int v = threadIdx.x; v < V; v += kSampThreads) mx = fmaxf(mx, row[v]);
    *m = blk_max(mx, s);
    float sm = 0.f;
    for (int v = threadIdx.x; v < V; v += kSampThreads) sm += fastexp32_dev(__fsub_rn(row[v], *m));
    const float S = blk_sum(sm, s);
    *norm = S > 0.f;
    *inv = *norm ? __fdiv_rn(1.f, S) : 1.f;
}

__device__ __forceinline__ float spec_p(const float *row, int v, float m, bool norm, float inv) {
    const float e = fastexp32_dev(__fsub_rn(row[v], m));
    return norm ? __fmul_rn(e, inv) : e;
}

// acceptPhase for one sequence (speculative.go:203-244): accept draft i
// while u_i < min(1, p_t/max(p_d, 1e-10)); on the first rejection draw the
// replacement from norm(max(0, p_t - p_d)) (resampleRejected 247-290, the
// target distribution if that is empty); all accepted: Sample the target's
// next row without penalties.
__global__ __launch_bounds__(kSampThreads) void spec_accept_kernel(const SpecArgs a) {
    __shared__ SampLds s;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int k = a.n_draft[b];
    const float *u = a.u + (int64_t)b * (a.max_k + 1);
    const float *dl = a.d_logits + (int64_t)b * a.max_k * a.V;
    const float *tl = a.t_logits + (int64_t)b * (a.max_k + 1) * a.V;
    for (int i = 0; i < k; i++) {
        const float *dr = dl + (int64_t)i * a.V, *tr = tl + (int64_t)i * a.V;
        float dm, di, tm, ti;
        bool dn, tn;
        spec_softmax(dr, a.V, s, &dm, &dn, &di);
        spec_softmax(tr, a.V, s, &tm, &tn, &ti);
        const int tok = a.d_tok[(int64_t)b * a.max_k + i];
        const float dP = spec_p(dr, tok, dm, dn, di), tP = spec_p(tr, tok, tm, tn, ti);
        float acc = __fdiv_rn(tP, dP > 1e-10f ? dP : 1e-10f);
        if (acc > 1.f) acc = 1.f;
        if (u[i] < acc) continue;
        auto adj = [&](int v) {
            const float d = __fsub_rn(spec_p(tr, v, tm, tn, ti), spec_p(dr, v, dm, dn, di));
            return d < 0.f ? 0.f : d;
        };
        float sa = 0.f;
        for (int v = tid; v < a.V; v += kSampThreads) sa += adj(v);
        const float SA = blk_sum(sa, s);
        int res;
        if (SA > 0.f) {
            const float inv = __fdiv_rn(1.f, SA);
            res = samp_draw(a.V, u[i + 1], 0, s, [&](int v) { return __fmul_rn(adj(v), inv); });
        } else {
            res = samp_draw(a.V, u[i + 1], 0, s, [&](int v) { return spec_p(tr, v, tm, tn, ti); });
        }
        if (tid == 0) {
            a.n_acc[b] = i;
            a.next[b] = res;
        }
        return;
    }
    RowCtx c;
    row_init(c, tl + (int64_t)k * a.V, a.V, a.temperature);
    const int t = sample_row(c, clamp_topk(a.top_k, a.V), clamp_topp(a.top_p), a.min_p, u[k], s);
    if (tid == 0) {
        a.n_acc[b] = k;
        a.next[b] = t;
    }
}

hipError_t launch_sample(hipStream_t st, const SampleArgs &a, int n_rows) {
    const size_t dyn = a.seen_off ? (size_t)((a.V + 31) >> 5) * 4 : 0;
    sample_kernel<<<n_rows, kSampThreads, dyn, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_greedy(hipStream_t st, const float *logits, int64_t stride, int V, int n_rows,
                         int32_t *out) {
    greedy_kernel<<<n_rows, kSampThreads, 0, st>>>(logits, stride, V, out);
    return hipGetLastError();
}

hipError_t launch_spec_accept(hipStream_t st, const SpecArgs &a, int n_rows) {
    spec_accept_kernel<<<n_rows, kSampThreads, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace rlx
