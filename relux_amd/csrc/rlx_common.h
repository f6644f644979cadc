// Shared device types, plan records and launcher declarations of librelux_kv.
//
// HBM layout of the paged caches (bf16 = uint16 bit patterns):
//   GQA K pool : [pool_pages][kv_heads][page_tokens/16][head_dim/32][16][32]
//                (16-token blocks stored k-step-major, see k_page_off; head_dim
//                <= 32: plain [16][head_dim] rows; head_dim is the stored one,
//                16/32/64/96/128/256, zero padded past the caller's)
//   GQA V pool : [pool_pages][kv_heads][head_dim][page_tokens]   (dim-major pages:
//                the tokens of one dim are contiguous, which is the operand
//                order the P.V matrix-core step consumes)
//   MLA pool   : [pool_pages][page_tokens][512 + 64]             (latent | rope key:
//                the caller's d_c <= 512 and d_r <= 64 elements, each zero padded)
//   page table : int32 [layers][max_seqs][max_pages_per_seq], -1 = empty entry
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

namespace rlx {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short sh4;
typedef __attribute__((ext_vector_type(4))) float fl4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

// Timing of the dominant kernels (rlx_cache_timing): a pair of events per
// launch, recorded just before and after it on the launch stream.  The
// events are created with hipEventDisableSystemFence (timing_event_flags):
// a default event's record performs a system-scope release -- an L2
// write-back -- whose cost lands inside the measured interval and delays
// the next launch.  The events are only read after a stream synchronize.
// RLX_TIME_FENCE=system restores default events and RLX_TIME_FENCE=device
// uses device-scope releases (comparison runs).
inline unsigned timing_event_flags() {
    static const unsigned f = [] {
        const char *e = getenv("RLX_TIME_FENCE");
        if (e && e[0] == 's') return (unsigned)hipEventDefault;
        if (e && e[0] == 'd') return (unsigned)hipEventReleaseToDevice;
        return (unsigned)hipEventDisableSystemFence;
    }();
    return f;
}

// Launch of a kernel that may be timed (e0 / e1 non-null).
template <typename... P, typename... A>
inline hipError_t launch_timed(void (*k)(P...), dim3 grid, dim3 block, hipStream_t s,
                               hipEvent_t e0, hipEvent_t e1, A... args) {
    if (e0) (void)hipEventRecord(e0, s);
    k<<<grid, block, 0, s>>>(args...);
    hipError_t e = hipGetLastError();
    if (e1) (void)hipEventRecord(e1, s);
    return e;
}

// dtype_convert.go:15-24: integer round-to-nearest-even, no NaN special case.
__host__ __device__ __forceinline__ uint16_t bf16_rne(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__host__ __device__ __forceinline__ float bf16_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

constexpr int kLayoutHSD = 0;
constexpr int kLayoutSHD = 1;
constexpr int kMaskCausal = 0;
constexpr int kMaskRef = 1;
constexpr int kMaskNone = 2;

constexpr int kMlaDc = 512;
constexpr int kMlaDr = 64;
constexpr int kMlaRow = kMlaDc + kMlaDr;  // 576 bf16 = 1152 B per token

// Element offset of (slot s, dim d) inside one kv head's K page.  Each
// 16-token block of the page is stored k-step-major: D/32 slabs of
// [16 tokens][32 dims] (head_dim <= 32: plain [16 tokens][D] rows).  A
// decode wave's MFMA A operand for one 32-wide k-step (16 rows x 64 B) is
// then 1 KB of contiguous memory per load instruction instead of 16
// half-lines, which is what lets the K stream reach the same HBM rate as
// the V stream.  Blocks start where row-major blocks would (block b at
// 16 * b * D), so page and block addressing are unchanged.
__host__ __device__ __forceinline__ int64_t k_page_off(int s, int d, int D) {
    if (D <= 32) return (int64_t)s * D + d;
    return ((int64_t)(s >> 4) * (D >> 5) + (d >> 5)) * 512 + (s & 15) * 32 + (d & 31);
}

// One table write: table[idx] = val.  Indices in one batch are unique.
struct Patch {
    int32_t idx;
    int32_t val;
};

// One appended token: destination page/slot and where its rows sit in the
// caller's source buffer (sequence's first call-row and its row count).
struct AppendTok {
    int32_t page;
    int32_t slot;
    int32_t seq_row0;
    int32_t seq_n;
};

// One sequence of an attention / gather call.
struct AttRow {
    int32_t tab;     // flat index of the sequence's first live table entry
    int32_t len;     // live tokens
    int32_t nq;      // query rows (the last nq live tokens)
    int32_t qrow;    // first call-row of this sequence's queries / outputs
    int32_t nsplit;  // context splits
    int32_t part;    // first partial slot of this sequence
    int32_t q0;      // GQA decode query tiling: first query of this row ...
    int32_t qn;      // ... and its query count (q0 = 0, qn = nq untiled)
};

// ---- per-call plans in the kernel arguments --------------------------------
// A small plan (the row list of a decode call, the patches and token
// destinations of an append) travels inside the kernel arguments instead of
// a staged host-to-device copy: one copy dispatch and one dependency less
// per call.  Kernels that take a plan take it as their FIRST argument, so it
// sits at offset 0 of the kernel-argument segment.
constexpr int kPlanArgBytes = 2048;
struct alignas(16) PlanArg {
    unsigned char b[kPlanArgBytes];
};
struct NoPlan {
    int unused;
};
template <bool ARG>
struct PlanSel {
    using T = NoPlan;
};
template <>
struct PlanSel<true> {
    using T = PlanArg;
};
typedef __attribute__((address_space(4))) const unsigned char kplan_byte;
__device__ __forceinline__ kplan_byte *kernarg_plan() {
    return (kplan_byte *)__builtin_amdgcn_kernarg_segment_ptr();
}
static_assert(sizeof(AttRow) == 32, "AttRow is 8 int32");
template <bool ARG>
__device__ __forceinline__ AttRow plan_row(const AttRow *rows, int i) {
    if constexpr (ARG) {
        const __attribute__((address_space(4))) int32_t *p =
            (const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + i * sizeof(AttRow));
        AttRow r;
        r.tab = p[0];
        r.len = p[1];
        r.nq = p[2];
        r.qrow = p[3];
        r.nsplit = p[4];
        r.part = p[5];
        r.q0 = p[6];
        r.qn = p[7];
        return r;
    } else {
        return rows[i];
    }
}
// Append plans: patches at byte 0, tokens at byte tok_off of the plan.
template <bool ARG>
__device__ __forceinline__ Patch plan_patch(const Patch *patches, int i) {
    if constexpr (ARG) {
        const __attribute__((address_space(4))) int32_t *p =
            (const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + i * sizeof(Patch));
        return Patch{p[0], p[1]};
    } else {
        return patches[i];
    }
}
template <bool ARG>
__device__ __forceinline__ AppendTok plan_tok(const AppendTok *toks, int tok_off, int i) {
    if constexpr (ARG) {
        const __attribute__((address_space(4))) int32_t *p =
            (const __attribute__((address_space(4))) int32_t *)(kernarg_plan() + tok_off +
                                                                i * sizeof(AppendTok));
        return AppendTok{p[0], p[1], p[2], p[3]};
    } else {
        return toks[i];
    }
}
// ---- append bodies shared by the append kernels and fused launches -------
// Load 8 consecutive source elements (f32 or bf16) and convert them to bf16
// with the reference's integer RNE rule (dtype_convert.go:15-24).
__device__ __forceinline__ void load8_bf16(const void *src, int64_t off, int src_bf16,
                                           uint16_t (&o)[8]) {
    if (src_bf16) {
        u32x4 v = *(const u32x4 *)((const uint16_t *)src + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = (uint16_t)(v[i] & 0xFFFFu);
            o[2 * i + 1] = (uint16_t)(v[i] >> 16);
        }
    } else {
        const float4 *f = (const float4 *)((const float *)src + off);
        float4 a = f[0], b = f[1];
        o[0] = bf16_rne(a.x); o[1] = bf16_rne(a.y); o[2] = bf16_rne(a.z); o[3] = bf16_rne(a.w);
        o[4] = bf16_rne(b.x); o[5] = bf16_rne(b.y); o[6] = bf16_rne(b.z); o[7] = bf16_rne(b.w);
    }
}

// One source element as bf16 bits (f32 sources: BF16FromF32, dtype_convert.go:15-24).
__device__ __forceinline__ uint16_t load1_bf16(const void *src, int64_t i, int src_bf16) {
    return src_bf16 ? ((const uint16_t *)src)[i] : bf16_rne(((const float *)src)[i]);
}

// MLA append, thread gid: table patch gid (gid < n_patch), and chunk gid of
// the n_tok x 72 chunks of 8 elements of the stored 576-element rows:
// elements [0, 512) hold the latent c (the caller's d_c of them, then
// zeros), [512, 576) the rope key (d_r, then zeros).  Chunks wholly inside
// the caller's data take one 8-element load when the source row stride
// allows it; the rest go element by element.
template <bool ARG>
__device__ __forceinline__ void mla_append_thread(int64_t gid, uint16_t *pool, int32_t *table,
                                                  const Patch *patches, int n_patch,
                                                  const AppendTok *toks, int tok_off, int n_tok,
                                                  const void *c_src, const void *kr_src,
                                                  int src_bf16, int dc, int dr, int P) {
    if (gid < n_patch) {
        const Patch pt = plan_patch<ARG>(patches, (int)gid);
        table[pt.idx] = pt.val;
    }
    constexpr int chunks = kMlaRow / 8;  // 72
    if (gid >= (int64_t)n_tok * chunks) return;
    const int t = (int)(gid / chunks);
    const int ch = (int)(gid - (int64_t)t * chunks);
    const AppendTok tk = plan_tok<ARG>(toks, tok_off, t);
    const bool lat = ch < kMlaDc / 8;
    const void *src = lat ? c_src : kr_src;
    const int width = lat ? dc : dr;                     // caller's elements per row
    const int e0 = lat ? ch * 8 : (ch - kMlaDc / 8) * 8;  // first element of the chunk
    uint16_t v[8];
    if (e0 + 8 <= width && width % 8 == 0) {
        load8_bf16(src, (int64_t)t * width + e0, src_bf16, v);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = (e0 + i < width) ? load1_bf16(src, (int64_t)t * width + e0 + i, src_bf16) : (uint16_t)0;
    }
    u32x4 pk;
#pragma unroll
    for (int i = 0; i < 4; i++) pk[i] = (uint32_t)v[2 * i] | ((uint32_t)v[2 * i + 1] << 16);
    *(u32x4 *)(pool + ((int64_t)tk.page * P + tk.slot) * kMlaRow + ch * 8) = pk;
}

// An MLA append carried by another launch (rlx_mla_append_attend: the
// absorb launch of the attention that follows).  plan non-null: patches and
// tokens in the kernel arguments (tokens at byte tok_off); else the device
// arrays patches / toks.
struct MlaAppendJob {
    const PlanArg *plan;
    int tok_off;
    uint16_t *pool;
    int32_t *table;
    const Patch *patches;
    int n_patch;
    const AppendTok *toks;
    int n_tok;
    const void *c_src;
    const void *kr_src;
    int src_bf16, dc, dr, P;
};

// (row, split) of a decode work-group: from the device work list, or -- plan
// in the arguments -- by binary search of the rows' first partial slots
// (wave-uniform scalar loads).
template <bool ARG>
__device__ __forceinline__ int2 plan_work(const int2 *work, int n_rows, int b) {
    if constexpr (ARG) {
        // part is field 5 of each 8-int row
        const __attribute__((address_space(4))) int32_t *p =
            (const __attribute__((address_space(4))) int32_t *)kernarg_plan();
        int lo = 0, hi = n_rows - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p[mid * 8 + 5] <= b)
                lo = mid;
            else
                hi = mid - 1;
        }
        return int2{lo, b - p[lo * 8 + 5]};
    } else {
        return work[b];
    }
}


// Upper bound on context splits of one sequence (the runtime sizes splits so
// that it holds).
constexpr int kMaxSplits = 1024;

// Merge weights of n split partials, computed by wave 0 of the block:
// fac[s] = 2^(m_s - M) (0 for an empty split), M = max_s m_s, and the
// return value (in *inv_l, LDS) is 1 / sum_s fac[s] l_s (0 if nothing was
// attended).  ml points at split 0's (m, l) pair; consecutive splits are
// `stride` pairs apart.  Callers __syncthreads() before reading fac/inv_l.
__device__ __forceinline__ void merge_weights(const float *__restrict__ ml, int64_t stride,
                                              int n, float *fac, float *inv_l) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    float M = -INFINITY;
    for (int s = lane; s < n; s += 64) {
        const float m = ml[(int64_t)s * stride * 2];
        fac[s] = m;
        M = fmaxf(M, m);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    float L = 0.f;
    for (int s = lane; s < n; s += 64) {
        const float m = fac[s];
        const float f = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - M);
        fac[s] = f;
        L += f * ml[(int64_t)s * stride * 2 + 1];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o);
    if (lane == 0) *inv_l = (L > 0.f) ? 1.f / L : 0.f;
}

// ---- token selection (rlx_sampling.hip) ------------------------------------
constexpr int kSampMaxVocab = 1 << 18;  // seen-token bitmap: 32 KB of LDS
constexpr int kSampMaxSeen = 4096;      // distinct tokens of a repetition window

struct SampleArgs {
    const float *logits;
    int64_t stride;  // elements between rows
    int V;
    float temperature;
    int top_k;
    float top_p, min_p;
    float rp, fp, pp;          // repeat / frequency / presence penalty
    const int32_t *seen_tok;   // per row: distinct window tokens, ascending
    const int32_t *seen_freq;  // ... and their counts
    const int32_t *seen_off;   // n_rows + 1 offsets; nullptr: no penalties
    // rlx_sample_async: the windows are counted on the device instead, from
    // row b's history hist[b * hist_stride .. + hist_len[b]) (hist nullptr:
    // the seen_* lists above, or no penalties)
    const int32_t *hist;
    int64_t hist_stride;
    const int32_t *hist_len;
    int window;                // repeat_window; <= 0: the whole history
    const float *u;            // one draw per row
    int32_t *out;
    // vocabulary split (nch > 0, set by plan_sample_split): row b's chunk c
    // covers entries [c * pch, min(V, (c + 1) * pch)) and leaves its top-k
    // candidates at part_v / part_i[(b * nch + c) * pcap ..] with its record
    // part_n[(b * nch + c) * 4 ..] = {count (-1: overflow), lower bound key
    // of its k-th largest, largest key, 0}
    int nch, pch, pcap;
    float *part_v;
    int32_t *part_i, *part_n;
};

struct SpecArgs {
    const float *d_logits;  // [rows][max_k][V]
    const float *t_logits;  // [rows][max_k + 1][V]
    const int32_t *d_tok;   // [rows][max_k]
    const int32_t *n_draft;  // [rows]
    int max_k, V;
    const float *u;  // [rows][max_k + 1] draws in order
    float temperature;
    int top_k;
    float top_p, min_p;
    int32_t *n_acc, *next;
    // per (row, position, side) figures (set by plan_spec_split):
    // rec[((b * max_k + i) * 2 + side) * 4 + {0, 1, 2}]: the row's max, its
    // fastexp32 sum, the draft token's probability (side 0 draft, 1 target);
    // st_mass[(b * sch + c) * 2 + {0, 1}]: the first rejection's chunk c
    // sums of max(0, p_t - p_d) and of p_t
    float *rec, *st_mass;
    int sch;
    // the next target row's top-k chunk lists, as SampleArgs
    int nch, pch, pcap;
    float *part_v;
    int32_t *part_i, *part_n;
};

// (e0, e1: optional timing events attached to the kernel's dispatch.)
hipError_t launch_sample(hipStream_t s, const SampleArgs &a, int n_rows, hipEvent_t e0 = nullptr,
                         hipEvent_t e1 = nullptr);
hipError_t launch_greedy(hipStream_t s, const float *logits, int64_t stride, int V, int n_rows,
                         int32_t *out, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
hipError_t launch_spec_accept(hipStream_t s, const SpecArgs &a, int n_rows,
                              hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
// Chunking and device scratch of the split token selection, from the
// arguments' vocabulary and sampler: returns the scratch bytes the call
// needs and, with `base` non-null, points the arguments into it (base: 256-B
// aligned).  Fails (-1) when a launch would exceed the grid's limits.
int64_t plan_sample_split(SampleArgs &a, int n_rows, char *base);
int64_t plan_spec_split(SpecArgs &a, int n_rows, char *base);

// ---- launchers (stream-ordered, return hipError_t of the launch) ----------
hipError_t launch_patch(hipStream_t s, int32_t *table, const Patch *p, int n);
hipError_t launch_patch_plan(hipStream_t s, int32_t *table, const PlanArg &plan, int n);
hipError_t launch_fill_i32(hipStream_t s, int32_t *dst, int32_t val, int64_t n);
// Page copies (spill tier): copy i moves `bytes` from src[i] to dst[i]; the
// pointer arrays are device-readable.
hipError_t launch_page_copy(hipStream_t s, const uint64_t *src, const uint64_t *dst, int n, int64_t bytes);

// plan: patches and tokens in the kernel arguments (tokens at byte tok_off);
// nullptr: patches / toks are device arrays.
hipError_t launch_kv_append(hipStream_t s, const PlanArg *plan, int tok_off, uint16_t *kpool,
                            uint16_t *vpool, int32_t *table,
                            const Patch *patches, int n_patch, const AppendTok *toks, int n_tok,
                            const void *k_src, const void *v_src, int src_bf16, int layout,
                            int kvh, int hd, int hdi, int P);
hipError_t launch_mla_append(hipStream_t s, const PlanArg *plan, int tok_off, uint16_t *pool,
                             int32_t *table, const Patch *patches,
                             int n_patch, const AppendTok *toks, int n_tok, const void *c_src,
                             const void *kr_src, int src_bf16, int dc, int dr, int P);

// rows of sw elements (esz = 2 or 4 bytes) to rows of dw: copied, then zeros.
hipError_t launch_repack_rows(hipStream_t s, const void *src, int sw, void *dst, int dw,
                              int64_t rows, int esz);
hipError_t launch_kv_gather(hipStream_t s, const uint16_t *kpool, const uint16_t *vpool,
                            const int32_t *table, const AttRow *rows, int n_rows, int max_len,
                            uint16_t *k_out, uint16_t *v_out, int kvh, int hd, int hdi, int P);
// The reference KVCache's byte image of a GQA sequence, gathered into
// scratch pages of the pool's layout.  Append i of a sequence put its
// [KVH, S_i, D] block raw into rows [r_i, r_i + S_i) of a [cap][KVH * D]
// buffer (kvcache.go:286-287, copyInto 407-423), and attention reads head h
// at token t from flat row h * T + t (mha.go:305-310): scratch (h, t) gets
// the logical row (kvh', r_i + s) of the D-row at flat index h * T + t =
// r_i * KVH + kvh' * S_i + s.
struct RefImgSeq {
    int32_t src_tab;    // table index of the sequence's first live page
    int32_t len;        // T
    int32_t chunk0;     // first of its chunks in the chunk list
    int32_t n_chunks;
    int32_t dst_page0;  // first scratch page (scratch pages of a sequence are consecutive)
    int32_t pad[3];
};
hipError_t launch_ref_image_gather(hipStream_t s, const uint16_t *kpool, const uint16_t *vpool,
                                   const int32_t *table, const RefImgSeq *seqs, int n_seqs,
                                   int max_len, const int2 *chunks, int kvh, int hd, int P,
                                   uint16_t *dk, uint16_t *dv, int32_t *dtable, int n_pages);
hipError_t launch_mla_gather(hipStream_t s, const uint16_t *pool, const int32_t *table,
                             const AttRow *rows, int n_rows, int max_len, uint16_t *c_out,
                             uint16_t *kr_out, int dc, int dr, int P);

// plan: the rows in the kernel arguments (nullptr: rows and work on the device).
hipError_t launch_gqa_decode(hipStream_t s, const PlanArg *plan, const uint16_t *kpool,
                             const uint16_t *vpool, const int32_t *table, const AttRow *rows,
                             int n_rows, const int4 *ranges, int n_ranges, const void *q, int q_bf16,
                             int layout, int H, int KVH, int hd, int hdi, int P, int total64,
                             int snap64, int ranges_off, float qscale,
                             int mask_mode, int nqt, float *part_o, float *part_ml, void *out,
                             int out_bf16, int max_qr, hipEvent_t ev0, hipEvent_t ev1);

// Sources of the prefill kernel: the paged GQA cache, or (MLA) per-sequence
// decompressed K_c / V^T plus rope keys from the paged latent rows.
constexpr int kSrcPaged = 0;
constexpr int kSrcDense = 1;

// Max / sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48),
// delivered to every lane, with gfx950's row swaps: v_permlane16_swap
// exchanges the odd rows of its first operand with the even rows of its
// second, v_permlane32_swap the upper half of the first with the lower half
// of the second.  Swapping a value with itself pairs each row with its
// neighbour, then each half with the other -- VALU lane exchanges with no
// LDS round trip.  The sum is (x0 + x1) + (x2 + x3) in every lane.
__device__ __forceinline__ float rows4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Two floats to packed bf16 with the hardware conversion (v_cvt_pk_bf16_f32,
// round to nearest even): the same bits as bf16_rne for every non-NaN
// input.  For attention weights only; cache bytes keep bf16_rne, whose NaN
// behaviour is the reference's.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
// acc + lo + hi of a packed bf16 pair in one VALU op (v_dot2c_f32_bf16
// against (1, 1): the products are exact, f32 accumulation).
__device__ __forceinline__ float add_bf16x2(uint32_t w, float acc) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w),
                                           __builtin_bit_cast(bf16x2_t, 0x3F803F80u), acc, false);
}

// ---- global-to-LDS rings ----------------------------------------------

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// [15:14], expcnt[6:4], lgkmcnt[11:8]).
#define RLX_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// 16 bytes per lane from global memory straight into LDS at lds_base +
// 16 * lane (global_load_lds_dwordx4, non-temporal).  Written as inline asm
// so that the compiler does not see an LDS write it cannot place: it would
// otherwise wait for every outstanding load before each LDS read, which
// serialises the ring.  The kernel orders these loads itself (explicit
// vmcnt waits, then a barrier) and the "memory" clobber keeps the compiler
// from moving LDS accesses across them.
__device__ __forceinline__ void lds_dma16(const void *gptr, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, off nt"
        :
        : "v"(gptr), "s"(lds_base)
        : "memory", "m0");
}
// The same load addressed as a wave-uniform base (SGPR pair) plus a 32-bit
// per-lane byte offset: no 64-bit address arithmetic per lane.
__device__ __forceinline__ void lds_dma16(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 nt"
        :
        : "v"(voff), "s"(sbase), "s"(lds_base)
        : "memory", "m0");
}
// The same without the non-temporal hint: the lines stay in L2 for other
// work-groups that read them soon after (the MLA decode's head groups, the
// query tiles of a dense prefill head, the feature tiles of the expansion).
__device__ __forceinline__ void lds_dma16_keep(const void *gptr, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, off"
        :
        : "v"(gptr), "s"(lds_base)
        : "memory", "m0");
}
__device__ __forceinline__ void lds_dma16_keep(const void *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(sbase), "s"(lds_base)
        : "memory", "m0");
}

// Work-group barrier for the ring: this wave's LDS accesses complete, then
// s_barrier.  Unlike __syncthreads() it does not wait for outstanding
// global loads, so ring loads stay in flight across it.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Query rows (token x head pairs of one head group) per prefill work-group.
constexpr int kPrefillRows = 256;

struct PrefillArgs {
    const uint16_t *kpool;  // paged: K pages (k-step-major 16-token blocks)
    const uint16_t *vpool;  // paged: V dim-major pages
    const uint16_t *kc;     // dense: K_c [H][Tp][vd] of the H heads expanded, sequence s at + part*H*vd
    const uint16_t *vt;     // dense: V^T [H][vd][Tp], same sequence offsets
    const uint16_t *kr;     // dense: rope keys [Tp][64] per sequence, sequence s at row part
    const int32_t *table;
    const AttRow *rows;     // dense: part = token offset of the sequence, nsplit = Tp
    const int4 *work;       // (row, head group, query tile, unused)
    const void *q;          // paged: [rows][H][qd]; dense: q_nope [rows][H][qd]
    const void *q2;         // dense: q_rope [rows][H][qd2]
    void *out;
    int q_bf16, layout, out_bf16, mask_mode;
    int H, KVH, P;
    int HQ, h0;  // q / out rows hold HQ heads; work-item head h is the caller's head h0 + h
    int pshift;  // log2(P) when P is a power of two, else -1
    float qscale;
    int qd;      // q (dense: q_nope) dims per head row: row stride; dims past it are zero
    int qd2;     // dense: q_rope dims per head row (d_r)
    int od;      // output dims per head row (row stride; dims past it are not written)
    int vd;      // V dims per row as stored: paged, the pool's head_dim; dense, the padded
                 // head dim of K_c / V^T (128 or 256)
    int dv0;     // first V dim of this launch (head dims of 256 run as two 128-dim launches)
};

hipError_t launch_prefill(hipStream_t s, int src, int hd, const PrefillArgs &a, int n_work,
                          hipEvent_t ev0, hipEvent_t ev1);
// W_UK / W_UV [d_c][H*D] transposed to wt [H*DP][512] (once per call): head
// dims padded with zero rows to DP (128 or 256), channels with zero columns
// to 512.
hipError_t launch_mla_wt(hipStream_t s, const uint16_t *w_uk, const uint16_t *w_uv, int H, int D,
                         int dc, int DP, uint16_t *wt_k, uint16_t *wt_v);
// K_c [H][Tp][DP] / V^T [H][DP][Tp] of H heads from their transposed weights
// (wt_k, wt_v: the heads' rows of the transposed matrices).
hipError_t launch_mla_rope_gather(hipStream_t s, const uint16_t *pool, const int32_t *table,
                                  const AttRow *rows, const int2 *work, int n_work, int P,
                                  uint16_t *kr);
hipError_t launch_mla_expand(hipStream_t s, const uint16_t *pool, const int32_t *table,
                             const AttRow *rows, const int2 *work, int n_work, int H, int DP, int P,
                             const uint16_t *wt_k, const uint16_t *wt_v, uint16_t *kc, uint16_t *vt,
                             int cus);

// Fused projection + RoPE + paged append (at most 64 rows per launch).
constexpr int kProjRows = 64;
constexpr int kProjModelGQA = 0;
constexpr int kProjModelMLA = 1;
constexpr int kProjModelOut = 2;  // out = x.W (+ residual): D = output features
// Matrices packed by launch_pack_proj: matrix i holds nh[i] heads of tw[i]
// columns, each padded to pw[i] features with zero columns (unused entries:
// nh = 0).
struct PackSrc {
    const void *m[4];
    int nh[4], tw[4], pw[4];
};
hipError_t launch_pack_proj(hipStream_t s, const PackSrc &src, int w_bf16, int K, uint16_t *out);
// Shapes of a projection: GQA (H, KVH, D = the caller's head dim, DS = the
// pool's, DW = the packed features per head); MLA (H, D = q_c dims per head,
// DW = packed q_c features per head,
// DR / DC = d_r / d_c and DRP / DCP = the same rounded up to 16, the packed
// widths of the rope heads and of the latent); kProjOut (D = output
// features, DW = the same rounded up to 16, the packed ones).
struct ProjDims {
    int H, KVH, D, DS, DR, DRP, DC, DCP, DW;
};
// Packed features per GQA head: the head dim when the q and k parts are
// whole 16-feature tiles (H D and KVH D multiples of 16), else the head dim
// rounded up to 16 (zero weights past it).
__host__ __device__ inline int gqa_pack_width(int H, int KVH, int D) {
    return ((H * D) % 16 == 0 && (KVH * D) % 16 == 0) ? D : (D + 15) / 16 * 16;
}
// Packed q_c features per MLA head: the head dim when the q_c part is whole
// 16-feature tiles (H D a multiple of 16), else rounded up to 16.
__host__ __device__ inline int mla_pack_width(int H, int D) {
    return (H * D) % 16 == 0 ? D : (D + 15) / 16 * 16;
}
__host__ __device__ inline int proj_features(int model, const ProjDims &pd) {
    return model == kProjModelGQA ? (pd.H + 2 * pd.KVH) * pd.DW
         : model == kProjModelMLA ? pd.H * (pd.DW + pd.DRP) + pd.DCP + pd.DRP
                                  : pd.DW;
}
hipError_t launch_proj_pad_zero(hipStream_t s, int model, const PlanArg *plan, const AppendTok *toks,
                                int tok_off, int rows, const ProjDims &pd, uint16_t *kpool,
                                uint16_t *vpool, int P);
hipError_t launch_proj(hipStream_t s, int model, const PlanArg *plan, const Patch *patches,
                       int n_patch, const AppendTok *toks, const int32_t *pos, int tok_off,
                       int pos_off, int rows, const void *x, int x_bf16, int K, const uint16_t *wp,
                       const ProjDims &pd, const float *rcos, const float *rsin, void *q_out,
                       void *q_out2, int q_bf16, uint16_t *kpool, uint16_t *vpool, int32_t *table,
                       int P, int cus, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);

// Work-groups of the decode kernels one CU holds at once (occupancy).
int mla_decode_wgs_per_cu(int nqt);

hipError_t launch_mla_decode(hipStream_t s, const PlanArg *plan, const uint16_t *pool,
                             const int32_t *table, const AttRow *rows, int n_rows,
                             const int2 *work, int n_work,
                             const void *q_nope, const void *q_rope, int q_bf16,
                             const uint16_t *w_uk, const uint16_t *w_uv, int H, int hd, int dc,
                             int dr, int total_q, int max_nq, int P, float qscale,
                             int mask_mode, int nqt, uint16_t *qlat, uint16_t *part_o,
                             float *part_ml, void *out, int out_bf16, int cus,
                             hipEvent_t ev0, hipEvent_t ev1, const MlaAppendJob *app = nullptr);

}  // namespace rlx
