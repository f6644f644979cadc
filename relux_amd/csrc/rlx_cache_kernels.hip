// Page-table patches, paged append (scatter) and paged gather (View).
//
// These kernels are byte movers: HBM-bound, one pass, 16-byte accesses
// on the contiguous side of every copy.
#include <algorithm>

#include "rlx_common.h"

namespace rlx {

__global__ void patch_kernel(int32_t *__restrict__ table, const Patch *__restrict__ p, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) table[p[i].idx] = p[i].val;
}

__global__ void fill_i32_kernel(int32_t *__restrict__ dst, int32_t val, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = val;
}

hipError_t launch_patch(hipStream_t s, int32_t *table, const Patch *p, int n) {
    if (n <= 0) return hipSuccess;
    patch_kernel<<<(n + 255) / 256, 256, 0, s>>>(table, p, n);
    return hipGetLastError();
}

// Table patches carried in the kernel arguments (at most kPlanArgBytes / 8
// per launch): no device copy of the patch list is needed.
__global__ __launch_bounds__(256) void patch_plan_kernel(PlanArg plan, int32_t *__restrict__ table, int n) {
    const int i = threadIdx.x;
    if (i < n) {
        const Patch p = plan_patch<true>(nullptr, i);
        table[p.idx] = p.val;
    }
}

hipError_t launch_patch_plan(hipStream_t s, int32_t *table, const PlanArg &plan, int n) {
    if (n <= 0) return hipSuccess;
    if (n > kPlanArgBytes / (int)sizeof(Patch)) return hipErrorInvalidValue;
    patch_plan_kernel<<<1, 256, 0, s>>>(plan, table, n);
    return hipGetLastError();
}

hipError_t launch_fill_i32(hipStream_t s, int32_t *dst, int32_t val, int64_t n) {
    if (n <= 0) return hipSuccess;
    fill_i32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(dst, val, n);
    return hipGetLastError();
}

// Whole-page copies between the HBM pools and the host spill tier (pinned
// host memory, which the device addresses directly): copy i moves `bytes`
// (a multiple of 16) from src[i] to dst[i], one work-group per page.  One
// side of every copy crosses the host link, so each thread puts 8 loads in
// flight before its stores.
__global__ __launch_bounds__(256) void page_copy_kernel(const uint64_t *__restrict__ src,
                                                        const uint64_t *__restrict__ dst, int64_t bytes) {
    const u32x4 *s = (const u32x4 *)src[blockIdx.x];
    u32x4 *d = (u32x4 *)dst[blockIdx.x];
    const int64_t n = bytes / 16;
    for (int64_t i0 = 0; i0 < n; i0 += 8 * 256) {
        u32x4 r[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t i = i0 + u * 256 + threadIdx.x;
            if (i < n) r[u] = s[i];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t i = i0 + u * 256 + threadIdx.x;
            if (i < n) d[i] = r[u];
        }
    }
}

hipError_t launch_page_copy(hipStream_t s, const uint64_t *src, const uint64_t *dst, int n, int64_t bytes) {
    if (n <= 0 || bytes <= 0) return hipSuccess;
    page_copy_kernel<<<n, 256, 0, s>>>(src, dst, bytes);
    return hipGetLastError();
}

// GQA append.  Thread = (token, kv head, 8-dim chunk of the stored head
// dim hd).  K goes to its page (k_page_off layout) with one 16-byte store; V
// goes to a dim-major page (8 strided 2-byte stores).  The caller's rows
// hold hdi <= hd dims (a multiple of 8); the stored dims past hdi are
// written as zeros.  The first n_patch threads also apply the table
// patches; the scatter itself takes its destinations from the plan, not the
// table.
template <bool ARG>
__global__ void kv_append_kernel(typename PlanSel<ARG>::T plan, uint16_t *__restrict__ kpool,
                                 uint16_t *__restrict__ vpool, int32_t *__restrict__ table,
                                 const Patch *__restrict__ patches, int n_patch,
                                 const AppendTok *__restrict__ toks, int tok_off, int n_tok,
                                 const void *__restrict__ k_src, const void *__restrict__ v_src,
                                 int src_bf16, int layout, int kvh, int hd, int hdi, int P) {
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid < n_patch) {
        const Patch pt = plan_patch<ARG>(patches, (int)gid);
        table[pt.idx] = pt.val;
    }
    const int chunks = hd >> 3;
    const int64_t per_tok = (int64_t)kvh * chunks;
    if (gid >= (int64_t)n_tok * per_tok) return;
    const int t = (int)(gid / per_tok);
    const int rem = (int)(gid - (int64_t)t * per_tok);
    const int h = rem / chunks;
    const int d0 = (rem - h * chunks) * 8;
    const AppendTok tk = plan_tok<ARG>(toks, tok_off, t);
    const int j = t - tk.seq_row0;  // row within its sequence
    int64_t src_off;
    if (layout == kLayoutSHD)
        src_off = ((int64_t)t * kvh + h) * hdi + d0;
    else
        src_off = (int64_t)tk.seq_row0 * kvh * hdi + ((int64_t)h * tk.seq_n + j) * hdi + d0;
    uint16_t kv[8] = {0, 0, 0, 0, 0, 0, 0, 0}, vv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (d0 < hdi) {
        load8_bf16(k_src, src_off, src_bf16, kv);
        load8_bf16(v_src, src_off, src_bf16, vv);
    }
    uint16_t *kd = kpool + ((int64_t)tk.page * kvh + h) * P * hd + k_page_off(tk.slot, d0, hd);
    u32x4 pk;
#pragma unroll
    for (int i = 0; i < 4; i++) pk[i] = (uint32_t)kv[2 * i] | ((uint32_t)kv[2 * i + 1] << 16);
    *(u32x4 *)kd = pk;
    uint16_t *vd = vpool + (((int64_t)tk.page * kvh + h) * hd + d0) * P + tk.slot;
#pragma unroll
    for (int i = 0; i < 8; i++) vd[(int64_t)i * P] = vv[i];
}

hipError_t launch_kv_append(hipStream_t s, const PlanArg *plan, int tok_off, uint16_t *kpool,
                            uint16_t *vpool, int32_t *table, const Patch *patches, int n_patch,
                            const AppendTok *toks, int n_tok, const void *k_src, const void *v_src,
                            int src_bf16, int layout, int kvh, int hd, int hdi, int P) {
    int64_t work = (int64_t)n_tok * kvh * (hd / 8);
    if (work < n_patch) work = n_patch;
    if (work <= 0) return hipSuccess;
    // One-wave work-groups: a decode step's append (a few thousand threads,
    // each one load and a few stores) then spreads over as many CUs as it has
    // waves instead of sitting on a handful.
    const unsigned grid = (unsigned)((work + 63) / 64);
    if (plan)
        kv_append_kernel<true><<<grid, 64, 0, s>>>(*plan, kpool, vpool, table, patches, n_patch,
                                                   toks, tok_off, n_tok, k_src, v_src, src_bf16,
                                                   layout, kvh, hd, hdi, P);
    else
        kv_append_kernel<false><<<grid, 64, 0, s>>>(NoPlan{0}, kpool, vpool, table, patches,
                                                    n_patch, toks, tok_off, n_tok, k_src, v_src,
                                                    src_bf16, layout, kvh, hd, hdi, P);
    return hipGetLastError();
}

// MLA append (one thread per table patch and per 16-byte chunk of a stored
// row; mla_append_thread).
template <bool ARG>
__global__ void mla_append_kernel(typename PlanSel<ARG>::T plan, uint16_t *__restrict__ pool,
                                  int32_t *__restrict__ table, const Patch *__restrict__ patches,
                                  int n_patch, const AppendTok *__restrict__ toks, int tok_off,
                                  int n_tok, const void *__restrict__ c_src,
                                  const void *__restrict__ kr_src, int src_bf16, int dc, int dr,
                                  int P) {
    mla_append_thread<ARG>((int64_t)blockIdx.x * blockDim.x + threadIdx.x, pool, table, patches,
                           n_patch, toks, tok_off, n_tok, c_src, kr_src, src_bf16, dc, dr, P);
}

hipError_t launch_mla_append(hipStream_t s, const PlanArg *plan, int tok_off, uint16_t *pool,
                             int32_t *table, const Patch *patches, int n_patch,
                             const AppendTok *toks, int n_tok, const void *c_src,
                             const void *kr_src, int src_bf16, int dc, int dr, int P) {
    int64_t work = (int64_t)n_tok * (kMlaRow / 8);
    if (work < n_patch) work = n_patch;
    if (work <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((work + 255) / 256);
    if (plan)
        mla_append_kernel<true><<<grid, 256, 0, s>>>(*plan, pool, table, patches, n_patch, toks,
                                                     tok_off, n_tok, c_src, kr_src, src_bf16, dc, dr, P);
    else
        mla_append_kernel<false><<<grid, 256, 0, s>>>(NoPlan{0}, pool, table, patches, n_patch,
                                                      toks, tok_off, n_tok, c_src, kr_src,
                                                      src_bf16, dc, dr, P);
    return hipGetLastError();
}

// Paged gather of GQA K and V into dense [kvh][T][hd] per sequence.
// grid.y = sequence of the call; x covers the sequence's work.  K: thread =
// (token, head, 8-dim chunk), 16-byte read and write.  V: thread = (head, dim,
// 8-token chunk), 16-byte read of a dim-major page row, 8 strided writes.
__global__ void kv_gather_kernel(const uint16_t *__restrict__ kpool,
                                 const uint16_t *__restrict__ vpool,
                                 const int32_t *__restrict__ table, const AttRow *__restrict__ rows,
                                 uint16_t *__restrict__ k_out, uint16_t *__restrict__ v_out,
                                 int kvh, int hd, int hdi, int P) {
    // Stored pages hold hd dims per head; the dense output holds the
    // caller's hdi (<= hd, a multiple of 8) and drops the zero padding.
    const AttRow R = rows[blockIdx.y];
    const int chunks = hdi >> 3;
    const int64_t nk = (int64_t)R.len * kvh * chunks;
    const int64_t base = (int64_t)R.qrow * kvh * hdi;  // qrow holds the output token offset
    for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < nk;
         gid += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(gid / ((int64_t)kvh * chunks));
        const int rem = (int)(gid - (int64_t)t * kvh * chunks);
        const int h = rem / chunks;
        const int d0 = (rem - h * chunks) * 8;
        const int page = table[R.tab + t / P];
        const int slot = t % P;
        u32x4 v = *(const u32x4 *)(kpool + ((int64_t)page * kvh + h) * P * hd + k_page_off(slot, d0, hd));
        *(u32x4 *)(k_out + base + ((int64_t)h * R.len + t) * hdi + d0) = v;
    }
    const int tchunks = (R.len + 7) >> 3;
    const int64_t nv = (int64_t)kvh * hdi * tchunks;
    for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < nv;
         gid += (int64_t)gridDim.x * blockDim.x) {
        const int tc = (int)(gid % tchunks);
        const int hd_i = (int)(gid / tchunks);
        const int h = hd_i / hdi;
        const int d = hd_i - h * hdi;
        const int t0 = tc * 8;
        const int page = table[R.tab + t0 / P];
        const int slot = t0 % P;
        u32x4 v = *(const u32x4 *)(vpool + (((int64_t)page * kvh + h) * hd + d) * P + slot);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (t0 + i < R.len) {
                uint32_t w = v[i >> 1];
                v_out[base + ((int64_t)h * R.len + t0 + i) * hdi + d] =
                    (uint16_t)((i & 1) ? (w >> 16) : (w & 0xFFFFu));
            }
        }
    }
}

hipError_t launch_kv_gather(hipStream_t s, const uint16_t *kpool, const uint16_t *vpool,
                            const int32_t *table, const AttRow *rows, int n_rows, int max_len,
                            uint16_t *k_out, uint16_t *v_out, int kvh, int hd, int hdi, int P) {
    if (n_rows <= 0 || max_len <= 0) return hipSuccess;
    int64_t work = (int64_t)max_len * kvh * (hd / 8);
    int blocks = (int)((work + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    kv_gather_kernel<<<dim3(blocks, n_rows), 256, 0, s>>>(kpool, vpool, table, rows, k_out, v_out,
                                                          kvh, hd, hdi, P);
    return hipGetLastError();
}

// Caller rows whose head width is not a multiple of 8 cross the C boundary
// through this copy: `rows` rows of sw 16-bit units to rows of dw units,
// the first min(sw, dw) units copied and the rest of a wider row zeroed
// (f32 rows count two units per element).  Thread = one destination unit.
__global__ void repack_rows_kernel(const uint16_t *__restrict__ src, int sw, uint16_t *__restrict__ dst,
                                   int dw, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / dw;
        const int k = (int)(i - r * dw);
        dst[i] = k < sw ? src[r * sw + k] : (uint16_t)0;
    }
}

hipError_t launch_repack_rows(hipStream_t s, const void *src, int sw, void *dst, int dw,
                              int64_t rows, int esz) {
    const int u = esz / 2;
    const int64_t n = rows * dw * u;
    if (n <= 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
    repack_rows_kernel<<<blocks, 256, 0, s>>>((const uint16_t *)src, sw * u, (uint16_t *)dst, dw * u, n);
    return hipGetLastError();
}

// Thread = (sequence, kv head h, token t, 8-dim octet).  chunks[c] =
// (first token r_c, size S_c) of each append, in order.
__global__ void ref_image_gather_kernel(const uint16_t *__restrict__ kpool,
                                        const uint16_t *__restrict__ vpool,
                                        const int32_t *__restrict__ table,
                                        const RefImgSeq *__restrict__ seqs,
                                        const int2 *__restrict__ chunks, int kvh, int hd, int P,
                                        uint16_t *__restrict__ dk, uint16_t *__restrict__ dv,
                                        int32_t *__restrict__ dtable, int n_pages) {
    const RefImgSeq q = seqs[blockIdx.y];
    if (blockIdx.y == 0)  // the scratch table: page i is entry i
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_pages;
             i += (int64_t)gridDim.x * blockDim.x)
            dtable[i] = (int32_t)i;
    const int oct = hd / 8;
    const int64_t n = (int64_t)kvh * q.len * oct;
    for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < n;
         gid += (int64_t)gridDim.x * blockDim.x) {
        const int o = (int)(gid % oct);
        const int64_t ht = gid / oct;
        const int h = (int)(ht / q.len), t = (int)(ht - (int64_t)h * q.len);
        // flat D-row rho = h*T + t lies in append c: r_c*KVH <= rho < (r_c + S_c)*KVH
        const int64_t rho = (int64_t)h * q.len + t;
        int lo = 0, hi = q.n_chunks - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((int64_t)chunks[q.chunk0 + mid].x * kvh <= rho)
                lo = mid;
            else
                hi = mid - 1;
        }
        const int2 ck = chunks[q.chunk0 + lo];
        const int64_t off = rho - (int64_t)ck.x * kvh;
        const int hs = (int)(off / ck.y);
        const int ts = ck.x + (int)(off - (int64_t)hs * ck.y);
        const int sp = table[q.src_tab + ts / P], ss = ts % P;
        const int dpg = q.dst_page0 + t / P, ds = t % P;
        const int d0 = o * 8;
        *(u32x4 *)(dk + ((int64_t)dpg * kvh + h) * P * hd + k_page_off(ds, d0, hd)) =
            *(const u32x4 *)(kpool + ((int64_t)sp * kvh + hs) * P * hd + k_page_off(ss, d0, hd));
#pragma unroll
        for (int i = 0; i < 8; i++)
            dv[(((int64_t)dpg * kvh + h) * hd + d0 + i) * P + ds] =
                vpool[(((int64_t)sp * kvh + hs) * hd + d0 + i) * P + ss];
    }
}

hipError_t launch_ref_image_gather(hipStream_t s, const uint16_t *kpool, const uint16_t *vpool,
                                   const int32_t *table, const RefImgSeq *seqs, int n_seqs,
                                   int max_len, const int2 *chunks, int kvh, int hd, int P,
                                   uint16_t *dk, uint16_t *dv, int32_t *dtable, int n_pages) {
    if (n_seqs <= 0) return hipSuccess;
    const int64_t work = std::max<int64_t>((int64_t)kvh * max_len * (hd / 8), n_pages);
    const int blocks = (int)std::min<int64_t>((work + 255) / 256, 4096);
    ref_image_gather_kernel<<<dim3(blocks, n_seqs), 256, 0, s>>>(kpool, vpool, table, seqs, chunks, kvh,
                                                                 hd, P, dk, dv, dtable, n_pages);
    return hipGetLastError();
}

// Paged gather of MLA rows into dense c [T][d_c] and kr [T][d_r] (the
// stored rows' zero padding dropped).  Thread = (token, 8-element chunk of
// the stored row).
__global__ void mla_gather_kernel(const uint16_t *__restrict__ pool,
                                  const int32_t *__restrict__ table,
                                  const AttRow *__restrict__ rows, uint16_t *__restrict__ c_out,
                                  uint16_t *__restrict__ kr_out, int dc, int dr, int P) {
    const AttRow R = rows[blockIdx.y];
    constexpr int chunks = kMlaRow / 8;
    const int64_t n = (int64_t)R.len * chunks;
    for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < n;
         gid += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(gid / chunks);
        const int ch = (int)(gid - (int64_t)t * chunks);
        const bool lat = ch < kMlaDc / 8;
        const int width = lat ? dc : dr;
        const int e0 = lat ? ch * 8 : (ch - kMlaDc / 8) * 8;
        if (e0 >= width) continue;  // padding only
        const int page = table[R.tab + t / P];
        const u32x4 v = *(const u32x4 *)(pool + ((int64_t)page * P + t % P) * kMlaRow + ch * 8);
        const int64_t row = (int64_t)R.qrow + t;
        uint16_t *dst = (lat ? c_out : kr_out) + row * width + e0;
        if (e0 + 8 <= width && width % 8 == 0) {
            *(u32x4 *)dst = v;
        } else {
            for (int i = 0; i < 8 && e0 + i < width; i++)
                dst[i] = (uint16_t)((i & 1) ? (v[i >> 1] >> 16) : (v[i >> 1] & 0xFFFFu));
        }
    }
}

hipError_t launch_mla_gather(hipStream_t s, const uint16_t *pool, const int32_t *table,
                             const AttRow *rows, int n_rows, int max_len, uint16_t *c_out,
                             uint16_t *kr_out, int dc, int dr, int P) {
    if (n_rows <= 0 || max_len <= 0) return hipSuccess;
    int64_t work = (int64_t)max_len * (kMlaRow / 8);
    int blocks = (int)((work + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    mla_gather_kernel<<<dim3(blocks, n_rows), 256, 0, s>>>(pool, table, rows, c_out, kr_out, dc, dr, P);
    return hipGetLastError();
}

}  // namespace rlx
