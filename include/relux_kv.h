/*
 * relux_kv.h -- C ABI of the MI355X (gfx950) KV-cache hot path for relux.
 *
 * One shared library, librelux_kv.so, exports these entry points.  They
 * replace the cache objects and the cached-attention loops of relux's
 * internal/transformer package; a Go host binds them with purego (no CGO),
 * see INTEGRATION.md.  Plain C types only: int32/int64/float, void* for
 * opaque handles and device buffers, int32* for small host arrays.  No
 * struct is passed by value.
 *
 * Conventions
 *   - Every entry returns int32: RLX_OK (0) or a negative RLX_ERR_* code;
 *     rlx_last_error() copies the message of the calling thread's last
 *     failure.
 *   - Bulk tensors (K/V/latent sources, queries, outputs, weights) are
 *     DEVICE pointers (from rlx_dev_alloc or any HIP allocation).  Small
 *     metadata (sequence ids, token counts, dumps) are HOST pointers.
 *   - A cache handle owns one in-order HIP stream; calls on a handle are
 *     asynchronous on that stream unless they return host data (lengths,
 *     tables, free lists), which synchronise.  rlx_cache_sync() waits.
 *     Calls on one handle must be serialised by the caller (the reference
 *     modules are not goroutine-safe either, module.go:62-63).
 *   - bf16 storage uses the reference's integer round-to-nearest-even
 *     conversion (dtype_convert.go:15-24), bit for bit.
 */
#ifndef RELUX_KV_H
#define RELUX_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define RLX_OK 0
#define RLX_ERR_INVALID -1     /* bad argument / shape                     */
#define RLX_ERR_OVERFLOW -2    /* capacity exceeded: the reference panics,
                                  kvcache.go:282-285, mla_cache.go:164-167 */
#define RLX_ERR_POOL -3        /* page pool exhausted                      */
#define RLX_ERR_LAYER -4       /* layer index out of range: the reference
                                  panics, kvcache.go:241-243               */
#define RLX_ERR_HIP -5         /* HIP runtime failure                      */
#define RLX_ERR_UNSUPPORTED -6 /* shape outside the compiled kernel set    */
#define RLX_ERR_STATE -7       /* rollback/evict beyond what is stored     */

/* ---- element types and layouts --------------------------------------- */
#define RLX_F32 0
#define RLX_BF16 1

/* Row layout of multi-sequence K/V sources and of queries/outputs.  A call
 * names n_seqs sequences; sequence i contributes n[i] rows, concatenated in
 * call order.
 *   RLX_LAYOUT_HSD: per sequence [heads][n][dim] -- the reference's
 *                   post-rearrange tensors (rearrangeBSNH, mha.go:789-803).
 *   RLX_LAYOUT_SHD: per sequence [n][heads][dim] -- projection output order. */
#define RLX_LAYOUT_HSD 0
#define RLX_LAYOUT_SHD 1

/* Attention mask for a call with n_q query rows on a sequence holding T
 * live tokens (the queries are the last n_q tokens appended).
 *   RLX_MASK_CAUSAL: query i attends keys j <= T - n_q + i.
 *   RLX_MASK_REF:    the reference's rule: mask j > i only when n_q == T,
 *                    else attend everything (mha.go:337-342, mla.go:365-370).
 *   RLX_MASK_NONE:   attend every live key. */
#define RLX_MASK_CAUSAL 0
#define RLX_MASK_REF 1
#define RLX_MASK_NONE 2

/* RoPE position rule of rlx_gqa_project_append:
 *   RLX_ROPE_OFFSET: token j of a sequence at absolute position
 *                    pos_offset + live_len + j (eviction keeps positions);
 *   RLX_ROPE_REF:    the reference's Apply(x, cacheLen): every row at
 *                    cacheLen when cacheLen > 0, else row j at j
 *                    (rope.go:151-158);
 *   RLX_ROPE_NONE:   no rotation. */
#define RLX_ROPE_OFFSET 0
#define RLX_ROPE_REF 1
#define RLX_ROPE_NONE 2

/* ---- runtime ---------------------------------------------------------- */
/* Select the device for this thread; must be a gfx950 GPU.  Replaces the
 * rnxa engine bring-up the ladder does (internal/compute/factory.go:32-85). */
int32_t rlx_init(int32_t device);
int32_t rlx_last_error(char *buf, int64_t len);
/* Library version string into buf. */
int32_t rlx_version(char *buf, int64_t len);

/* Device buffers for a host without a HIP binding of its own.  Replaces
 * the host-side staging the rnxa MatMulFloat32 path performs
 * (internal/compute/rnxa.go:219-227). */
int32_t rlx_dev_alloc(int64_t bytes, void **out);
int32_t rlx_dev_free(void *ptr);
int32_t rlx_h2d(void *dst, const void *src, int64_t bytes);
int32_t rlx_d2h(void *dst, const void *src, int64_t bytes);
int32_t rlx_device_sync(void);

/* ---- instrumentation (no reference counterpart) ----------------------- */
/* enable is a mask: RLX_TIME_ATTEND brackets the main attention kernel of
 * every later attend call on this handle with HIP events (on the handle's
 * stream), RLX_TIME_PROJECT every projection kernel of
 * rlx_gqa_project_append / rlx_mla_project_append, RLX_TIME_SELECT the
 * kernel of rlx_greedy / rlx_sample / rlx_spec_accept, RLX_TIME_COPY the
 * page copies of rlx_spill / rlx_restore (one interval per call); 0
 * disables.  Either way the recorded intervals are discarded. */
#define RLX_TIME_ATTEND 1
#define RLX_TIME_PROJECT 2
#define RLX_TIME_SELECT 4
#define RLX_TIME_COPY 8
int32_t rlx_cache_timing(void *cache, int32_t enable);
/* Synchronise, then report the summed duration (ms) and number of the
 * timed kernel launches recorded since the last call, and clear them. */
int32_t rlx_cache_kernel_time(void *cache, float *total_ms, int32_t *count);

/* ---- cache lifetime --------------------------------------------------- */
/* Paged bf16 GQA K/V cache for `layers` layers.  Replaces
 * NewKVCacheSized(numLayers, maxLen, numKVHeads, headDim, BFloat16)
 * (kvcache.go:66-93): capacity per sequence is max_pages_per_seq *
 * page_tokens tokens; pool_pages pages per layer are shared by up to
 * max_seqs sequences.  head_dim 1 to 256 (pages store 16, 32, 64, 96, 128
 * or 256 dims, the caller's zero padded; a head_dim that is not a multiple
 * of 8 -- the reference's tests use 2 and 4 -- crosses every call padded
 * to the next multiple of 8 through a per-handle adapter buffer, and
 * rlx_gqa_attend_noalloc / rlx_gqa_project_append refuse it with
 * RLX_ERR_UNSUPPORTED); page_tokens a multiple of 16. */
int32_t rlx_kv_create(int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t page_tokens,
                      int32_t pool_pages, int32_t max_seqs, int32_t max_pages_per_seq, void **out);

/* Paged bf16 MLA latent cache: per token the latent c^KV (d_c) and the
 * post-RoPE k^R (d_r).  Replaces NewMLACache(numLayers, maxLen, dC, dHR)
 * (mla_cache.go:38-59), whose f32 storage becomes bf16 here.
 * d_c <= 512 and even d_r <= 64 (rows stored as 512 + 64 elements, zero
 * padded; the reference's defaults 4*head_dim and head_dim/2 for head_dim
 * <= 128, and the DeepSeek-V2/V3 shapes 512 / 64). */
int32_t rlx_mla_create(int32_t layers, int32_t d_c, int32_t d_r, int32_t page_tokens,
                       int32_t pool_pages, int32_t max_seqs, int32_t max_pages_per_seq, void **out);

int32_t rlx_cache_destroy(void *cache);
/* Drop every sequence and return all pages.  Replaces KVCache.Reset /
 * MLACache.Reset (kvcache.go:174-202, mla_cache.go:118-133); stored bytes
 * are not cleared (the length is what makes them invisible). */
int32_t rlx_cache_reset(void *cache);
int32_t rlx_cache_sync(void *cache);
/* Use `stream` (a hipStream_t, default priority) for this handle's work
 * instead of its own stream; NULL selects the device's null stream (the
 * default stream of a framework such as torch).  Pending work on the old
 * stream is waited for first. */
int32_t rlx_cache_set_stream(void *cache, void *stream);
/* Device scratch, grown ahead of time.  The attention, prefill and
 * token-selection calls take their scratch (split partials, expanded
 * latents, staged plans) from a per-handle workspace, and calls whose
 * plans do not fit the kernel arguments stage them through 8 upload slots
 * (pinned host + device); a call that needs more than either holds grows it
 * on the spot (stream sync, hipFree, hipMalloc inside that call).  This
 * grows the workspace to at least workspace_bytes, every staging slot to
 * at least staging_bytes and the adapter buffer (rows of a head_dim, d_model
 * or k_in that the kernels take padded) to at least adapter_bytes now, so
 * that a serving loop pays for it once at set-up; a size the current
 * capacity covers leaves it unchanged.  No reference counterpart: the
 * reference's scratch is Go heap memory. */
int32_t rlx_cache_reserve(void *cache, uint64_t workspace_bytes, uint64_t staging_bytes,
                          uint64_t adapter_bytes);
/* out[0] workspace capacity, out[1] the largest workspace any call on the
 * handle has asked for, out[2] the smallest staging slot's capacity, out[3]
 * the largest plan any call has staged, out[4] adapter capacity, out[5] the
 * largest adapter request (bytes).  A trial run of the largest calls
 * followed by rlx_cache_reserve(out[1], out[3], out[5]) on a fresh handle
 * keeps every later call of those sizes from allocating. */
int32_t rlx_cache_memory(void *cache, uint64_t *out);

/* ---- append (scatter into pages) -------------------------------------- */
/* Append n_tok[i] tokens to sequence seq_ids[i] of `layer`, converting to
 * bf16 with BF16FromF32.  k_src/v_src hold the rows of all n_seqs
 * sequences in `src_layout` ([kv_heads][n][head_dim] or [n][kv_heads][...]).
 * Replaces KVCache.Append + copyInto (kvcache.go:240-316, 407-438) for a
 * batch of sequences; pages are taken from the layer's LIFO free list as
 * page boundaries are crossed.  Fails without changing state on overflow
 * (RLX_ERR_OVERFLOW) or pool exhaustion (RLX_ERR_POOL). */
int32_t rlx_kv_append(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                      const int32_t *n_tok, const void *k_src, const void *v_src,
                      int32_t src_dtype, int32_t src_layout);

/* ---- fused pre-attention step (projection + RoPE + append) ------------- */
/* Pack a GQA layer's W_q [d_model][H*D], W_k and W_v [d_model][KVH*D] (the
 * reference's in-row/out-col layout, mha.go:84-100, bf16 or f32) into the
 * bf16 layout rlx_gqa_project_append streams: N = (H + 2*KVH)*W output
 * features (q heads, then k heads, then v heads, W each: W = D when H*D and
 * KVH*D are multiples of 16, else D rounded up to 16 with zero weights past
 * D); element (n, k) at
 * ((n/16 * K/32 + k/32) * 16 + n%16) * 32 + k%32 of out (N * K bf16, K =
 * d_model rounded up to 32 with zero rows; the projection then copies x rows
 * of a d_model that is not a multiple of 32 to that width through the
 * handle's adapter buffer).  Runs on the null stream.  No reference counterpart: a one-time
 * weight preparation. */
int32_t rlx_pack_qkv(const void *w_q, const void *w_k, const void *w_v, int32_t w_dtype,
                     int32_t d_model, int32_t num_heads, int32_t kv_heads, int32_t head_dim,
                     void *out);
/* q = x.W_q, k = x.W_k, v = x.W_v for the n_tok[i] new tokens of each
 * sequence (x [sum n][d_model], f32 or bf16), RoPE of q and k with the
 * caller's tables rope_cos/rope_sin [rope_rows][head_dim/2] (f32, device) at
 * the positions rope_mode selects, then the paged append of k and v (bf16
 * round-to-nearest-even); q_out [sum n][num_heads][head_dim] receives the
 * rotated queries for rlx_gqa_attend.  head_dim is the cache's (its pages
 * may store it padded: the padding of the new rows is written with zeros);
 * any even head_dim (RoPE rotates pairs; an odd one fails with
 * RLX_ERR_UNSUPPORTED), with weights packed by rlx_pack_qkv for the same
 * heads.  Replaces mha.go:250-289
 * (matmulBatched3D x3, rearrange, RotaryEmbedding.Apply, KVCache.Append).
 * Projections run on MFMA (bf16 operands, f32 sums): results match the
 * reference's f32 loops within tolerance, not bit for bit.  A position at
 * or past rope_rows fails with RLX_ERR_OVERFLOW (the reference panics). */
int32_t rlx_gqa_project_append(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_tok, const void *x, int32_t x_dtype,
                               int32_t d_model, const void *w_packed, int32_t num_heads,
                               const float *rope_cos, const float *rope_sin, int32_t rope_rows,
                               int32_t rope_mode, void *q_out, int32_t q_dtype);

/* MLA layer: pack W_Q [d_model][H*D], W_QR [d_model][H*d_r], W_DKV
 * [d_model][d_c] and W_KR [d_model][d_r] (mla.go:39-44, bf16 or f32) into
 * out (N = H*(D + d_r') + d_c' + d_r' features, d_r' and d_c' = d_r and
 * d_c rounded up to 16 with zero columns, the same fragment layout as
 * rlx_pack_qkv) for rlx_mla_project_append on a cache of these d_c / d_r.
 * q_c heads are packed head_dim features wide, or rounded up to 16 (zero
 * columns) when H*head_dim is not a multiple of 16; d_model padded as for
 * rlx_pack_qkv.  Null stream.  No reference
 * counterpart: a one-time weight preparation. */
int32_t rlx_pack_mla_proj(const void *w_q, const void *w_qr, const void *w_dkv, const void *w_kr,
                          int32_t w_dtype, int32_t d_model, int32_t num_heads, int32_t head_dim,
                          int32_t d_c, int32_t d_r, void *out);
/* q_c = x.W_Q -> q_nope_out [sum n][H][head_dim]; q_r = RoPE(x.W_QR) ->
 * q_rope_out [sum n][H][d_r]; c = x.W_DKV and k^R = RoPE(x.W_KR) appended
 * as the tokens' latent rows (bf16), zero padded past the cache's d_c and
 * d_r.  Tables [rope_rows][d_r/2] (f32, device), positions as for
 * rlx_gqa_project_append.  The q outputs are the
 * inputs of rlx_mla_attend.  Replaces mla.go:279-314 (four
 * matmulBatched3D, RotaryEmbedding.Apply of q^R and k^R, MLACache.Append);
 * within tolerance of the reference's f32 loops, not bit for bit. */
int32_t rlx_mla_project_append(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_tok, const void *x, int32_t x_dtype,
                               int32_t d_model, const void *w_packed, int32_t num_heads,
                               int32_t head_dim, const float *rope_cos, const float *rope_sin,
                               int32_t rope_rows, int32_t rope_mode, void *q_nope_out,
                               void *q_rope_out, int32_t q_dtype);

/* The step after attention: out[r] = x[r] . W (+ residual[r]) for `rows`
 * rows -- the output projection (mha.go:356-360 W_O, x = the attention
 * output [rows][H*D]; mla.go:384-389) and the transformer block's residual
 * add (transformer_block.go:119-142), which the reference runs on the host.
 * W [k_in][n_out] (the reference's in-row/out-col layout, bf16 or f32) is
 * packed once by rlx_pack_out into n_out' * k_in' bf16 (n_out' = n_out
 * rounded up to 16, k_in' = k_in rounded up to 32, zero weights in the
 * padding; x rows of a k_in that is not a multiple of 32 are copied to the
 * padded width through the handle's adapter buffer).  x: device
 * [rows][k_in] (RLX_F32 / RLX_BF16; f32 rows are
 * used at f32 precision); residual: NULL or device [rows][n_out] in
 * out_dtype; out: device [rows][n_out].  Runs on cache's stream. */
int32_t rlx_pack_out(const void *w, int32_t w_dtype, int32_t k_in, int32_t n_out, void *out);
int32_t rlx_out_project(void *cache, int32_t rows, const void *x, int32_t x_dtype, int32_t k_in,
                        const void *w_packed, int32_t n_out, const void *residual, void *out,
                        int32_t out_dtype);

/* MLA: c_src [sum n][d_c], kr_src [sum n][d_r] (post-RoPE).  Replaces
 * MLACache.Append (mla_cache.go:152-182). */
int32_t rlx_mla_append(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_tok, const void *c_src, const void *kr_src,
                       int32_t src_dtype);

/* ---- paged gather (View) ---------------------------------------------- */
/* Copy the live tokens of each listed sequence through the page table into
 * dense bf16 device buffers: k_out/v_out per sequence [kv_heads][T][head_dim]
 * (the shape View returns, kvcache.go:363-380), concatenated in call order. */
int32_t rlx_kv_gather(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                      void *k_out, void *v_out);
/* MLA: c_out [T][d_c], kr_out [T][d_r] per sequence (mla_cache.go:222-233). */
int32_t rlx_mla_gather(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       void *c_out, void *kr_out);

/* ---- attention over the cache ----------------------------------------- */
/* GQA flash-decoding / verify / chunked prefill over the paged cache for
 * n_seqs sequences with n_q[i] query rows each.  q and out: [rows of all
 * sequences] in qo_layout with num_heads heads of head_dim; head h reads
 * KV head h / (num_heads / kv_heads).  scale <= 0 selects 1/sqrt(head_dim).
 * Replaces mha.go:291-348 (View, widen, GQA expand, score/softmax/PV
 * loops).  Exact exp softmax with f32 accumulation; the reference's
 * fastexp32 weights are matched within tolerance, not bit for bit. */
int32_t rlx_gqa_attend(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                       int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                       int32_t out_dtype);

/* rlx_gqa_attend reading the keys and values as the reference KVCache
 * holds them: each Append copies its [KVH, S, D] block raw into the next S
 * rows of a [cap][KVH*D] buffer (kvcache.go:286-287, copyInto 407-423) and
 * MHA.forwardCached reads head h at token t from flat row h*T + t
 * (mha.go:305-310) -- for KVH > 1 a permutation of the logical rows, which
 * this call reproduces from the sequence's append history (relux's own
 * decode outputs; RLX_MASK_REF gives its mask rule too).  Sequences whose
 * tokens are no longer exactly their appends' (evicted, or a rollback that
 * cut an append in two) give RLX_ERR_STATE.  Same arguments as
 * rlx_gqa_attend; at most 32 query rows per kv head per work-group (larger
 * calls are tiled), no FA2 path. */
int32_t rlx_gqa_attend_ref_image(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                                 const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                                 int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                                 int32_t out_dtype);
/* The cache half of MHA.forwardCached in one call: append the n_tok[i] >= 1
 * new tokens' K and V rows (k_src / v_src, src_dtype and src_layout as for
 * rlx_kv_append), then the attention of those tokens (n_q = n_tok) as
 * rlx_gqa_attend.  Replaces mha.go:283-348 (KVCache.Append, View, widen,
 * expand, attention) with one call, the counterpart of
 * rlx_mla_append_attend; it launches the append and then the attention, so
 * cache contents and outputs are those of the two calls, bit for bit.
 * Every argument is checked before anything is appended. */
int32_t rlx_gqa_append_attend(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                              const int32_t *n_tok, const void *k_src, const void *v_src,
                              int32_t src_dtype, int32_t src_layout, int32_t num_heads,
                              const void *q, int32_t q_dtype, int32_t qo_layout, float scale,
                              int32_t mask_mode, void *out, int32_t out_dtype);
/* rlx_gqa_attend for decode and verify calls, allocating nothing: no
 * reference counterpart.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as rlx_gqa_attend; the
 * split partials go to a fixed 32 MiB scratch array per device (held until
 * the process ends) instead of the cache's workspace, pending page-table
 * writes travel in kernel arguments, and no staging buffer is used.  Limits
 * (RLX_ERR_UNSUPPORTED beyond them, nothing launched): at most 32 query rows
 * per kv head, at most 64 rows (sequences, or query tiles of head_dim 16/32
 * calls), partials within the scratch, a head_dim that is a multiple of 8
 * (others would need adapter memory).  rlx_init(device) must have run.
 * Every call on a device shares its scratch: calls that overlap on one
 * device (different streams) race. */
int32_t rlx_gqa_attend_noalloc(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_q, int32_t num_heads, const void *q,
                               int32_t q_dtype, int32_t qo_layout, float scale, int32_t mask_mode,
                               void *out, int32_t out_dtype);

/* MLA absorbed decode / chunked prefill.  q_nope [rows][num_heads][head_dim],
 * q_rope [rows][num_heads][d_r] (post-RoPE), w_uk and w_uv bf16
 * [d_c][num_heads*head_dim] exactly as MLA.W_UK/W_UV are stored (mla.go:42-43),
 * out [rows][num_heads][head_dim].  Computes the same attention as
 * mla.go:316-377 (decompress-all) by absorbing W_UK into the query and
 * W_UV into the output.  scale <= 0 selects 1/sqrt(head_dim + d_r).
 * head_dim 1 to 256; one that is not a multiple of 8 crosses padded with
 * zero dims (q_nope, w_uk, w_uv copied into the handle's adapter buffer,
 * out copied back). */
int32_t rlx_mla_attend(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_q, int32_t num_heads, int32_t head_dim, const void *q_nope,
                       const void *q_rope, int32_t q_dtype, const void *w_uk, const void *w_uv,
                       float scale, int32_t mask_mode, void *out, int32_t out_dtype);
/* The cache half of MLA.forwardCached in one call: append the n_tok[i] >= 1
 * new tokens' latent rows (c_src / kr_src as for rlx_mla_append), then the
 * attention of those tokens (n_q = n_tok) as rlx_mla_attend.  Replaces
 * mla.go:308-377 (MLACache.Append, View, decompress, attention).  Same
 * cache contents and outputs as the two calls in sequence, bit for bit; on
 * the decode path the append runs inside the attention's first launch (one
 * launch fewer per step).  Every argument is checked before anything is
 * appended, including the size of a prefill's expansion.  A resource
 * failure after that (workspace allocation, staging) still appends the
 * tokens -- host state and device table agree, as after rlx_mla_append --
 * and returns the error without attention outputs. */
int32_t rlx_mla_append_attend(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                              const int32_t *n_tok, const void *c_src, const void *kr_src,
                              int32_t src_dtype, int32_t num_heads, int32_t head_dim,
                              const void *q_nope, const void *q_rope, int32_t q_dtype,
                              const void *w_uk, const void *w_uv, float scale, int32_t mask_mode,
                              void *out, int32_t out_dtype);

/* ---- speculative rollback, eviction, compaction (no reference) -------- */
/* Remove the last n_tokens[i] tokens of sequence seq_ids[i], in list order
 * (layer -1: every layer).  Pages left empty return to the free list, last
 * page first, so that append(a||b); rollback(|b|) leaves exactly the state
 * of append(a).  Validated in full before any change.  The reference never
 * truncates its caches (speculative.go:146-156); this is the rejected-draft
 * rollback its SpeculativeDecoder.Generate loop (speculative.go:131-156)
 * needs after acceptPhase. */
int32_t rlx_rollback(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                     const int32_t *n_tokens);
/* Drop the oldest n_pages[i] full pages of sequence seq_ids[i] (layer -1:
 * every layer); their tokens leave attention, the RoPE position of later
 * tokens is kept (pos_offset grows by n_pages*page_tokens).  Freed pages are
 * pushed oldest first.  No reference counterpart. */
int32_t rlx_evict(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                  const int32_t *n_pages);
/* Rewrite page-table rows so live pages start at entry 0, logical order
 * kept; K/V bytes do not move (layer -1: every layer). */
int32_t rlx_compact(void *cache, int32_t layer);
/* Free every page of one sequence, spilled pages included (layer -1: every
 * layer). */
int32_t rlx_seq_release(void *cache, int32_t layer, int32_t seq);

/* ---- host spill tier (no reference counterpart) ----------------------- */
/* The reference's file-backed caches (NewKVCacheFile, kvcache.go:95-166;
 * the MLA variant, mla_cache.go:61-113) keep the whole cache in a file
 * mapped MAP_SHARED.  Here the file (or pinned host memory) is a second
 * tier below the HBM pool: pages spilled to it leave attention exactly as
 * evicted pages do, and can be put back in front of their sequence.
 *
 * Attach a tier of host_pages slots, one layer's page each (GQA: the K page
 * then the V page of every kv head, as stored in HBM; MLA: the latent
 * rows); slot bytes and counts via rlx_spill_info.  path NULL or "":
 * pinned host memory; otherwise the file is created or truncated to size
 * and mapped MAP_SHARED -- the caller owns the file (it is not deleted).
 * host_pages 0 detaches.  Fails while the tier holds pages. */
int32_t rlx_spill_attach(void *cache, const char *path, int64_t host_pages);
/* Move the oldest n_pages[i] full pages of sequence seq_ids[i] (layer -1:
 * every layer) to the tier: the device state afterwards is exactly that of
 * rlx_evict with the same arguments (pages pushed oldest first, first and
 * pos_offset advance).  Slots are taken 0, 1, 2, ... from a LIFO free list.
 * With a file tier the bytes are in the file when the call returns.
 * RLX_ERR_POOL when the tier has too few free slots (no change). */
int32_t rlx_spill(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                  const int32_t *n_pages);
/* Put the n_pages[i] most recently spilled pages of sequence seq_ids[i]
 * back in front of it (layer -1: every layer): newest spilled page first,
 * each into a page popped from the free list; len grows and pos_offset
 * shrinks by n_pages*page_tokens, so the sequence's bytes and positions
 * are those before the spill.  Live table entries move right when fewer
 * than n_pages entries precede them.  A later rlx_evict of the sequence
 * drops its spilled pages too (they would no longer adjoin its resident
 * tokens).  RLX_ERR_STATE / RLX_ERR_POOL / RLX_ERR_OVERFLOW, no change. */
int32_t rlx_restore(void *cache, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                    const int32_t *n_pages);
/* Tier slots holding (layer, seq)'s spilled pages, oldest first (at most
 * cap written); *n_out = their count. */
int32_t rlx_spill_slots(void *cache, int32_t layer, int32_t seq, int64_t *slots_out, int32_t cap,
                        int32_t *n_out);
/* info[0..3] = slots, bytes per slot, free slots, 1 if file-backed. */
int32_t rlx_spill_info(void *cache, int64_t *info);

/* ---- token selection on the device (synchronising) -------------------- */
/* Sampler fields (sampler.go:33-43) except Rand: every rng.Float32() draw
 * is passed in.  NewSampler's defaults are temperature 1, top_p 1, the
 * rest 0.  Clamps as the reference: temperature <= 0 -> 1e-5, top_k < 0 or
 * >= vocab -> off, top_p outside (0, 1) -> off. */
typedef struct {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float repeat_penalty;
    float frequency_penalty;
    float presence_penalty;
    int32_t repeat_window;
} rlx_sampler_t;

/* The calls below run on `cache`'s stream (any GQA or MLA handle) and copy
 * their small results to host memory before returning.  logits are DEVICE
 * f32 rows (row_stride elements apart); every other array is host memory. */

/* Sampler.Greedy (sampler.go:56-68) per row: first index of the maximum. */
int32_t rlx_greedy(void *cache, const float *logits, int32_t n_rows, int32_t vocab,
                   int64_t row_stride, int32_t *out_tokens);
/* Sampler.Sample (sampler.go:73-210) per row: penalties over the row's
 * previous tokens prev_tokens[prev_offsets[r] .. prev_offsets[r+1]) (both
 * may be NULL: no penalties; with penalties, vocab <= 262144 and at most
 * 4096 distinct tokens per window), temperature, top-k, fastexp32 softmax,
 * top-p, min-p, then the draw uniforms[r].  Sums are block-parallel, so a
 * draw within a few ulp of a cumulative boundary may land one token over;
 * top-p keeps every token tied with the cutoff probability. */
int32_t rlx_sample(void *cache, const float *logits, int32_t n_rows, int32_t vocab,
                   int64_t row_stride, const rlx_sampler_t *params, const int32_t *prev_tokens,
                   const int32_t *prev_offsets, const float *uniforms, int32_t *out_tokens);
/* Sampler.Sample (sampler.go:73-262) over device-resident state, for a
 * decode loop whose tokens never leave the GPU: the stages of rlx_sample,
 * with each row's repetition window counted on the device from a token
 * history.  Row b's history is history[b * hist_stride .. + hist_len[b])
 * (device int32; hist_len device int32 [n_rows], clamped to
 * [0, hist_stride]); its window is the last repeat_window entries (all of
 * them when repeat_window <= 0), and the longest possible window,
 * min(repeat_window, hist_stride) or hist_stride, must be at most 4096
 * (RLX_ERR_UNSUPPORTED otherwise).  history NULL: no penalties.  uniforms
 * (the rng.Float32() draws) are device f32 [n_rows]; out_tokens device
 * int32 [n_rows].  Enqueued on the cache's stream: nothing is copied to or
 * from the host and the call does not wait -- except the first call that
 * needs a larger cache workspace (the split path's chunk lists, top-k in
 * (0, 256] past 8192 entries), which synchronises the stream and
 * allocates it once.  Same tokens as rlx_sample given the same windows
 * and draws. */
int32_t rlx_sample_async(void *cache, const float *logits, int32_t n_rows, int32_t vocab,
                         int64_t row_stride, const rlx_sampler_t *params, const int32_t *history,
                         int64_t hist_stride, const int32_t *hist_len, const float *uniforms,
                         int32_t *out_tokens);
/* SpeculativeDecoder.acceptPhase + resampleRejected (speculative.go:203-290)
 * for n_rows sequences at once.  draft_logits [n_rows][max_k][vocab] and
 * target_logits [n_rows][max_k+1][vocab] (device f32; target row i scores
 * draft i, row n_draft the token after the last draft); draft_tokens
 * [n_rows][max_k], n_draft [n_rows] (<= max_k); uniforms [n_rows][max_k+1],
 * consumed in the reference's order: one acceptance test per draft up to
 * the first rejection, then one draw for the resample (or, all accepted,
 * for Sample over the next target row with `params`, no penalties).
 * Outputs per row: accepted drafts and the next token.  The caller then
 * rolls its caches back (rlx_rollback) to the committed prefix. */
int32_t rlx_spec_accept(void *cache, const float *draft_logits, const float *target_logits,
                        const int32_t *draft_tokens, const int32_t *n_draft, int32_t n_rows,
                        int32_t max_k, int32_t vocab, const float *uniforms,
                        const rlx_sampler_t *params, int32_t *n_accepted, int32_t *next_token);
/* rlx_spec_accept over device-resident state, for a speculative loop whose
 * drafts and tokens never leave the GPU: draft_tokens [n_rows][max_k],
 * n_draft [n_rows] and uniforms [n_rows][max_k+1] are device arrays, and
 * n_accepted / next_token [n_rows] device int32 outputs.  The draft counts
 * and ids are not seen by the host: a count is clamped to [0, max_k] and
 * an id outside [0, vocab) is treated as a rejection at its position.
 * Enqueued on the cache's stream; nothing is copied and the call does not
 * wait -- except the first call that needs a larger cache workspace (the
 * per-draft figures and chunk sums), which synchronises the stream and
 * allocates it once.  Same results as rlx_spec_accept on valid inputs. */
int32_t rlx_spec_accept_async(void *cache, const float *draft_logits, const float *target_logits,
                              const int32_t *draft_tokens, const int32_t *n_draft, int32_t n_rows,
                              int32_t max_k, int32_t vocab, const float *uniforms,
                              const rlx_sampler_t *params, int32_t *n_accepted, int32_t *next_token);

/* ---- state queries (synchronising) ------------------------------------ */
/* Live token count; replaces TotalLen (kvcache.go:383-388). */
int32_t rlx_seq_len(void *cache, int32_t layer, int32_t seq, int32_t *len_out);
/* {live_len, first_entry, pos_offset, pages_in_use}. */
int32_t rlx_seq_state(void *cache, int32_t layer, int32_t seq, int32_t *state4_out);
/* Copy the DEVICE page-table row (max_pages_per_seq int32, -1 = empty). */
int32_t rlx_page_table(void *cache, int32_t layer, int32_t seq, int32_t *row_out);
/* Copy the layer's free-page stack bottom..top; *n_out = its depth. */
int32_t rlx_free_list(void *cache, int32_t layer, int32_t *out, int32_t cap, int32_t *n_out);
/* Device address of a layer's page pools (for zero-copy inspection). */
int32_t rlx_pool_ptr(void *cache, int32_t layer, void **k_pool, void **v_pool);

#ifdef __cplusplus
}
#endif
#endif /* RELUX_KV_H */
