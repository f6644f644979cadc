// Host runtime and C ABI of librelux_kv: cache handles, page pools, the
// page-table state machine (append / rollback / evict / compact), plan
// staging, and dispatch to the kernels.
//
// State ownership: the host keeps the authoritative integer state of every
// (layer, sequence) -- live length, first live table entry, RoPE position
// offset, pages in use -- plus a mirror of the page table and the LIFO free
// stack of each layer.  The device holds the page pools and the page table
// the kernels read.  Table writes are batched as (index, value) patches,
// coalesced by index, and applied on the stream before the next kernel that
// reads the table (fused into append, or a patch kernel).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/relux_kv.h"
#include "rlx_common.h"

using namespace rlx;

// Scratch of rlx_gqa_attend_noalloc: the split partials of a decode call
// live here instead of in a workspace the library allocates.  One copy per
// device, held until the process ends; every no-alloc call on a device
// shares it, so calls that overlap on one device (different streams) race.
// Host code never uses the array's name as an address: rlx_init looks up
// each device's copy with hipGetSymbolAddress and keeps it in g_scratch.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices];  // per device: address of its `scratch` copy

thread_local std::string g_err;

int32_t fail(int32_t code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail(RLX_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));        \
    } while (0)

enum Kind { kGQA = 0, kMLA = 1 };

struct SeqState {
    int32_t len = 0;         // live tokens
    int32_t first = 0;       // first live entry of the table row
    int32_t pos_offset = 0;  // absolute position of the first live token
    int32_t pages = 0;       // live pages
    // GQA: token counts of the appends, oldest first -- the reference
    // KVCache lays each append's [KVH, S, D] block out raw, so its byte
    // image follows from them.  chunks_ok is cleared by a rollback that
    // cuts an append in two.
    std::vector<int32_t> chunks;
    bool chunks_ok = true;
};

struct LayerState {
    uint16_t *pool0 = nullptr;  // GQA K pages (k-step-major blocks) / MLA latent rows
    uint16_t *pool1 = nullptr;  // GQA V dim-major pages
    std::vector<int32_t> table;       // [max_seqs * max_pages], -1 empty
    std::vector<int32_t> free_stack;  // back() is the next page handed out
    std::vector<SeqState> seqs;
};

struct Slot {
    void *host = nullptr;
    void *dev = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;
    bool pending = false;
};

constexpr int kSlots = 8;

// Host spill tier: slots of one layer's page each, holding the page's bytes
// exactly as stored in HBM (GQA: the K page then the V page of every kv
// head; MLA: the latent rows).  Backed by pinned host memory or by a file
// mapped MAP_SHARED (the reference's file-backed caches, kvcache.go:95-166).
struct SpillTier {
    uint8_t *base = nullptr;      // host address of slot 0
    uint8_t *dev_base = nullptr;  // the same memory as the device addresses it (pinned tier)
    uint8_t *bounce = nullptr;    // file tier: pinned staging the copy kernel reads / writes
    uint8_t *dev_bounce = nullptr;
    int64_t bounce_slots = 0;
    int64_t slots = 0;
    size_t slot_bytes = 0;
    size_t map_bytes = 0;  // non-zero: file mapping
    std::vector<int64_t> free_stack;                   // back() is the next slot handed out
    std::vector<std::vector<std::vector<int64_t>>> held;  // [layer][seq]: slots, oldest page first
};

struct Cache {
    int kind = kGQA;
    int layers = 0, kvh = 0, hd = 0, P = 0, pool_pages = 0, max_seqs = 0, max_pages = 0;
    int hdi = 0;  // GQA: the kernels' caller head dim (hd, the stored one, may be larger: zero padding)
    int hdu = 0;  // GQA: the caller's head dim as given (hdi = hdu rounded up to a multiple of 8)
    int dc = 0, dr = 0;
    int device = 0;
    int cus = 256;  // compute units of the device
    std::vector<LayerState> L;
    int32_t *d_table = nullptr;
    hipStream_t own = nullptr, stream = nullptr;
    std::map<int64_t, int32_t> pending;  // flat table index -> value
    Slot slots[kSlots];
    int next_slot = 0;
    void *ws = nullptr;
    size_t ws_cap = 0;
    size_t ws_peak = 0;     // largest workspace a call asked for
    void *ad = nullptr;     // adapter rows of head dims that are not multiples of 8
    size_t ad_cap = 0;
    size_t ad_peak = 0;     // largest adapter request
    size_t stage_peak = 0;  // largest plan a call staged
    SpillTier spill;
    // Attention-kernel timing: event pairs, reused across reports.
    int timing = 0;  // RLX_TIME_* mask
    std::vector<std::pair<hipEvent_t, hipEvent_t>> tev;
    size_t tev_used = 0;

    int64_t row_base(int layer, int seq) const {
        return ((int64_t)layer * max_seqs + seq) * max_pages;
    }
    void set_entry(int layer, int seq, int k, int32_t v) {
        const int64_t idx = row_base(layer, seq) + k;
        L[layer].table[idx - (int64_t)layer * max_seqs * max_pages] = v;
        pending[idx] = v;
    }
    int32_t entry(int layer, int seq, int k) const {
        return L[layer].table[(int64_t)seq * max_pages + k];
    }
};

// Copy `bytes` of host data into the next staging slot and enqueue its
// upload; returns the device address the kernels should read.
int32_t stage(Cache *c, const void *data, size_t bytes, void **dev_out) {
    Slot &s = c->slots[c->next_slot];
    c->next_slot = (c->next_slot + 1) % kSlots;
    c->stage_peak = std::max(c->stage_peak, bytes);
    if (s.pending) {
        HIP_TRY(hipEventSynchronize(s.ev));
        s.pending = false;
    }
    if (bytes > s.cap) {
        size_t cap = std::max<size_t>(bytes, 64 * 1024);
        cap = (cap + 4095) & ~(size_t)4095;
        // The device copy of this slot may still be read by queued kernels.
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (s.host) HIP_TRY(hipHostFree(s.host));
        if (s.dev) HIP_TRY(hipFree(s.dev));
        s.host = nullptr;
        s.dev = nullptr;
        HIP_TRY(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
        HIP_TRY(hipMalloc(&s.dev, cap));
        s.cap = cap;
    }
    if (bytes) {
        memcpy(s.host, data, bytes);
        HIP_TRY(hipMemcpyAsync(s.dev, s.host, bytes, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(hipEventRecord(s.ev, c->stream));
        s.pending = true;
    }
    *dev_out = s.dev;
    return RLX_OK;
}

// Append plans: patches then tokens (16-byte aligned), in the kernel
// arguments when they fit, else staged.  Fills *plan or the device pointers.
int32_t append_plan(Cache *c, const std::vector<Patch> &patches,
                    const std::vector<AppendTok> &toks, PlanArg *plan_arg, const PlanArg **plan,
                    int *tok_off, const Patch **d_patches, const AppendTok **d_toks) {
    const size_t off = (patches.size() * sizeof(Patch) + 15) & ~(size_t)15;
    *plan = nullptr;
    *d_patches = nullptr;
    *d_toks = nullptr;
    *tok_off = (int)off;
    if (off + toks.size() * sizeof(AppendTok) <= sizeof(PlanArg)) {
        if (!patches.empty()) memcpy(plan_arg->b, patches.data(), patches.size() * sizeof(Patch));
        if (!toks.empty()) memcpy(plan_arg->b + off, toks.data(), toks.size() * sizeof(AppendTok));
        *plan = plan_arg;
        return RLX_OK;
    }
    std::vector<char> bytes(off + toks.size() * sizeof(AppendTok));
    if (!patches.empty()) memcpy(bytes.data(), patches.data(), patches.size() * sizeof(Patch));
    if (!toks.empty()) memcpy(bytes.data() + off, toks.data(), toks.size() * sizeof(AppendTok));
    void *dev;
    int32_t rc = stage(c, bytes.data(), bytes.size(), &dev);
    if (rc) return rc;
    *d_patches = (const Patch *)dev;
    *d_toks = (const AppendTok *)((char *)dev + off);
    return RLX_OK;
}

// Serialise a list of PODs into one byte blob with 16-byte aligned parts.
struct Blob {
    std::vector<char> bytes;
    template <class T>
    size_t add(const std::vector<T> &v) {
        size_t off = (bytes.size() + 15) & ~(size_t)15;
        bytes.resize(off + v.size() * sizeof(T));
        if (!v.empty()) memcpy(bytes.data() + off, v.data(), v.size() * sizeof(T));
        return off;
    }
};

std::vector<Patch> take_pending(Cache *c) {
    std::vector<Patch> p;
    p.reserve(c->pending.size());
    for (auto &kv : c->pending) p.push_back(Patch{(int32_t)kv.first, kv.second});
    c->pending.clear();
    return p;
}

// Apply pending table patches now (before a kernel that reads the table).
int32_t flush_patches(Cache *c) {
    if (c->pending.empty()) return RLX_OK;
    std::vector<Patch> p = take_pending(c);
    Blob b;
    b.add(p);
    void *dev;
    int32_t rc = stage(c, b.bytes.data(), b.bytes.size(), &dev);
    if (rc) return rc;
    HIP_TRY(launch_patch(c->stream, c->d_table, (const Patch *)dev, (int)p.size()));
    return RLX_OK;
}

// Apply pending table patches through the kernel arguments (up to 256 per
// launch): no staging slot, so nothing is allocated.
int32_t flush_patches_inline(Cache *c) {
    constexpr int kPer = kPlanArgBytes / (int)sizeof(Patch);
    while (!c->pending.empty()) {
        PlanArg pa;
        int n = 0;
        auto it = c->pending.begin();
        for (; it != c->pending.end() && n < kPer; ++it, ++n) {
            const Patch p{(int32_t)it->first, it->second};
            memcpy(pa.b + n * sizeof(Patch), &p, sizeof p);
        }
        HIP_TRY(launch_patch_plan(c->stream, c->d_table, pa, n));
        c->pending.erase(c->pending.begin(), it);
    }
    return RLX_OK;
}

int32_t ensure_ws(Cache *c, size_t bytes) {
    c->ws_peak = std::max(c->ws_peak, bytes);
    if (bytes <= c->ws_cap) return RLX_OK;
    // RLX_WS_MAX_KB caps the workspace (tests force the failure path of a
    // call with it; unset or 0: no cap).
    if (const char *lim = getenv("RLX_WS_MAX_KB")) {
        const long long kb = atoll(lim);
        if (kb > 0 && bytes > (size_t)kb << 10)
            return fail(RLX_ERR_HIP, "workspace of %zu bytes exceeds RLX_WS_MAX_KB=%lld", bytes, kb);
    }
    size_t cap = std::max(bytes, c->ws_cap * 2);
    cap = (cap + 65535) & ~(size_t)65535;
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->ws) HIP_TRY(hipFree(c->ws));
    c->ws = nullptr;
    c->ws_cap = 0;
    HIP_TRY(hipMalloc(&c->ws, cap));
    c->ws_cap = cap;
    return RLX_OK;
}

// Caller rows of a head dim that is not a multiple of 8 cross the boundary
// through the handle's adapter buffer: inputs are copied to rows of the next
// multiple of 8 (zero filled: zero dims add nothing to a dot product and
// RoPE pairs (2i, 2i + 1) stay within the caller's dims), the kernels run on
// those, and outputs are copied back at the caller's width.  Regions of
// `bytes[i]` each, 256-byte aligned; growing the buffer waits for the stream
// first (queued kernels may still read the old one).
int32_t adapter_regions(Cache *c, const size_t *bytes, int n, char **out) {
    size_t off[8], total = 0;
    for (int i = 0; i < n; i++) {
        off[i] = total;
        total += (bytes[i] + 255) & ~(size_t)255;
    }
    c->ad_peak = std::max(c->ad_peak, total);
    if (total > c->ad_cap) {
        const size_t cap = (std::max(total, c->ad_cap * 2) + 65535) & ~(size_t)65535;
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (c->ad) HIP_TRY(hipFree(c->ad));
        c->ad = nullptr;
        c->ad_cap = 0;
        HIP_TRY(hipMalloc(&c->ad, cap));
        c->ad_cap = cap;
    }
    for (int i = 0; i < n; i++) out[i] = (char *)c->ad + off[i];
    return RLX_OK;
}

Cache *as_cache(void *h) { return static_cast<Cache *>(h); }

// Next event pair bracketing a kernel of the given kind (RLX_TIME_*), or
// nulls when that kind is not being timed.
int32_t timing_events(Cache *c, hipEvent_t *e0, hipEvent_t *e1, int kind = RLX_TIME_ATTEND) {
    *e0 = *e1 = nullptr;
    if (!(c->timing & kind)) return RLX_OK;
    if (c->tev_used == c->tev.size()) {
        hipEvent_t a, b;
        HIP_TRY(hipEventCreateWithFlags(&a, timing_event_flags()));
        HIP_TRY(hipEventCreateWithFlags(&b, timing_event_flags()));
        c->tev.emplace_back(a, b);
    }
    *e0 = c->tev[c->tev_used].first;
    *e1 = c->tev[c->tev_used].second;
    c->tev_used++;
    return RLX_OK;
}

int32_t check_layer(Cache *c, int layer, bool allow_all) {
    if (allow_all && layer == -1) return RLX_OK;
    if (layer < 0 || layer >= c->layers)
        return fail(RLX_ERR_LAYER, "layerIdx=%d out of range [0, %d)", layer, c->layers);
    return RLX_OK;
}

int32_t check_seqs(Cache *c, int n_seqs, const int32_t *seq_ids) {
    if (n_seqs < 0 || (n_seqs > 0 && !seq_ids)) return fail(RLX_ERR_INVALID, "bad sequence list");
    std::vector<char> seen(c->max_seqs, 0);
    for (int i = 0; i < n_seqs; i++) {
        const int s = seq_ids[i];
        if (s < 0 || s >= c->max_seqs)
            return fail(RLX_ERR_INVALID, "seq id %d out of range [0, %d)", s, c->max_seqs);
        if (seen[s]) return fail(RLX_ERR_INVALID, "seq id %d listed twice in one call", s);
        seen[s] = 1;
    }
    return RLX_OK;
}

void reset_layer_state(Cache *c, LayerState &ls) {
    ls.table.assign((size_t)c->max_seqs * c->max_pages, -1);
    ls.free_stack.resize(c->pool_pages);
    // Pages are handed out 0, 1, 2, ... from a fresh pool.
    for (int i = 0; i < c->pool_pages; i++) ls.free_stack[i] = c->pool_pages - 1 - i;
    ls.seqs.assign(c->max_seqs, SeqState{});
}

int32_t create_common(Cache *c) {
    HIP_TRY(hipGetDevice(&c->device));
    HIP_TRY(hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, c->device));
    HIP_TRY(hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking));
    c->stream = c->own;
    for (auto &s : c->slots) HIP_TRY(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
    const int64_t tab_n = (int64_t)c->layers * c->max_seqs * c->max_pages;
    HIP_TRY(hipMalloc(&c->d_table, tab_n * sizeof(int32_t)));
    HIP_TRY(launch_fill_i32(c->stream, c->d_table, -1, tab_n));
    c->L.resize(c->layers);
    for (auto &ls : c->L) reset_layer_state(c, ls);
    size_t page_bytes = (c->kind == kGQA) ? (size_t)c->kvh * c->P * c->hd * 2 : (size_t)c->P * kMlaRow * 2;
    for (auto &ls : c->L) {
        HIP_TRY(hipMalloc(&ls.pool0, page_bytes * c->pool_pages));
        // Zeroed so that never-written slots hold finite values.
        HIP_TRY(hipMemsetAsync(ls.pool0, 0, page_bytes * c->pool_pages, c->stream));
        if (c->kind == kGQA) {
            HIP_TRY(hipMalloc(&ls.pool1, page_bytes * c->pool_pages));
            HIP_TRY(hipMemsetAsync(ls.pool1, 0, page_bytes * c->pool_pages, c->stream));
        }
    }
    HIP_TRY(hipStreamSynchronize(c->stream));
    return RLX_OK;
}

void destroy_cache(Cache *c) {
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->own) (void)hipStreamSynchronize(c->own);
    for (auto &ls : c->L) {
        if (ls.pool0) (void)hipFree(ls.pool0);
        if (ls.pool1) (void)hipFree(ls.pool1);
    }
    if (c->d_table) (void)hipFree(c->d_table);
    if (c->ws) (void)hipFree(c->ws);
    if (c->ad) (void)hipFree(c->ad);
    for (auto &p : c->tev) {
        (void)hipEventDestroy(p.first);
        (void)hipEventDestroy(p.second);
    }
    for (auto &s : c->slots) {
        if (s.host) (void)hipHostFree(s.host);
        if (s.dev) (void)hipFree(s.dev);
        if (s.ev) (void)hipEventDestroy(s.ev);
    }
    if (c->spill.base) {
        if (c->spill.map_bytes)
            (void)munmap(c->spill.base, c->spill.map_bytes);
        else
            (void)hipHostFree(c->spill.base);
    }
    if (c->spill.bounce) (void)hipHostFree(c->spill.bounce);
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
}

// Give the spilled slots of (layer, seq) back to the tier, newest first.
void release_spilled(Cache *c, int layer, int seq) {
    if (c->spill.held.empty()) return;
    auto &h = c->spill.held[layer][seq];
    for (auto it = h.rbegin(); it != h.rend(); ++it) c->spill.free_stack.push_back(*it);
    h.clear();
}

void reset_spill(Cache *c) {
    SpillTier &t = c->spill;
    if (!t.base) return;
    t.free_stack.resize(t.slots);
    for (int64_t i = 0; i < t.slots; i++) t.free_stack[i] = t.slots - 1 - i;  // slots 0, 1, 2, ...
    t.held.assign(c->layers, std::vector<std::vector<int64_t>>(c->max_seqs));
}

// Bytes of one layer's page in the K (or latent) pool and in the V pool.
size_t page_bytes0(const Cache *c) {
    return (c->kind == kGQA) ? (size_t)c->kvh * c->P * c->hd * 2 : (size_t)c->P * kMlaRow * 2;
}
size_t page_bytes1(const Cache *c) { return (c->kind == kGQA) ? page_bytes0(c) : 0; }

// Plan the page allocations of one append call on one layer.  Validates
// everything first so that a failing call changes no state.
int32_t plan_append(Cache *c, int layer, int n_seqs, const int32_t *seq_ids, const int32_t *n_tok,
                    std::vector<AppendTok> &toks) {
    LayerState &ls = c->L[layer];
    int64_t need_pages = 0;
    for (int i = 0; i < n_seqs; i++) {
        if (!n_tok || n_tok[i] < 0) return fail(RLX_ERR_INVALID, "negative token count");
        const SeqState &s = ls.seqs[seq_ids[i]];
        const int64_t new_len = (int64_t)s.len + n_tok[i];
        const int64_t pages_after = (new_len + c->P - 1) / c->P;
        if (s.first + pages_after > c->max_pages)
            return fail(RLX_ERR_OVERFLOW,
                        "Append: layer %d overflow: total=%d + newLen=%d > capacity=%d", layer,
                        s.len, n_tok[i], (c->max_pages - s.first) * c->P);
        need_pages += pages_after - s.pages;
    }
    if (need_pages > (int64_t)ls.free_stack.size())
        return fail(RLX_ERR_POOL, "page pool exhausted: layer %d needs %lld pages, %zu free", layer,
                    (long long)need_pages, ls.free_stack.size());
    int32_t row0 = 0;
    for (int i = 0; i < n_seqs; i++) {
        const int seq = seq_ids[i];
        SeqState &s = ls.seqs[seq];
        for (int j = 0; j < n_tok[i]; j++) {
            const int pos = s.len + j;
            const int k = s.first + pos / c->P;
            if (pos % c->P == 0) {
                const int32_t page = ls.free_stack.back();
                ls.free_stack.pop_back();
                c->set_entry(layer, seq, k, page);
                s.pages++;
            }
            toks.push_back(AppendTok{c->entry(layer, seq, k), pos % c->P, row0, n_tok[i]});
        }
        s.len += n_tok[i];
        if (n_tok[i] > 0) s.chunks.push_back(n_tok[i]);
        row0 += n_tok[i];
    }
    return RLX_OK;
}

// Context splits of the MLA decode, per row: nsplit_r = ceil(len_r /
// target) with target = ceil(sum of lengths / (slots - rows)) tokens (at
// least kMlaMinSplit), so that the work-groups -- sum of nsplit_r <= slots,
// the CUs times the work-groups one CU holds -- fit one residency round and
// none holds more than `target` tokens, whatever the mix of lengths.  A
// row's splits are near-equal (mla_split_bound in the kernel); at most
// len / 64 and kMaxSplits splits per row.
constexpr int kMlaMinSplit = 128;
std::vector<int> mla_splits(const std::vector<int> &lens, int64_t slots) {
    static const int64_t slot_override = [] {
        const char *e = getenv("RLX_DECODE_SLOTS");  // tuning override
        return e ? (int64_t)atoll(e) : (int64_t)0;
    }();
    static const int min_override = [] {
        const char *e = getenv("RLX_DECODE_MIN_SPLIT");  // tuning override
        return e ? atoi(e) : 0;
    }();
    if (slot_override > 0) slots = slot_override;
    const int min_split = min_override > 0 ? min_override : kMlaMinSplit;
    int64_t total = 0;
    for (int L : lens) total += L;
    const int64_t free_slots = std::max<int64_t>(1, slots - (int64_t)lens.size());
    const int64_t target = std::max<int64_t>(min_split, (total + free_slots - 1) / free_slots);
    std::vector<int> n(lens.size());
    for (size_t i = 0; i < lens.size(); i++) {
        const int64_t want = (lens[i] + target - 1) / target;
        n[i] = (int)std::max<int64_t>(1, std::min<int64_t>({want, lens[i] / 64, kMaxSplits}));
    }
    return n;
}

// Prefill work order for the 8 XCDs.  Work-group b runs on XCD b % 8 and
// each XCD has its own L2, so all query tiles of one (sequence, head group)
// -- which stream the same K/V blocks in the same order -- are placed on one
// XCD at consecutive positions: the XCD then fetches each block from HBM once.
// Groups go to the least-loaded XCD, largest first; shorter XCD lists are
// padded with empty items (row -1).
constexpr int kXcds = 8;
std::vector<int4> xcd_order(const std::vector<std::vector<int4>> &groups,
                            const std::vector<double> &cost) {
    static const bool plain = [] {
        const char *e = getenv("RLX_PREFILL_ORDER");  // tuning override: "plain"
        return e && strcmp(e, "plain") == 0;
    }();
    if (plain) {
        std::vector<int4> out;
        for (auto &g : groups) out.insert(out.end(), g.begin(), g.end());
        return out;
    }
    std::vector<int> idx(groups.size());
    for (size_t i = 0; i < idx.size(); i++) idx[i] = (int)i;
    std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return cost[a] > cost[b]; });
    std::vector<std::vector<int4>> lists(kXcds);
    std::vector<double> load(kXcds, 0.0);
    for (int g : idx) {
        const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
        load[x] += cost[g];
        lists[x].insert(lists[x].end(), groups[g].begin(), groups[g].end());
    }
    size_t n = 0;
    for (auto &l : lists) n = std::max(n, l.size());
    std::vector<int4> out(n * kXcds, int4{-1, 0, 0, 0});
    for (int x = 0; x < kXcds; x++)
        for (size_t i = 0; i < lists[x].size(); i++) out[i * kXcds + x] = lists[x][i];
    return out;
}

// Keys a prefill query tile attends (its work is proportional).
int tile_keys(const AttRow &r, int mask_mode, int toks, int qt) {
    const int jmax = std::min(r.nq - 1, qt * toks + toks - 1);
    if (mask_mode == RLX_MASK_CAUSAL) return std::min(r.len, r.len - r.nq + jmax + 1);
    if (mask_mode == RLX_MASK_REF && r.nq == r.len) return jmax + 1;
    return r.len;
}

// One AttRow per sequence, or -- with qtile > 0 (GQA decode kernel only) --
// one per tile of at most qtile queries, each with its own context splits.
// Cuts of the GQA decode ranges, in units of 64 padded positions: cut i is
// floor(i * total / n), moved onto the nearer row boundary when one lies
// within snap units (pre: the rows' padded starts, pre.back() = total).  The
// decode kernel computes the same cuts when its rows travel in the arguments.
void gqa_range_cuts(const int *pre, int n_rows, int n, int snap, int *cuts) {
    const int total = pre[n_rows];
    for (int i = 0; i <= n; i++) {
        const int b = (int)((int64_t)i * total / n);
        cuts[i] = b;
        if (b <= 0 || b >= total) continue;
        const int r = (int)(std::upper_bound(pre, pre + n_rows + 1, b) - pre) - 1;
        const int d0 = b - pre[r], d1 = pre[r + 1] - b;
        if (std::min(d0, d1) <= snap) cuts[i] = d0 <= d1 ? pre[r] : pre[r + 1];
    }
}

// Rows of a GQA decode call: one AttRow per sequence or, with qtile > 0,
// per tile of at most qtile queries.  Writes the first `cap` rows into
// rows[] and the number needed into *n_out (callers size or reject by it).
int32_t gqa_decode_rows(Cache *c, int layer, int n_seqs, const int32_t *seq_ids, const int32_t *n_q,
                        int qtile, AttRow *rows, int cap, int *n_out) {
    const LayerState &ls = c->L[layer];
    int n = 0, qrow = 0;
    for (int i = 0; i < n_seqs; i++) {
        const SeqState &s = ls.seqs[seq_ids[i]];
        const int nq = n_q ? n_q[i] : 1;
        if (s.len <= 0) return fail(RLX_ERR_STATE, "sequence %d holds no tokens", seq_ids[i]);
        if (nq < 1 || nq > s.len)
            return fail(RLX_ERR_INVALID, "n_q=%d must be in [1, len=%d]", nq, s.len);
        const int step = qtile > 0 ? qtile : nq;
        for (int q0 = 0; q0 < nq; q0 += step, n++) {
            if (n >= cap) continue;
            AttRow &r = rows[n];
            r.tab = (int32_t)(c->row_base(layer, seq_ids[i]) + s.first);
            r.len = s.len;
            r.nq = nq;
            r.qrow = qrow;
            r.nsplit = 1;
            r.part = n;
            r.q0 = q0;
            r.qn = std::min(step, nq - q0);
        }
        qrow += nq;
    }
    *n_out = n;
    return RLX_OK;
}

// Balanced ranges of the GQA decode split: the rows' tokens, each row padded
// to a multiple of 64, laid end to end and cut into one near-equal range per
// CU's worth of kv heads (work-groups = ranges x kv heads ~ CUs), cuts within
// kGqaSnap64 units of a row boundary moved onto it.  Every work-group then
// streams about the same number of tokens whatever the length mix, and one
// work-group per CU is the residency that measured fastest (splits by one
// fixed chunk left work-groups of very different sizes, and some CUs with
// several of them).  Fills ranges[] (first row, its padded start, [lo, hi)
// in 64-position units) and every row's part / nsplit (partial slot of
// (row r, range i) = r + i); pre[n_rows + 1] and cuts[n_ranges + 1] are the
// caller's scratch.  Returns the number of ranges (at most cus / kvh).
constexpr int kGqaSnap64 = 4;
// Work-groups per CU of the GQA decode (tuning override RLX_GQA_WG_PER_CU,
// 1..4; default 1).
// Bytes the MLA prefill may expand K_c and V^T into at once (4 GiB: config
// 4's 2.15 GB in one group; tuning override RLX_MLA_EXPAND_MB, read per call).
int64_t mla_expand_budget() {
    const char *e = getenv("RLX_MLA_EXPAND_MB");
    const int64_t mb = e ? atoll(e) : 0;
    return mb > 0 ? mb << 20 : (int64_t)4 << 30;
}

constexpr int kGqaLongRange = 4096;  // tokens per range that make a call "long"
int gqa_wg_per_cu() {
    static const int v = [] {
        const char *e = getenv("RLX_GQA_WG_PER_CU");
        const int x = e ? atoi(e) : 1;
        return (x >= 1 && x <= 4) ? x : 1;
    }();
    return v;
}
int gqa_decode_split(const Cache *c, AttRow *rows, int n_rows, int *pre, int *cuts, int4 *ranges,
                     int *total64_out) {
    pre[0] = 0;
    for (int i = 0; i < n_rows; i++) pre[i + 1] = pre[i] + (rows[i].len + 63) / 64;
    const int total64 = pre[n_rows];
    // Ranges per kv head: one work-group per CU, except for long calls
    // (at least kGqaLongRange tokens per range), which take three quarters
    // of the CUs, rounded down to a multiple of the 8 XCDs so that range i of
    // every kv head runs on the same XCD (work-group b runs on XCD b mod 8).
    // Measured on the 8k headline (16 x 8192, 8 kv heads; fraction of 8 TB/s
    // by ranges per kv head): 16: 0.71, 20: 0.78, 22: 0.81, 23: 0.81,
    // 24: 0.84, 25: 0.82, 26: 0.82, 28: 0.82, 30: 0.80, 32: 0.81, 48: 0.77,
    // 64: 0.80; at 32k, 24: 0.88 against 0.85; config 2 (1 150 tokens per
    // range at 32) keeps every CU: 0.685 against 0.655 at 24.
    // RLX_GQA_RANGES overrides the count (tuning; at most the full count,
    // which the callers' range arrays are sized for).
    static const int ranges_override = [] {
        const char *e = getenv("RLX_GQA_RANGES");
        return e ? atoi(e) : 0;
    }();
    const int full = std::max(1, std::min(c->cus * gqa_wg_per_cu() / c->kvh, c->cus));
    int want = full;
    const int q3 = (full * 3 / 4) / 8 * 8;
    // (At least 2 ranges per XCD: with 16 kv heads or more the full count is
    // kept.)
    if (q3 >= 16 && (int64_t)total64 * 64 >= (int64_t)q3 * kGqaLongRange) want = q3;
    if (ranges_override > 0) want = std::min(ranges_override, full);
    const int n_ranges = std::max(1, std::min(want, total64));
    gqa_range_cuts(pre, n_rows, n_ranges, kGqaSnap64, cuts);
    for (int k = 0; k < n_rows; k++) rows[k].part = -1;
    int r = 0;
    for (int i = 0; i < n_ranges; i++) {
        const int lo = cuts[i], hi = cuts[i + 1];
        // first row with live tokens past lo
        while (r < n_rows && (int64_t)pre[r] * 64 + rows[r].len <= (int64_t)lo * 64) r++;
        ranges[i] = int4{r, r < n_rows ? pre[r] : total64, lo, hi};
        for (int k = r; k < n_rows && pre[k] < hi; k++) {
            if (rows[k].part < 0) rows[k].part = k + i;
            rows[k].nsplit = i - (rows[k].part - k) + 1;
        }
    }
    *total64_out = total64;
    return n_ranges;
}

// One AttRow per sequence of an attention call, with nsplit[i] context
// splits (nullptr: one) and its work items (row, split).
int32_t build_rows(Cache *c, int layer, int n_seqs, const int32_t *seq_ids, const int32_t *n_q,
                   const int *nsplit, std::vector<AttRow> &rows, std::vector<int2> &work,
                   int *total_q, int *max_nq, int *total_parts) {
    LayerState &ls = c->L[layer];
    int qrow = 0, part = 0, mx = 0;
    for (int i = 0; i < n_seqs; i++) {
        const SeqState &s = ls.seqs[seq_ids[i]];
        const int nq = n_q ? n_q[i] : 1;
        if (s.len <= 0) return fail(RLX_ERR_STATE, "sequence %d holds no tokens", seq_ids[i]);
        if (nq < 1 || nq > s.len)
            return fail(RLX_ERR_INVALID, "n_q=%d must be in [1, len=%d]", nq, s.len);
        AttRow r;
        r.tab = (int32_t)(c->row_base(layer, seq_ids[i]) + s.first);
        r.len = s.len;
        r.nq = nq;
        r.qrow = qrow;
        r.nsplit = nsplit ? nsplit[i] : 1;
        r.part = part;
        r.q0 = 0;
        r.qn = nq;
        for (int sp = 0; sp < r.nsplit; sp++) work.push_back(int2{(int)rows.size(), sp});
        rows.push_back(r);
        part += r.nsplit;
        qrow += nq;
        mx = std::max(mx, nq);
    }
    *total_q = qrow;
    *max_nq = mx;
    *total_parts = part;
    return RLX_OK;
}

// One layer's page moving between its pool page and a tier slot.
struct PageMove {
    int layer;
    int32_t page;
    int64_t slot;
};

// Copy the pages of `mv` to the tier (to_host) or back, with the page copy
// kernel: pinned slots are addressed directly; a file tier goes through the
// pinned staging buffer in chunks, the host copying between it and the
// mapping around each kernel.
int32_t copy_spill_pages(Cache *c, const std::vector<PageMove> &mv, bool to_host) {
    SpillTier &t = c->spill;
    if (mv.empty()) return RLX_OK;
    const size_t b0 = page_bytes0(c), b1 = page_bytes1(c), sb = t.slot_bytes;
    hipEvent_t e0, e1;
    int32_t rc = timing_events(c, &e0, &e1, RLX_TIME_COPY);
    if (rc) return rc;
    if (e0) HIP_TRY(hipEventRecord(e0, c->stream));
    const size_t chunk = t.map_bytes ? (size_t)t.bounce_slots : mv.size();
    for (size_t i0 = 0; i0 < mv.size(); i0 += chunk) {
        const size_t n = std::min(chunk, mv.size() - i0);
        if (t.map_bytes && !to_host)
            for (size_t j = 0; j < n; j++) memcpy(t.bounce + j * sb, t.base + (size_t)mv[i0 + j].slot * sb, sb);
        std::vector<uint64_t> addr(4 * n);  // src0, dst0, src1, dst1
        for (size_t j = 0; j < n; j++) {
            const PageMove &m = mv[i0 + j];
            const uint8_t *host = t.map_bytes ? t.dev_bounce + j * sb : t.dev_base + (size_t)m.slot * sb;
            const uint8_t *d0 = (const uint8_t *)c->L[m.layer].pool0 + (size_t)m.page * b0;
            const uint8_t *d1 = b1 ? (const uint8_t *)c->L[m.layer].pool1 + (size_t)m.page * b1 : nullptr;
            addr[j] = (uint64_t)(to_host ? d0 : host);
            addr[n + j] = (uint64_t)(to_host ? host : d0);
            addr[2 * n + j] = (uint64_t)(to_host ? d1 : host + b0);
            addr[3 * n + j] = (uint64_t)(to_host ? host + b0 : d1);
        }
        void *dev;
        if ((rc = stage(c, addr.data(), addr.size() * sizeof(uint64_t), &dev))) return rc;
        const uint64_t *a = (const uint64_t *)dev;
        HIP_TRY(launch_page_copy(c->stream, a, a + n, (int)n, (int64_t)b0));
        if (b1) HIP_TRY(launch_page_copy(c->stream, a + 2 * n, a + 3 * n, (int)n, (int64_t)b1));
        if (t.map_bytes) {
            HIP_TRY(hipStreamSynchronize(c->stream));
            if (to_host)
                for (size_t j = 0; j < n; j++) memcpy(t.base + (size_t)mv[i0 + j].slot * sb, t.bounce + j * sb, sb);
        }
    }
    if (e1) HIP_TRY(hipEventRecord(e1, c->stream));
    return RLX_OK;
}

}  // namespace

extern "C" {

int32_t rlx_init(int32_t device) {
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(RLX_ERR_INVALID, "device %d of %d", device, n);
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(RLX_ERR_UNSUPPORTED, "device %d is %s; librelux_kv is built for gfx950", device,
                    prop.gcnArchName);
    if (device >= kMaxDevices) return fail(RLX_ERR_UNSUPPORTED, "device %d >= %d", device, kMaxDevices);
    if (!g_scratch[device]) {
        // This device's copy of the no-alloc scratch (the device is current).
        void *p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(RLX_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
        g_scratch[device] = p;
    }
    return RLX_OK;
}

int32_t rlx_last_error(char *buf, int64_t len) {
    if (!buf || len <= 0) return RLX_ERR_INVALID;
    snprintf(buf, (size_t)len, "%s", g_err.c_str());
    return RLX_OK;
}

int32_t rlx_version(char *buf, int64_t len) {
    if (!buf || len <= 0) return RLX_ERR_INVALID;
    snprintf(buf, (size_t)len, "librelux_kv 0.1 gfx950");
    return RLX_OK;
}

int32_t rlx_dev_alloc(int64_t bytes, void **out) {
    if (!out || bytes < 0) return fail(RLX_ERR_INVALID, "bad alloc request");
    *out = nullptr;
    if (bytes == 0) return RLX_OK;
    HIP_TRY(hipMalloc(out, (size_t)bytes));
    return RLX_OK;
}

int32_t rlx_dev_free(void *ptr) {
    if (ptr) HIP_TRY(hipFree(ptr));
    return RLX_OK;
}

int32_t rlx_h2d(void *dst, const void *src, int64_t bytes) {
    if (bytes > 0) HIP_TRY(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
    return RLX_OK;
}

int32_t rlx_d2h(void *dst, const void *src, int64_t bytes) {
    if (bytes > 0) HIP_TRY(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
    return RLX_OK;
}

int32_t rlx_device_sync(void) {
    HIP_TRY(hipDeviceSynchronize());
    return RLX_OK;
}

int32_t rlx_kv_create(int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t page_tokens,
                      int32_t pool_pages, int32_t max_seqs, int32_t max_pages_per_seq,
                      void **out) {
    if (!out) return fail(RLX_ERR_INVALID, "null out");
    *out = nullptr;
    if (layers <= 0) return fail(RLX_ERR_INVALID, "NewKVCacheSized: numLayers=%d, must be > 0", layers);
    if (kv_heads <= 0 || pool_pages <= 0 || max_seqs <= 0 || max_pages_per_seq <= 0)
        return fail(RLX_ERR_INVALID, "kv_heads, pool_pages, max_seqs, max_pages must be > 0");
    if (head_dim <= 0 || head_dim > 256)
        return fail(RLX_ERR_UNSUPPORTED, "head_dim=%d (supported: 1 to 256)", head_dim);
    if (page_tokens <= 0 || page_tokens % 16 != 0)
        return fail(RLX_ERR_UNSUPPORTED, "page_tokens=%d must be a positive multiple of 16", page_tokens);
    Cache *c = new Cache;
    c->kind = kGQA;
    c->layers = layers;
    c->kvh = kv_heads;
    // Pages store the smallest supported head dim >= head_dim; the dims past
    // head_dim hold zeros (written by every append).  The kernels take caller
    // rows of a multiple of 8 dims: other widths are padded at the boundary.
    c->hdu = head_dim;
    c->hdi = (head_dim + 7) & ~7;
    static const int kStoredDims[] = {16, 32, 64, 96, 128, 256};
    for (int d : kStoredDims)
        if (d >= c->hdi) {
            c->hd = d;
            break;
        }
    c->P = page_tokens;
    c->pool_pages = pool_pages;
    c->max_seqs = max_seqs;
    c->max_pages = max_pages_per_seq;
    int32_t rc = create_common(c);
    if (rc) {
        destroy_cache(c);
        return rc;
    }
    *out = c;
    return RLX_OK;
}

int32_t rlx_mla_create(int32_t layers, int32_t d_c, int32_t d_r, int32_t page_tokens,
                       int32_t pool_pages, int32_t max_seqs, int32_t max_pages_per_seq,
                       void **out) {
    if (!out) return fail(RLX_ERR_INVALID, "null out");
    *out = nullptr;
    if (layers <= 0) return fail(RLX_ERR_INVALID, "NewMLACache: numLayers=%d, must be > 0", layers);
    if (pool_pages <= 0 || max_seqs <= 0 || max_pages_per_seq <= 0)
        return fail(RLX_ERR_INVALID, "pool_pages, max_seqs, max_pages must be > 0");
    // NewMLA (mla.go:67-79) takes any dC and an even dHR; the stored row is
    // the 512 + 64 layout, zero padded past the caller's dims.
    if (d_c <= 0 || d_r <= 0 || d_r % 2 != 0)
        return fail(RLX_ERR_INVALID, "NewMLACache: dC=%d dHR=%d (both > 0, dHR even)", d_c, d_r);
    if (d_c > kMlaDc || d_r > kMlaDr)
        return fail(RLX_ERR_UNSUPPORTED, "MLA d_c=%d d_r=%d (at most %d and %d)", d_c, d_r, kMlaDc,
                    kMlaDr);
    if (page_tokens <= 0 || page_tokens % 16 != 0)
        return fail(RLX_ERR_UNSUPPORTED, "page_tokens=%d must be a positive multiple of 16", page_tokens);
    Cache *c = new Cache;
    c->kind = kMLA;
    c->layers = layers;
    c->dc = d_c;
    c->dr = d_r;
    c->P = page_tokens;
    c->pool_pages = pool_pages;
    c->max_seqs = max_seqs;
    c->max_pages = max_pages_per_seq;
    int32_t rc = create_common(c);
    if (rc) {
        destroy_cache(c);
        return rc;
    }
    *out = c;
    return RLX_OK;
}

int32_t rlx_cache_destroy(void *h) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    destroy_cache(as_cache(h));
    return RLX_OK;
}

int32_t rlx_cache_reset(void *h) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    for (auto &ls : c->L) reset_layer_state(c, ls);
    reset_spill(c);
    c->pending.clear();
    HIP_TRY(launch_fill_i32(c->stream, c->d_table, -1, (int64_t)c->layers * c->max_seqs * c->max_pages));
    return RLX_OK;
}

int32_t rlx_cache_sync(void *h) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    HIP_TRY(hipStreamSynchronize(as_cache(h)->stream));
    return RLX_OK;
}

int32_t rlx_cache_set_stream(void *h, void *stream) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    HIP_TRY(hipStreamSynchronize(c->stream));
    // NULL is the device's null stream (torch's default stream reports 0).
    c->stream = (hipStream_t)stream;
    return RLX_OK;
}

int32_t rlx_cache_reserve(void *h, uint64_t ws_bytes, uint64_t stage_bytes, uint64_t ad_bytes) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (ws_bytes > c->ws_cap) {
        const size_t cap = ((size_t)ws_bytes + 65535) & ~(size_t)65535;
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (c->ws) HIP_TRY(hipFree(c->ws));
        c->ws = nullptr;
        c->ws_cap = 0;
        HIP_TRY(hipMalloc(&c->ws, cap));
        c->ws_cap = cap;
    }
    if (ad_bytes > c->ad_cap) {
        const size_t cap = ((size_t)ad_bytes + 65535) & ~(size_t)65535;
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (c->ad) HIP_TRY(hipFree(c->ad));
        c->ad = nullptr;
        c->ad_cap = 0;
        HIP_TRY(hipMalloc(&c->ad, cap));
        c->ad_cap = cap;
    }
    for (Slot &s : c->slots) {
        if (stage_bytes <= s.cap) continue;
        const size_t cap = ((size_t)stage_bytes + 4095) & ~(size_t)4095;
        // The slot's device copy may still be read by queued kernels.
        HIP_TRY(hipStreamSynchronize(c->stream));
        s.pending = false;
        if (s.host) HIP_TRY(hipHostFree(s.host));
        if (s.dev) HIP_TRY(hipFree(s.dev));
        s.host = nullptr;
        s.dev = nullptr;
        s.cap = 0;
        HIP_TRY(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
        HIP_TRY(hipMalloc(&s.dev, cap));
        s.cap = cap;
    }
    return RLX_OK;
}

int32_t rlx_cache_memory(void *h, uint64_t *out) {
    if (!h || !out) return fail(RLX_ERR_INVALID, "null argument");
    const Cache *c = as_cache(h);
    size_t smin = c->slots[0].cap;
    for (const Slot &s : c->slots) smin = std::min(smin, s.cap);
    out[0] = c->ws_cap;
    out[1] = c->ws_peak;
    out[2] = smin;
    out[3] = c->stage_peak;
    out[4] = c->ad_cap;
    out[5] = c->ad_peak;
    return RLX_OK;
}

int32_t rlx_cache_timing(void *h, int32_t enable) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->timing = enable;
    c->tev_used = 0;
    return RLX_OK;
}

int32_t rlx_cache_kernel_time(void *h, float *total_ms, int32_t *count) {
    if (!h || !total_ms || !count) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    HIP_TRY(hipStreamSynchronize(c->stream));
    double sum = 0.0;
    for (size_t i = 0; i < c->tev_used; i++) {
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, c->tev[i].first, c->tev[i].second));
        sum += ms;
    }
    *total_ms = (float)sum;
    *count = (int32_t)c->tev_used;
    c->tev_used = 0;
    return RLX_OK;
}

// Rows (tokens x kv heads) an append of n_tok tokens per sequence carries.
static int64_t append_rows(const Cache *c, int n_seqs, const int32_t *n_tok) {
    int64_t n = 0;
    for (int i = 0; n_tok && i < n_seqs; i++) n += std::max(0, n_tok[i]);
    return n * c->kvh;
}

// rlx_kv_append after its argument checks.  pad: two adapter regions for
// the K and V rows of a padded head dim, carved by the caller before
// anything changes (so that a failed allocation leaves the cache as it
// was), or null.
static int32_t kv_append_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                              const int32_t *n_tok, const void *k_src, const void *v_src,
                              int32_t src_dtype, int32_t src_layout, char *const *pad) {
    int32_t rc;
    std::vector<AppendTok> toks;
    if ((rc = plan_append(c, layer, n_seqs, seq_ids, n_tok, toks))) return rc;
    if (!toks.empty() && (!k_src || !v_src)) return fail(RLX_ERR_INVALID, "null K/V source");
    if (pad && !toks.empty()) {
        const int esz = src_dtype == RLX_BF16 ? 2 : 4;
        const int64_t rows = append_rows(c, n_seqs, n_tok);
        HIP_TRY(launch_repack_rows(c->stream, k_src, c->hdu, pad[0], c->hdi, rows, esz));
        HIP_TRY(launch_repack_rows(c->stream, v_src, c->hdu, pad[1], c->hdi, rows, esz));
        k_src = pad[0];
        v_src = pad[1];
    }
    std::vector<Patch> patches = take_pending(c);
    PlanArg plan_arg;
    const PlanArg *plan;
    int tok_off;
    const Patch *d_patches;
    const AppendTok *d_toks;
    if ((rc = append_plan(c, patches, toks, &plan_arg, &plan, &tok_off, &d_patches, &d_toks)))
        return rc;
    LayerState &ls = c->L[layer];
    HIP_TRY(launch_kv_append(c->stream, plan, tok_off, ls.pool0, ls.pool1, c->d_table, d_patches,
                             (int)patches.size(), d_toks, (int)toks.size(), k_src, v_src,
                             src_dtype == RLX_BF16, src_layout, c->kvh, c->hd, c->hdi, c->P));
    return RLX_OK;
}

static int32_t kv_append_check(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               int32_t src_dtype, int32_t src_layout) {
    if (c->kind != kGQA) return fail(RLX_ERR_INVALID, "rlx_kv_append on an MLA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (src_dtype != RLX_F32 && src_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "src_dtype");
    if (src_layout != RLX_LAYOUT_HSD && src_layout != RLX_LAYOUT_SHD) return fail(RLX_ERR_INVALID, "src_layout");
    return RLX_OK;
}

int32_t rlx_kv_append(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                      const int32_t *n_tok, const void *k_src, const void *v_src,
                      int32_t src_dtype, int32_t src_layout) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = kv_append_check(c, layer, n_seqs, seq_ids, src_dtype, src_layout);
    if (rc) return rc;
    char *pad[2] = {nullptr, nullptr};
    const int64_t rows = append_rows(c, n_seqs, n_tok);
    const bool padded = c->hdu != c->hdi && rows > 0;
    if (padded) {
        const size_t b = (size_t)rows * c->hdi * (src_dtype == RLX_BF16 ? 2 : 4);
        const size_t sz[2] = {b, b};
        if ((rc = adapter_regions(c, sz, 2, pad))) return rc;
    }
    return kv_append_impl(c, layer, n_seqs, seq_ids, n_tok, k_src, v_src, src_dtype, src_layout,
                          padded ? pad : nullptr);
}

int32_t rlx_pack_qkv(const void *w_q, const void *w_k, const void *w_v, int32_t w_dtype,
                     int32_t d_model, int32_t num_heads, int32_t kv_heads, int32_t head_dim,
                     void *out) {
    if (!w_q || !w_k || !w_v || !out) return fail(RLX_ERR_INVALID, "null weight pointer");
    if (w_dtype != RLX_F32 && w_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "w_dtype");
    if (d_model <= 0 || num_heads <= 0 || kv_heads <= 0 || head_dim <= 0)
        return fail(RLX_ERR_INVALID, "d_model, heads and head_dim must be > 0");
    const int pw = gqa_pack_width(num_heads, kv_heads, head_dim);
    const PackSrc src{{w_q, w_k, w_v, w_q},
                      {num_heads, kv_heads, kv_heads, 0},
                      {head_dim, head_dim, head_dim, 0},
                      {pw, pw, pw, 0}};
    HIP_TRY(launch_pack_proj(nullptr, src, w_dtype == RLX_BF16, d_model, (uint16_t *)out));
    return RLX_OK;
}

int32_t rlx_pack_out(const void *w, int32_t w_dtype, int32_t k_in, int32_t n_out, void *out) {
    if (!w || !out) return fail(RLX_ERR_INVALID, "null weight pointer");
    if (w_dtype != RLX_F32 && w_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "w_dtype");
    if (k_in <= 0 || n_out <= 0) return fail(RLX_ERR_INVALID, "k_in and n_out must be > 0");
    // (n_out packed as a multiple of 16 features, k_in as one of 32 rows: zeros)
    const PackSrc src{{w, w, w, w}, {1, 0, 0, 0}, {n_out, 0, 0, 0}, {(n_out + 15) / 16 * 16, 0, 0, 0}};
    HIP_TRY(launch_pack_proj(nullptr, src, w_dtype == RLX_BF16, k_in, (uint16_t *)out));
    return RLX_OK;
}

int32_t rlx_out_project(void *h, int32_t rows, const void *x, int32_t x_dtype, int32_t k_in,
                        const void *w_packed, int32_t n_out, const void *residual, void *out,
                        int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (rows < 0 || k_in <= 0 || n_out <= 0) return fail(RLX_ERR_INVALID, "rlx_out_project: rows/k_in/n_out");
    if (rows == 0) return RLX_OK;
    if (!x || !w_packed || !out) return fail(RLX_ERR_INVALID, "rlx_out_project: null pointer");
    if ((x_dtype != RLX_F32 && x_dtype != RLX_BF16) || (out_dtype != RLX_F32 && out_dtype != RLX_BF16))
        return fail(RLX_ERR_INVALID, "rlx_out_project: dtype");
    const size_t xb = x_dtype == RLX_BF16 ? 2 : 4, ob = out_dtype == RLX_BF16 ? 2 : 4;
    int32_t rc;
    // x rows of a width that is not a multiple of 32: copied to rows of the
    // next multiple with zeros (the packed weights hold zero rows there).
    const int kp = (k_in + 31) / 32 * 32;
    if (kp != k_in) {
        const size_t sz[1] = {(size_t)rows * kp * xb};
        char *pad[1];
        if ((rc = adapter_regions(c, sz, 1, pad))) return rc;
        HIP_TRY(launch_repack_rows(c->stream, x, k_in, pad[0], kp, rows, (int)xb));
        x = pad[0];
        k_in = kp;
    }
    for (int r0 = 0; r0 < rows; r0 += kProjRows) {
        const int n = std::min(kProjRows, rows - r0);
        hipEvent_t e0, e1;
        if ((rc = timing_events(c, &e0, &e1, RLX_TIME_PROJECT))) return rc;
        ProjDims pd{};
        pd.D = n_out;
        pd.DW = (n_out + 15) / 16 * 16;
        HIP_TRY(launch_proj(c->stream, kProjModelOut, nullptr, nullptr, 0, nullptr, nullptr, 0, 0, n,
                            (const char *)x + (size_t)r0 * k_in * xb, x_dtype == RLX_BF16, k_in,
                            (const uint16_t *)w_packed, pd, nullptr, nullptr,
                            (char *)out + (size_t)r0 * n_out * ob,
                            residual ? (void *)((const char *)residual + (size_t)r0 * n_out * ob) : nullptr,
                            out_dtype == RLX_BF16, nullptr, nullptr, nullptr, 0, c->cus, e0, e1));
    }
    return RLX_OK;
}

int32_t rlx_pack_mla_proj(const void *w_q, const void *w_qr, const void *w_dkv, const void *w_kr,
                          int32_t w_dtype, int32_t d_model, int32_t num_heads, int32_t head_dim,
                          int32_t d_c, int32_t d_r, void *out) {
    if (!w_q || !w_qr || !w_dkv || !w_kr || !out) return fail(RLX_ERR_INVALID, "null weight pointer");
    if (w_dtype != RLX_F32 && w_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "w_dtype");
    if (d_model <= 0 || num_heads <= 0 || head_dim <= 0 || d_c <= 0 || d_r <= 0)
        return fail(RLX_ERR_INVALID, "d_model, heads, head_dim, d_c and d_r must be > 0");
    const int drp = (d_r + 15) & ~15, dcp = (d_c + 15) & ~15;
    const PackSrc src{{w_q, w_qr, w_dkv, w_kr},
                      {num_heads, num_heads, 1, 1},
                      {head_dim, d_r, d_c, d_r},
                      {mla_pack_width(num_heads, head_dim), drp, dcp, drp}};
    HIP_TRY(launch_pack_proj(nullptr, src, w_dtype == RLX_BF16, d_model, (uint16_t *)out));
    return RLX_OK;
}

}  // extern "C"

namespace {

// Shared body of the fused projection + RoPE + append entry points.
int32_t project_append(Cache *c, int model, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_tok, const void *x, int32_t x_dtype, int32_t d_model,
                       const void *w_packed, const ProjDims &pd, const float *rope_cos,
                       const float *rope_sin, int32_t rope_rows, int32_t rope_mode, void *q_out,
                       void *q_out2, int32_t q_dtype) {
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (x_dtype != RLX_F32 && x_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "x_dtype");
    if (q_dtype != RLX_F32 && q_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "q_dtype");
    if (rope_mode < RLX_ROPE_OFFSET || rope_mode > RLX_ROPE_NONE) return fail(RLX_ERR_INVALID, "rope_mode");
    if (d_model <= 0) return fail(RLX_ERR_INVALID, "d_model=%d must be positive", d_model);
    if (rope_mode != RLX_ROPE_NONE && (!rope_cos || !rope_sin || rope_rows <= 0))
        return fail(RLX_ERR_INVALID, "RoPE tables required");
    LayerState &ls = c->L[layer];
    // RoPE position of every new token (rope.go:151-158 for the reference rule).
    std::vector<int32_t> pos;
    int total = 0;
    for (int i = 0; i < n_seqs; i++) {
        if (!n_tok || n_tok[i] < 0) return fail(RLX_ERR_INVALID, "negative token count");
        const SeqState &st = ls.seqs[seq_ids[i]];
        for (int j = 0; j < n_tok[i]; j++) {
            int p = -1;
            if (rope_mode == RLX_ROPE_OFFSET) p = st.pos_offset + st.len + j;
            if (rope_mode == RLX_ROPE_REF) p = st.len > 0 ? st.len : j;
            if (p >= 0 && p >= rope_rows)
                return fail(RLX_ERR_OVERFLOW, "RotaryEmbedding.Apply: position %d >= maxSeqLen %d", p, rope_rows);
            pos.push_back(p);
        }
        total += n_tok[i];
    }
    if (total == 0) return RLX_OK;
    if (!x || !w_packed || !q_out || (model == kProjModelMLA && !q_out2))
        return fail(RLX_ERR_INVALID, "null x / weights / q_out");
    // x rows of a width that is not a multiple of 32: copied to rows of the
    // next multiple with zeros (the packed weights hold zero rows there),
    // before anything is appended.
    const int kp = (d_model + 31) / 32 * 32;
    if (kp != d_model) {
        const int xe = x_dtype == RLX_BF16 ? 2 : 4;
        const size_t sz[1] = {(size_t)total * kp * xe};
        char *pad[1];
        if ((rc = adapter_regions(c, sz, 1, pad))) return rc;
        HIP_TRY(launch_repack_rows(c->stream, x, d_model, pad[0], kp, total, xe));
        x = pad[0];
        d_model = kp;
    }
    std::vector<AppendTok> toks;
    if ((rc = plan_append(c, layer, n_seqs, seq_ids, n_tok, toks))) return rc;
    std::vector<Patch> patches = take_pending(c);
    const int xb = x_dtype == RLX_BF16 ? 2 : 4, qb = q_dtype == RLX_BF16 ? 2 : 4;
    for (int r0 = 0; r0 < total; r0 += kProjRows) {
        const int rows = std::min(kProjRows, total - r0);
        const std::vector<Patch> none;
        const std::vector<Patch> &pt = (r0 == 0) ? patches : none;
        const size_t toff = (pt.size() * sizeof(Patch) + 15) & ~(size_t)15;
        const size_t poff = toff + rows * sizeof(AppendTok);
        std::vector<char> bytes(poff + rows * sizeof(int32_t));
        if (!pt.empty()) memcpy(bytes.data(), pt.data(), pt.size() * sizeof(Patch));
        memcpy(bytes.data() + toff, toks.data() + r0, rows * sizeof(AppendTok));
        memcpy(bytes.data() + poff, pos.data() + r0, rows * sizeof(int32_t));
        PlanArg plan_arg;
        const PlanArg *plan = nullptr;
        const Patch *d_p = nullptr;
        const AppendTok *d_t = nullptr;
        const int32_t *d_pos = nullptr;
        if (bytes.size() <= sizeof(PlanArg)) {
            memcpy(plan_arg.b, bytes.data(), bytes.size());
            plan = &plan_arg;
        } else {
            void *dev;
            if ((rc = stage(c, bytes.data(), bytes.size(), &dev))) return rc;
            d_p = (const Patch *)dev;
            d_t = (const AppendTok *)((char *)dev + toff);
            d_pos = (const int32_t *)((char *)dev + poff);
        }
        // zeros in the stored dims past the caller's (none at the stored shapes)
        HIP_TRY(launch_proj_pad_zero(c->stream, model, plan, d_t, (int)toff, rows, pd, ls.pool0, ls.pool1,
                                     c->P));
        hipEvent_t e0, e1;
        if ((rc = timing_events(c, &e0, &e1, RLX_TIME_PROJECT))) return rc;
        char *q2 = model == kProjModelMLA ? (char *)q_out2 + (size_t)r0 * pd.H * pd.DR * qb : nullptr;
        HIP_TRY(launch_proj(c->stream, model, plan, d_p, (int)pt.size(), d_t, d_pos, (int)toff,
                            (int)poff, rows, (const char *)x + (size_t)r0 * d_model * xb,
                            x_dtype == RLX_BF16, d_model, (const uint16_t *)w_packed, pd, rope_cos,
                            rope_sin, (char *)q_out + (size_t)r0 * pd.H * pd.D * qb, q2,
                            q_dtype == RLX_BF16, ls.pool0, ls.pool1, c->d_table, c->P, c->cus, e0, e1));
    }
    return RLX_OK;
}

}  // namespace

extern "C" {

int32_t rlx_gqa_project_append(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_tok, const void *x, int32_t x_dtype,
                               int32_t d_model, const void *w_packed, int32_t num_heads,
                               const float *rope_cos, const float *rope_sin, int32_t rope_rows,
                               int32_t rope_mode, void *q_out, int32_t q_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kGQA) return fail(RLX_ERR_INVALID, "rlx_gqa_project_append on an MLA cache");
    if (c->hdu % 2 != 0)
        return fail(RLX_ERR_UNSUPPORTED, "rlx_gqa_project_append: RoPE needs an even head_dim (%d)", c->hdu);
    if (num_heads <= 0 || num_heads % c->kvh != 0)
        return fail(RLX_ERR_INVALID, "numHeads=%d not divisible by numKVHeads=%d", num_heads, c->kvh);
    // The packed features come in 16-feature tiles, each within one of the
    // q / k / v parts: heads are packed DW features wide (rlx_pack_qkv).
    ProjDims pd{};
    pd.H = num_heads;
    pd.KVH = c->kvh;
    pd.D = c->hdu;
    pd.DS = c->hd;
    pd.DW = gqa_pack_width(num_heads, c->kvh, c->hdu);
    return project_append(c, kProjModelGQA, layer, n_seqs, seq_ids, n_tok, x, x_dtype, d_model,
                          w_packed, pd, rope_cos, rope_sin, rope_rows, rope_mode, q_out, nullptr,
                          q_dtype);
}

int32_t rlx_mla_project_append(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_tok, const void *x, int32_t x_dtype,
                               int32_t d_model, const void *w_packed, int32_t num_heads,
                               int32_t head_dim, const float *rope_cos, const float *rope_sin,
                               int32_t rope_rows, int32_t rope_mode, void *q_nope_out,
                               void *q_rope_out, int32_t q_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kMLA) return fail(RLX_ERR_INVALID, "rlx_mla_project_append on a GQA cache");
    if (num_heads <= 0 || head_dim <= 0 || head_dim > 256)
        return fail(RLX_ERR_UNSUPPORTED, "num_heads=%d head_dim=%d (head_dim 1 to 256)", num_heads, head_dim);
    ProjDims pd{};
    pd.H = num_heads;
    pd.D = head_dim;
    pd.DW = mla_pack_width(num_heads, head_dim);
    pd.DR = c->dr;
    pd.DRP = (c->dr + 15) & ~15;
    pd.DC = c->dc;
    pd.DCP = (c->dc + 15) & ~15;
    return project_append(c, kProjModelMLA, layer, n_seqs, seq_ids, n_tok, x, x_dtype, d_model,
                          w_packed, pd, rope_cos, rope_sin, rope_rows, rope_mode, q_nope_out,
                          q_rope_out, q_dtype);
}

int32_t rlx_mla_append(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_tok, const void *c_src, const void *kr_src,
                       int32_t src_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kMLA) return fail(RLX_ERR_INVALID, "rlx_mla_append on a GQA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (src_dtype != RLX_F32 && src_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "src_dtype");
    std::vector<AppendTok> toks;
    if ((rc = plan_append(c, layer, n_seqs, seq_ids, n_tok, toks))) return rc;
    if (!toks.empty() && (!c_src || !kr_src)) return fail(RLX_ERR_INVALID, "null latent source");
    std::vector<Patch> patches = take_pending(c);
    PlanArg plan_arg;
    const PlanArg *plan;
    int tok_off;
    const Patch *d_patches;
    const AppendTok *d_toks;
    if ((rc = append_plan(c, patches, toks, &plan_arg, &plan, &tok_off, &d_patches, &d_toks)))
        return rc;
    HIP_TRY(launch_mla_append(c->stream, plan, tok_off, c->L[layer].pool0, c->d_table, d_patches,
                              (int)patches.size(), d_toks, (int)toks.size(), c_src, kr_src,
                              src_dtype == RLX_BF16, c->dc, c->dr, c->P));
    return RLX_OK;
}

static int32_t gather_rows(Cache *c, int layer, int n_seqs, const int32_t *seq_ids,
                           std::vector<AttRow> &rows, int *max_len) {
    LayerState &ls = c->L[layer];
    int off = 0, mx = 0;
    for (int i = 0; i < n_seqs; i++) {
        const SeqState &s = ls.seqs[seq_ids[i]];
        AttRow r{};
        r.tab = (int32_t)(c->row_base(layer, seq_ids[i]) + s.first);
        r.len = s.len;
        r.qrow = off;  // token offset of this sequence in the dense output
        rows.push_back(r);
        off += s.len;
        mx = std::max(mx, s.len);
    }
    *max_len = mx;
    return RLX_OK;
}

int32_t rlx_kv_gather(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                      void *k_out, void *v_out) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kGQA) return fail(RLX_ERR_INVALID, "rlx_kv_gather on an MLA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if ((rc = flush_patches(c))) return rc;
    std::vector<AttRow> rows;
    int max_len = 0;
    gather_rows(c, layer, n_seqs, seq_ids, rows, &max_len);
    if (max_len == 0) return RLX_OK;
    if (!k_out || !v_out) return fail(RLX_ERR_INVALID, "null gather output");
    void *ko = k_out, *vo = v_out;
    int64_t pad_rows = 0;
    if (c->hdu != c->hdi) {  // gathered at the padded width, then narrowed
        for (const AttRow &r : rows) pad_rows += r.len;
        pad_rows *= c->kvh;
        const size_t sz[2] = {(size_t)pad_rows * c->hdi * 2, (size_t)pad_rows * c->hdi * 2};
        char *pad[2];
        if ((rc = adapter_regions(c, sz, 2, pad))) return rc;
        ko = pad[0];
        vo = pad[1];
    }
    Blob b;
    size_t o_r = b.add(rows);
    void *dev;
    if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
    LayerState &ls = c->L[layer];
    HIP_TRY(launch_kv_gather(c->stream, ls.pool0, ls.pool1, c->d_table,
                             (const AttRow *)((char *)dev + o_r), n_seqs, max_len,
                             (uint16_t *)ko, (uint16_t *)vo, c->kvh, c->hd, c->hdi, c->P));
    if (pad_rows > 0) {
        HIP_TRY(launch_repack_rows(c->stream, ko, c->hdi, k_out, c->hdu, pad_rows, 2));
        HIP_TRY(launch_repack_rows(c->stream, vo, c->hdi, v_out, c->hdu, pad_rows, 2));
    }
    return RLX_OK;
}

int32_t rlx_mla_gather(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       void *c_out, void *kr_out) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kMLA) return fail(RLX_ERR_INVALID, "rlx_mla_gather on a GQA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if ((rc = flush_patches(c))) return rc;
    std::vector<AttRow> rows;
    int max_len = 0;
    gather_rows(c, layer, n_seqs, seq_ids, rows, &max_len);
    if (max_len == 0) return RLX_OK;
    if (!c_out || !kr_out) return fail(RLX_ERR_INVALID, "null gather output");
    Blob b;
    size_t o_r = b.add(rows);
    void *dev;
    if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
    HIP_TRY(launch_mla_gather(c->stream, c->L[layer].pool0, c->d_table,
                              (const AttRow *)((char *)dev + o_r), n_seqs, max_len,
                              (uint16_t *)c_out, (uint16_t *)kr_out, c->dc, c->dr, c->P));
    return RLX_OK;
}

}  // extern "C"

namespace {
// Query rows of one kv head one decode work-group holds: 32 (two 16-wide
// tiles), 16 for head_dim 256 (whose work-group needs the register file for
// one tile).
int gqa_rows_cap(const Cache *c) { return c->hd >= 256 ? 16 : 32; }

// Argument checks shared by the GQA attention entry points.
int32_t check_gqa_attend(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                         int32_t num_heads, int32_t q_dtype, int32_t qo_layout, int32_t mask_mode,
                         int32_t out_dtype) {
    if (c->kind != kGQA) return fail(RLX_ERR_INVALID, "GQA attention on an MLA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (num_heads <= 0 || num_heads % c->kvh != 0)
        return fail(RLX_ERR_INVALID, "numHeads=%d not divisible by numKVHeads=%d", num_heads, c->kvh);
    if (q_dtype != RLX_F32 && q_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "q_dtype");
    if (out_dtype != RLX_F32 && out_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "out_dtype");
    if (qo_layout != RLX_LAYOUT_HSD && qo_layout != RLX_LAYOUT_SHD) return fail(RLX_ERR_INVALID, "qo_layout");
    if (mask_mode < RLX_MASK_CAUSAL || mask_mode > RLX_MASK_NONE) return fail(RLX_ERR_INVALID, "mask_mode");
    return RLX_OK;
}
// Whether GQA calls with more query rows per kv head than the decode kernel
// holds run as FA2 chunked prefill: stored head dims 64, 128 and 256 (any
// caller head_dim they hold), any G = heads per kv head up to 256 (a tile
// holds floor(256 / G) tokens); other shapes tile their queries through
// the decode kernel.
bool gqa_use_fa2(const Cache *c, int G) {
    return (c->hd == 64 || c->hd == 128 || c->hd == 256) && G <= kPrefillRows;
}

// Query / output rows of a GQA call: sum of n_q (1 per sequence if null)
// times the query heads.
int64_t gqa_qo_rows(int n_seqs, const int32_t *n_q, int num_heads) {
    int64_t n = 0;
    for (int i = 0; i < n_seqs; i++) n += n_q ? std::max(0, n_q[i]) : 1;
    return n * num_heads;
}

// A GQA attention call on (q, out), through adapter rows of the padded head
// dim when the caller's is not a multiple of 8.  extra / pad: further
// regions to carve in the same adapter allocation (the K / V rows of
// rlx_gqa_append_attend), returned in pad.
template <class F>
int32_t gqa_call_padded(Cache *c, int64_t rows, const void *q, int32_t q_dtype, void *out,
                        int32_t out_dtype, F call, size_t extra = 0, char **pad = nullptr) {
    if (c->hdu == c->hdi || rows <= 0) return call(q, out);
    const int qe = q_dtype == RLX_BF16 ? 2 : 4, oe = out_dtype == RLX_BF16 ? 2 : 4;
    const size_t sz[4] = {(size_t)rows * c->hdi * qe, (size_t)rows * c->hdi * oe, extra, extra};
    char *p[4];
    int32_t rc = adapter_regions(c, sz, extra ? 4 : 2, p);
    if (rc) return rc;
    if (pad) {
        pad[0] = p[2];
        pad[1] = p[3];
    }
    HIP_TRY(launch_repack_rows(c->stream, q, c->hdu, p[0], c->hdi, rows, qe));
    if ((rc = call((const void *)p[0], (void *)p[1]))) return rc;
    HIP_TRY(launch_repack_rows(c->stream, p[1], c->hdi, out, c->hdu, rows, oe));
    return RLX_OK;
}

// GQA attention after the argument checks.
int32_t gqa_attend_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                        const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                        int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                        int32_t out_dtype) {
    int32_t rc = RLX_OK;
    const int G = num_heads / c->kvh;
    LayerState &ls = c->L[layer];
    std::vector<int> lens(n_seqs);
    int max_nq = 0;
    for (int i = 0; i < n_seqs; i++) {
        lens[i] = ls.seqs[seq_ids[i]].len;
        max_nq = std::max(max_nq, n_q ? n_q[i] : 1);
    }
    const int max_qr = G * max_nq;
    // Query rows past cap (the decode kernel's per kv head) take FA2 or query
    // tiles (gqa_use_fa2).
    const bool fa2 = gqa_use_fa2(c, G);
    const int cap = gqa_rows_cap(c);
    if (max_qr > cap && !fa2 && G > cap)
        return fail(RLX_ERR_UNSUPPORTED, "heads per kv head = %d with head_dim %d (at most %d)", G,
                    c->hdi, cap);
    if (max_qr > cap && fa2) {
        // Chunked prefill / long verify: FA2 tiles of kPrefillRows query rows.
        std::vector<AttRow> rows;
        std::vector<int2> unused;
        int total_q = 0, mnq = 0, parts = 0;
        if ((rc = build_rows(c, layer, n_seqs, seq_ids, n_q, nullptr, rows, unused, &total_q, &mnq, &parts)))
            return rc;
        const int toks = kPrefillRows / G;
        std::vector<std::vector<int4>> groups;
        std::vector<double> cost;
        for (int i = 0; i < n_seqs; i++) {
            const int tiles = (rows[i].nq + toks - 1) / toks;
            for (int kvh = 0; kvh < c->kvh; kvh++) {
                groups.emplace_back();
                cost.push_back(0.0);
                for (int qt = tiles - 1; qt >= 0; qt--) {
                    groups.back().push_back(int4{i, kvh, qt, 0});
                    cost.back() += tile_keys(rows[i], mask_mode, toks, qt);
                }
            }
        }
        const std::vector<int4> work = xcd_order(groups, cost);
        if ((rc = flush_patches(c))) return rc;
        Blob b;
        size_t o_r = b.add(rows), o_w = b.add(work);
        void *dev;
        if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
        if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)c->hdu));
        PrefillArgs a{};
        a.kpool = ls.pool0;
        a.vpool = ls.pool1;
        a.table = c->d_table;
        a.rows = (const AttRow *)((char *)dev + o_r);
        a.work = (const int4 *)((char *)dev + o_w);
        a.q = q;
        a.out = out;
        a.q_bf16 = q_dtype == RLX_BF16;
        a.layout = qo_layout;
        a.out_bf16 = out_dtype == RLX_BF16;
        a.mask_mode = mask_mode;
        a.H = num_heads;
        a.HQ = num_heads;
        a.h0 = 0;
        a.KVH = c->kvh;
        a.P = c->P;
        a.pshift = (c->P & (c->P - 1)) == 0 ? __builtin_ctz((unsigned)c->P) : -1;
        a.qscale = scale * 1.4426950408889634f;
        a.qd = c->hdi;
        a.od = c->hdi;
        a.vd = c->hd;
        a.dv0 = 0;
        hipEvent_t e0, e1;
        if ((rc = timing_events(c, &e0, &e1))) return rc;
        HIP_TRY(launch_prefill(c->stream, kSrcPaged, c->hd, a, (int)work.size(), e0, e1));
        return RLX_OK;
    }
    const int qtile = max_qr > cap ? cap / G : 0;
    const int nqt = std::min(max_qr, cap) > 16 ? 2 : 1;
    int n_rows = 0;
    if ((rc = gqa_decode_rows(c, layer, n_seqs, seq_ids, n_q, qtile, nullptr, 0, &n_rows))) return rc;
    std::vector<AttRow> rows(n_rows);
    if ((rc = gqa_decode_rows(c, layer, n_seqs, seq_ids, n_q, qtile, rows.data(), n_rows, &n_rows)))
        return rc;
    std::vector<int> pre(n_rows + 1), cuts(c->cus + 2);
    std::vector<int4> ranges(c->cus + 1);
    int total64 = 0;
    const int n_ranges = gqa_decode_split(c, rows.data(), n_rows, pre.data(), cuts.data(),
                                          ranges.data(), &total64);
    ranges.resize(n_ranges);
    const int parts = n_rows + n_ranges;
    if ((rc = flush_patches(c))) return rc;
    const int QRP = 16 * nqt;
    const size_t po_bytes = (size_t)parts * c->kvh * QRP * c->hd * sizeof(float);
    const size_t pm_bytes = (size_t)parts * c->kvh * QRP * 2 * sizeof(float);
    if ((rc = ensure_ws(c, po_bytes + pm_bytes))) return rc;
    // Rows travel in the kernel arguments when they fit, followed by the
    // ranges when those fit too (else the kernel recomputes its range from
    // the rows: <= 64 rows, one per lane); otherwise rows and ranges are
    // staged to the device.
    PlanArg plan_arg;
    const PlanArg *plan = nullptr;
    const AttRow *d_rows = nullptr;
    const int4 *d_ranges = nullptr;
    int ranges_off = -1;
    const size_t rows_bytes = rows.size() * sizeof(AttRow);
    if (rows_bytes <= sizeof(PlanArg)) {
        memcpy(plan_arg.b, rows.data(), rows_bytes);
        if (rows_bytes + ranges.size() * sizeof(int4) <= sizeof(PlanArg)) {
            memcpy(plan_arg.b + rows_bytes, ranges.data(), ranges.size() * sizeof(int4));
            ranges_off = (int)rows_bytes;
        }
        plan = &plan_arg;
    } else {
        Blob b;
        size_t o_r = b.add(rows), o_w = b.add(ranges);
        void *dev;
        if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
        d_rows = (const AttRow *)((char *)dev + o_r);
        d_ranges = (const int4 *)((char *)dev + o_w);
    }
    if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)c->hdu));
    const float qscale = scale * 1.4426950408889634f;
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1))) return rc;
    HIP_TRY(launch_gqa_decode(c->stream, plan, ls.pool0, ls.pool1, c->d_table, d_rows, n_rows,
                              d_ranges, n_ranges, q, q_dtype == RLX_BF16, qo_layout, num_heads,
                              c->kvh, c->hd, c->hdi, c->P, total64, kGqaSnap64, ranges_off, qscale,
                              mask_mode, nqt, (float *)c->ws, (float *)((char *)c->ws + po_bytes),
                              out, out_dtype == RLX_BF16, std::min(max_qr, cap), e0, e1));
    return RLX_OK;
}
}  // namespace

extern "C" {

int32_t rlx_gqa_attend(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                       int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                       int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = check_gqa_attend(c, layer, n_seqs, seq_ids, num_heads, q_dtype, qo_layout,
                                  mask_mode, out_dtype);
    if (rc) return rc;
    if (n_seqs == 0) return RLX_OK;
    if (!q || !out) return fail(RLX_ERR_INVALID, "null q/out");
    return gqa_call_padded(c, gqa_qo_rows(n_seqs, n_q, num_heads), q, q_dtype, out, out_dtype,
                           [&](const void *qk, void *ok) {
                               return gqa_attend_impl(c, layer, n_seqs, seq_ids, n_q, num_heads, qk,
                                                      q_dtype, qo_layout, scale, mask_mode, ok, out_dtype);
                           });
}

int32_t rlx_gqa_append_attend(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                              const int32_t *n_tok, const void *k_src, const void *v_src,
                              int32_t src_dtype, int32_t src_layout, int32_t num_heads,
                              const void *q, int32_t q_dtype, int32_t qo_layout, float scale,
                              int32_t mask_mode, void *out, int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = check_gqa_attend(c, layer, n_seqs, seq_ids, num_heads, q_dtype, qo_layout,
                                  mask_mode, out_dtype);
    if (rc) return rc;
    if (src_dtype != RLX_F32 && src_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "src_dtype");
    if (src_layout != RLX_LAYOUT_HSD && src_layout != RLX_LAYOUT_SHD) return fail(RLX_ERR_INVALID, "src_layout");
    for (int i = 0; i < n_seqs; i++)
        if (!n_tok || n_tok[i] < 1)
            return fail(RLX_ERR_INVALID, "rlx_gqa_append_attend: every sequence appends at least one token");
    if (n_seqs == 0) return RLX_OK;
    if (!q || !out || !k_src || !v_src) return fail(RLX_ERR_INVALID, "null q/out/k/v");
    {
        // the attention's shape limit, checked before anything is appended
        int mx = 0;
        for (int i = 0; i < n_seqs; i++) mx = std::max(mx, n_tok[i]);
        const int Gq = num_heads / c->kvh, cap = gqa_rows_cap(c);
        const bool fa2 = gqa_use_fa2(c, Gq);
        if (Gq * mx > cap && !fa2 && Gq > cap)
            return fail(RLX_ERR_UNSUPPORTED, "heads per kv head = %d with head_dim %d (at most %d)", Gq,
                        c->hdi, cap);
    }
    // Every argument is checked: the append, then the attention of the
    // appended tokens.  (Carrying the append inside the decode launch --
    // the wave that reads a block holding an appended token writing it
    // first -- was measured and not adopted: the writing wave's wait for its
    // stores cost the decode kernel 1.6-2.1 us, against the append launch's
    // 4.4 us, and lowered the kernel's fraction of peak on every call.)
    // (A padded head dim carves the K / V adapter rows with q's and out's,
    // before anything is appended.)
    if ((rc = kv_append_check(c, layer, n_seqs, seq_ids, src_dtype, src_layout))) return rc;
    const int64_t kv_rows = append_rows(c, n_seqs, n_tok);
    const size_t kv_bytes = (size_t)kv_rows * c->hdi * (src_dtype == RLX_BF16 ? 2 : 4);
    char *pad[2] = {nullptr, nullptr};
    return gqa_call_padded(
        c, gqa_qo_rows(n_seqs, n_tok, num_heads), q, q_dtype, out, out_dtype,
        [&](const void *qk, void *ok) {
            int32_t r = kv_append_impl(c, layer, n_seqs, seq_ids, n_tok, k_src, v_src, src_dtype,
                                       src_layout, pad[0] ? pad : nullptr);
            if (r) return r;
            return gqa_attend_impl(c, layer, n_seqs, seq_ids, n_tok, num_heads, qk, q_dtype, qo_layout,
                                   scale, mask_mode, ok, out_dtype);
        },
        c->hdu != c->hdi ? kv_bytes : 0, pad);
}

static int32_t gqa_ref_image_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                                  const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                                  int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                                  int32_t out_dtype) {
    int32_t rc;
    LayerState &ls = c->L[layer];
    const int G = num_heads / c->kvh;
    const int cap = gqa_rows_cap(c);
    if (G > cap)
        return fail(RLX_ERR_UNSUPPORTED, "heads per kv head = %d with head_dim %d (at most %d)", G, c->hdi, cap);
    // The byte image of each sequence, from its appends: scratch pages of
    // the pool's layout, one run of pages per sequence.
    std::vector<RefImgSeq> seqs(n_seqs);
    std::vector<int2> chunks;
    int n_pages = 0, max_len = 0, max_nq = 1;
    for (int i = 0; i < n_seqs; i++) {
        const SeqState &st = ls.seqs[seq_ids[i]];
        int64_t sum = 0;
        for (int32_t n : st.chunks) sum += n;
        if (!st.chunks_ok || st.pos_offset != 0 || sum != st.len)
            return fail(RLX_ERR_STATE,
                        "sequence %d: its tokens are no longer the appends' (evicted, or a rollback cut an "
                        "append), so the reference byte image is undefined",
                        seq_ids[i]);
        if (st.len <= 0) return fail(RLX_ERR_STATE, "sequence %d holds no tokens", seq_ids[i]);
        RefImgSeq &r = seqs[i];
        r = RefImgSeq{};
        r.src_tab = (int32_t)(c->row_base(layer, seq_ids[i]) + st.first);
        r.len = st.len;
        r.chunk0 = (int32_t)chunks.size();
        r.n_chunks = (int32_t)st.chunks.size();
        r.dst_page0 = n_pages;
        int32_t t0 = 0;
        for (int32_t n : st.chunks) {
            chunks.push_back(int2{t0, n});
            t0 += n;
        }
        n_pages += (st.len + c->P - 1) / c->P;
        max_len = std::max(max_len, (int)st.len);
        max_nq = std::max(max_nq, n_q ? n_q[i] : 1);
    }
    // Rows of the decode kernel (query tiles past cap rows per kv head), each
    // pointing at its sequence's scratch pages.
    const int max_qr = G * max_nq;
    const int qtile = max_qr > cap ? cap / G : 0;
    const int nqt = std::min(max_qr, cap) > 16 ? 2 : 1;
    int n_rows = 0;
    if ((rc = gqa_decode_rows(c, layer, n_seqs, seq_ids, n_q, qtile, nullptr, 0, &n_rows))) return rc;
    std::vector<AttRow> rows(n_rows);
    if ((rc = gqa_decode_rows(c, layer, n_seqs, seq_ids, n_q, qtile, rows.data(), n_rows, &n_rows)))
        return rc;
    for (int i = 0, r = 0; i < n_seqs; i++) {  // gqa_decode_rows' order: sequences, then query tiles
        const int nq = n_q ? n_q[i] : 1;
        const int step = qtile > 0 ? qtile : nq;
        for (int q0 = 0; q0 < nq; q0 += step) rows[r++].tab = seqs[i].dst_page0;
    }
    std::vector<int> pre(n_rows + 1), cuts(c->cus + 2);
    std::vector<int4> ranges(c->cus + 1);
    int total64 = 0;
    const int n_ranges = gqa_decode_split(c, rows.data(), n_rows, pre.data(), cuts.data(), ranges.data(),
                                          &total64);
    ranges.resize(n_ranges);
    const int parts = n_rows + n_ranges;
    if ((rc = flush_patches(c))) return rc;
    const int QRP = 16 * nqt;
    const size_t page_bytes = (size_t)c->kvh * c->P * c->hd * 2;
    const size_t img_bytes = ((size_t)n_pages * page_bytes + 255) & ~(size_t)255;
    const size_t tab_bytes = ((size_t)n_pages * 4 + 255) & ~(size_t)255;
    const size_t po_bytes = (size_t)parts * c->kvh * QRP * c->hd * sizeof(float);
    const size_t pm_bytes = (size_t)parts * c->kvh * QRP * 2 * sizeof(float);
    if ((rc = ensure_ws(c, 2 * img_bytes + tab_bytes + po_bytes + pm_bytes))) return rc;
    char *ws = (char *)c->ws;
    uint16_t *dk = (uint16_t *)ws, *dv = (uint16_t *)(ws + img_bytes);
    int32_t *dtable = (int32_t *)(ws + 2 * img_bytes);
    float *po = (float *)(ws + 2 * img_bytes + tab_bytes);
    float *pm = (float *)((char *)po + po_bytes);
    Blob b;
    const size_t o_s = b.add(seqs), o_c = b.add(chunks), o_r = b.add(rows), o_w = b.add(ranges);
    void *dev;
    if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
    HIP_TRY(launch_ref_image_gather(c->stream, ls.pool0, ls.pool1, c->d_table,
                                    (const RefImgSeq *)((char *)dev + o_s), n_seqs, max_len,
                                    (const int2 *)((char *)dev + o_c), c->kvh, c->hd, c->P, dk, dv, dtable,
                                    n_pages));
    if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)c->hdu));
    const float qscale = scale * 1.4426950408889634f;
    HIP_TRY(launch_gqa_decode(c->stream, nullptr, dk, dv, dtable, (const AttRow *)((char *)dev + o_r), n_rows,
                              (const int4 *)((char *)dev + o_w), n_ranges, q, q_dtype == RLX_BF16, qo_layout,
                              num_heads, c->kvh, c->hd, c->hdi, c->P, total64, kGqaSnap64, -1, qscale,
                              mask_mode, nqt, po, pm, out, out_dtype == RLX_BF16, std::min(max_qr, cap),
                              nullptr, nullptr));
    return RLX_OK;
}

int32_t rlx_gqa_attend_ref_image(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                                 const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                                 int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                                 int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = check_gqa_attend(c, layer, n_seqs, seq_ids, num_heads, q_dtype, qo_layout, mask_mode,
                                  out_dtype);
    if (rc) return rc;
    if (n_seqs == 0) return RLX_OK;
    if (!q || !out) return fail(RLX_ERR_INVALID, "null q/out");
    return gqa_call_padded(c, gqa_qo_rows(n_seqs, n_q, num_heads), q, q_dtype, out, out_dtype,
                           [&](const void *qk, void *ok) {
                               return gqa_ref_image_impl(c, layer, n_seqs, seq_ids, n_q, num_heads, qk,
                                                         q_dtype, qo_layout, scale, mask_mode, ok,
                                                         out_dtype);
                           });
}

int32_t rlx_gqa_attend_noalloc(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_q, int32_t num_heads, const void *q, int32_t q_dtype,
                               int32_t qo_layout, float scale, int32_t mask_mode, void *out,
                               int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = check_gqa_attend(c, layer, n_seqs, seq_ids, num_heads, q_dtype, qo_layout,
                                  mask_mode, out_dtype);
    if (rc) return rc;
    if (n_seqs == 0) return RLX_OK;
    if (!q || !out) return fail(RLX_ERR_INVALID, "null q/out");
    if (c->hdu != c->hdi)
        return fail(RLX_ERR_UNSUPPORTED,
                    "rlx_gqa_attend_noalloc: head_dim %d is not a multiple of 8 (its rows would cross "
                    "through adapter memory)", c->hdu);
    void *scr = (c->device >= 0 && c->device < kMaxDevices) ? g_scratch[c->device] : nullptr;
    if (!scr) return fail(RLX_ERR_STATE, "no scratch address for device %d (rlx_init not run)", c->device);
    const int G = num_heads / c->kvh;
    int max_nq = 0;
    for (int i = 0; i < n_seqs; i++) max_nq = std::max(max_nq, n_q ? n_q[i] : 1);
    const int max_qr = G * max_nq;
    // Decode and verify calls only: the FA2 path's work lists are staged.
    const bool fa2 = gqa_use_fa2(c, G);
    const int cap = gqa_rows_cap(c);
    if (max_qr > cap && (fa2 || G > cap))
        return fail(RLX_ERR_UNSUPPORTED,
                    "rlx_gqa_attend_noalloc takes at most %d query rows per kv head (got %d); "
                    "use rlx_gqa_attend", cap, max_qr);
    const int qtile = max_qr > cap ? cap / G : 0;
    const int nqt = std::min(max_qr, cap) > 16 ? 2 : 1;
    // Rows (and ranges when they fit) travel in the kernel arguments.
    constexpr int kRowCap = kPlanArgBytes / (int)sizeof(AttRow);
    constexpr int kRangeCap = 1024;
    AttRow rows[kRowCap];
    int n_rows = 0;
    if ((rc = gqa_decode_rows(c, layer, n_seqs, seq_ids, n_q, qtile, rows, kRowCap, &n_rows))) return rc;
    if (n_rows > kRowCap)
        return fail(RLX_ERR_UNSUPPORTED,
                    "rlx_gqa_attend_noalloc takes at most %d rows (sequences or query tiles), got %d",
                    kRowCap, n_rows);
    if (std::min(c->cus * gqa_wg_per_cu() / c->kvh, c->cus) > kRangeCap)
        return fail(RLX_ERR_UNSUPPORTED, "%d CUs x %d work-groups per CU", c->cus, gqa_wg_per_cu());
    int pre[kRowCap + 1], cuts[kRangeCap + 1];
    int4 ranges[kRangeCap];
    int total64 = 0;
    const int n_ranges = gqa_decode_split(c, rows, n_rows, pre, cuts, ranges, &total64);
    const int QRP = 16 * nqt;
    const size_t parts = (size_t)n_rows + n_ranges;
    const size_t po_bytes = parts * c->kvh * QRP * c->hd * sizeof(float);
    const size_t pm_bytes = parts * c->kvh * QRP * 2 * sizeof(float);
    if (po_bytes + pm_bytes > kNoAllocScratchBytes)
        return fail(RLX_ERR_UNSUPPORTED,
                    "rlx_gqa_attend_noalloc: call needs %zu scratch bytes, the scratch holds %zu",
                    po_bytes + pm_bytes, kNoAllocScratchBytes);
    if ((rc = flush_patches_inline(c))) return rc;
    PlanArg plan;
    const size_t rows_bytes = (size_t)n_rows * sizeof(AttRow);
    memcpy(plan.b, rows, rows_bytes);
    int ranges_off = -1;
    if (rows_bytes + (size_t)n_ranges * sizeof(int4) <= sizeof(PlanArg)) {
        memcpy(plan.b + rows_bytes, ranges, (size_t)n_ranges * sizeof(int4));
        ranges_off = (int)rows_bytes;
    }
    if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)c->hdu));
    HIP_TRY(launch_gqa_decode(c->stream, &plan, c->L[layer].pool0, c->L[layer].pool1, c->d_table,
                              nullptr, n_rows, nullptr, n_ranges, q, q_dtype == RLX_BF16, qo_layout,
                              num_heads, c->kvh, c->hd, c->hdi, c->P, total64, kGqaSnap64, ranges_off,
                              scale * 1.4426950408889634f, mask_mode, nqt, (float *)scr,
                              (float *)((char *)scr + po_bytes), out, out_dtype == RLX_BF16,
                              std::min(max_qr, cap), nullptr, nullptr));
    return RLX_OK;
}

// Whether an MLA call runs as FA2 chunked prefill (latents expanded per
// call) rather than the absorbed decode kernel: past kMlaGroupRowsMax query
// rows (heads x queries) per sequence.  Up to that the absorbed kernel runs
// head groups of 32 rows, each re-reading the sequence's latent rows (1152 B
// per token and group) -- far less than an expansion writes and reads back
// (4 bytes x 128 dims x heads per token) at decode and verify sizes.
// RLX_MLA_FA2_ROWS overrides the bound (tests run both paths on one shape;
// read per call).
constexpr int kMlaGroupRowsMax = 1024;
static bool mla_use_fa2(const Cache *c, int max_qr, int head_dim) {
    (void)c;
    const char *e = getenv("RLX_MLA_FA2_ROWS");
    const int lim = (e && atoi(e) > 0) ? atoi(e) : kMlaGroupRowsMax;
    return max_qr > lim && head_dim <= 256;
}

// Padded head dim of the expanded K_c / V^T rows of an MLA prefill.
static int mla_prefill_dp(int head_dim) { return head_dim <= 128 ? 128 : 256; }

// Heads per expansion of an MLA prefill over tok_off padded tokens: the
// expanded K_c and V^T of hg heads (2 x tok_off x hg x DP bf16) stay within
// the expansion budget and the kernels' 32-bit element offsets.  0: not even
// one head fits.
static int mla_prefill_heads(int64_t tok_off, int num_heads, int dp) {
    const int64_t head_bytes = 2 * tok_off * dp * 2;
    const int64_t hg_budget = mla_expand_budget() / head_bytes;
    const int64_t hg_index = INT32_MAX / (tok_off * dp);
    return (int)std::max<int64_t>(0, std::min<int64_t>({(int64_t)num_heads, hg_budget, hg_index}));
}

// The prefill size check of an MLA call, before anything is appended:
// add_tok[i] tokens are appended to sequence i first (null: none).
static int32_t mla_prefill_check(Cache *c, int layer, int n_seqs, const int32_t *seq_ids,
                                 const int32_t *n_q, const int32_t *add_tok, int num_heads,
                                 int head_dim) {
    int max_nq = 0;
    for (int i = 0; i < n_seqs; i++) max_nq = std::max(max_nq, n_q ? n_q[i] : 1);
    if (!mla_use_fa2(c, num_heads * max_nq, head_dim)) return RLX_OK;
    int64_t tok_off = 0;
    for (int i = 0; i < n_seqs; i++)
        tok_off += ((int64_t)c->L[layer].seqs[seq_ids[i]].len + (add_tok ? add_tok[i] : 0) + 127) / 128 * 128;
    const int dp = mla_prefill_dp(head_dim);
    if (tok_off > 0 && mla_prefill_heads(tok_off, num_heads, dp) < 1)
        return fail(RLX_ERR_UNSUPPORTED,
                    "MLA prefill call too large: one head expands to %lld bytes over %lld tokens",
                    (long long)(2 * tok_off * dp * 2), (long long)tok_off);
    return RLX_OK;
}

// Argument checks of an MLA attention call that change nothing (shared by
// rlx_mla_attend and rlx_mla_append_attend, which checks before appending).
static int32_t mla_attend_check(Cache *c, int32_t n_seqs, const int32_t *n_q, int32_t num_heads,
                                int32_t head_dim, const void *q_nope, const void *q_rope,
                                int32_t q_dtype, const void *w_uk, const void *w_uv,
                                int32_t mask_mode, void *out, int32_t out_dtype) {
    if (num_heads <= 0 || head_dim <= 0 || head_dim > 256)
        return fail(RLX_ERR_UNSUPPORTED, "num_heads=%d head_dim=%d (head_dim 1 to 256)", num_heads, head_dim);
    if (q_dtype != RLX_F32 && q_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "q_dtype");
    if (out_dtype != RLX_F32 && out_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "out_dtype");
    if (mask_mode < RLX_MASK_CAUSAL || mask_mode > RLX_MASK_NONE) return fail(RLX_ERR_INVALID, "mask_mode");
    if (n_seqs == 0) return RLX_OK;
    if (!q_nope || !q_rope || !w_uk || !w_uv || !out) return fail(RLX_ERR_INVALID, "null operand");
    // (Calls of more than 32 query rows per sequence take the FA2 path, which
    // covers every head_dim accepted above.)
    return RLX_OK;
}

// MLA attention after the checks; app: an append to run first, in the
// attention's first launch where the path allows (rlx_mla_append_attend).
static int32_t mla_attend_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                               const int32_t *n_q, int32_t num_heads, int32_t head_dim,
                               const void *q_nope, const void *q_rope, int32_t q_dtype,
                               const void *w_uk, const void *w_uv, float scale, int32_t mask_mode,
                               void *out, int32_t out_dtype, const MlaAppendJob *app) {
    int32_t rc = RLX_OK;
    LayerState &ls = c->L[layer];
    int max_nq = 0;
    for (int i = 0; i < n_seqs; i++) max_nq = std::max(max_nq, n_q ? n_q[i] : 1);
    const int max_qr = num_heads * max_nq;
    if (mla_use_fa2(c, max_qr, head_dim)) {
        if (app)
            HIP_TRY(launch_mla_append(c->stream, app->plan, app->tok_off, app->pool, app->table,
                                      app->patches, app->n_patch, app->toks, app->n_tok, app->c_src,
                                      app->kr_src, app->src_bf16, app->dc, app->dr, app->P));
        // Chunked prefill: expand the latents into per-head K_c / V^T, then
        // FA2 tiles of kPrefillRows query tokens per head.
        std::vector<AttRow> rows;
        std::vector<int2> unused;
        int total_q = 0, mnq = 0, parts = 0;
        if ((rc = build_rows(c, layer, n_seqs, seq_ids, n_q, nullptr, rows, unused, &total_q, &mnq, &parts)))
            return rc;
        std::vector<int2> dwork;
        std::vector<std::vector<int4>> pgroups;
        std::vector<double> pcost;
        int64_t tok_off = 0;
        for (int i = 0; i < n_seqs; i++) {
            const int Tp = (rows[i].len + 127) / 128 * 128;
            rows[i].part = (int32_t)tok_off;  // token offset in the expanded buffers
            rows[i].nsplit = Tp;              // padded length (row pitch of V^T)
            for (int t0 = 0; t0 < Tp; t0 += 128) dwork.push_back(int2{i, t0});
            const int tiles = (rows[i].nq + kPrefillRows - 1) / kPrefillRows;
            for (int h = 0; h < num_heads; h++) {
                pgroups.emplace_back();
                pcost.push_back(0.0);
                for (int qt = tiles - 1; qt >= 0; qt--) {
                    pgroups.back().push_back(int4{i, h, qt, 0});
                    pcost.back() += tile_keys(rows[i], mask_mode, kPrefillRows, qt);
                }
            }
            tok_off += Tp;
        }
        // Heads per expansion (mla_prefill_heads); larger calls run head
        // group by head group (expansion, then FA2 over the group's heads).
        // The entry points refused a call where not one head fits.
        const int dp = mla_prefill_dp(head_dim);
        const int hg = mla_prefill_heads(tok_off, num_heads, dp);
        if (hg < 1) return fail(RLX_ERR_UNSUPPORTED, "MLA prefill call too large");
        const int n_groups = (num_heads + hg - 1) / hg;
        // work items of the group of heads [0, hg) (the xcd order), reused by
        // every group with its heads counted from the group's first
        std::vector<std::vector<int4>> pg_grp;
        std::vector<double> pc_grp;
        for (size_t k = 0; k < pgroups.size(); k++)
            if (pgroups[k][0].y < hg) {
                pg_grp.push_back(pgroups[k]);
                pc_grp.push_back(pcost[k]);
            }
        const std::vector<int4> pwork = xcd_order(pg_grp, pc_grp);
        if ((rc = flush_patches(c))) return rc;
        const size_t w_bytes = (size_t)num_heads * dp * kMlaDc * 2;
        const size_t e_bytes = (size_t)tok_off * hg * dp * 2;
        const size_t r_bytes = (size_t)tok_off * kMlaDr * 2;  // rope keys of the call
        if ((rc = ensure_ws(c, 2 * w_bytes + 2 * e_bytes + r_bytes))) return rc;
        Blob b;
        size_t o_r = b.add(rows), o_d = b.add(dwork), o_p = b.add(pwork);
        void *dev;
        if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
        char *ws = (char *)c->ws;
        uint16_t *wt_k = (uint16_t *)ws, *wt_v = (uint16_t *)(ws + w_bytes);
        uint16_t *kc = (uint16_t *)(ws + 2 * w_bytes), *vt = (uint16_t *)(ws + 2 * w_bytes + e_bytes);
        uint16_t *kr = (uint16_t *)(ws + 2 * w_bytes + 2 * e_bytes);
        const AttRow *drows = (const AttRow *)((char *)dev + o_r);
        HIP_TRY(launch_mla_wt(c->stream, (const uint16_t *)w_uk, (const uint16_t *)w_uv, num_heads, head_dim,
                              c->dc, dp, wt_k, wt_v));
        HIP_TRY(launch_mla_rope_gather(c->stream, ls.pool0, c->d_table, drows,
                                       (const int2 *)((char *)dev + o_d), (int)dwork.size(), c->P, kr));
        if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)(head_dim + c->dr)));
        hipEvent_t e0, e1;
        if ((rc = timing_events(c, &e0, &e1))) return rc;
        for (int g = 0; g < n_groups; g++) {
            const int h0 = g * hg, nh = std::min(hg, num_heads - h0);
            HIP_TRY(launch_mla_expand(c->stream, ls.pool0, c->d_table, drows,
                                      (const int2 *)((char *)dev + o_d), (int)dwork.size(), nh, dp,
                                      c->P, wt_k + (size_t)h0 * dp * kMlaDc,
                                      wt_v + (size_t)h0 * dp * kMlaDc, kc, vt, c->cus));
            PrefillArgs a{};
            a.kc = kc;
            a.vt = vt;
            a.kr = kr;
            a.table = c->d_table;
            a.rows = drows;
            a.work = (const int4 *)((char *)dev + o_p);
            a.q = q_nope;
            a.q2 = q_rope;
            a.out = out;
            a.q_bf16 = q_dtype == RLX_BF16;
            a.layout = RLX_LAYOUT_SHD;
            a.out_bf16 = out_dtype == RLX_BF16;
            a.mask_mode = mask_mode;
            a.H = nh;
            a.KVH = nh;
            a.HQ = num_heads;
            a.h0 = h0;
            a.P = c->P;
            a.pshift = (c->P & (c->P - 1)) == 0 ? __builtin_ctz((unsigned)c->P) : -1;
            a.qscale = scale * 1.4426950408889634f;
            a.qd = head_dim;
            a.qd2 = c->dr;
            a.od = head_dim;
            a.vd = dp;
            a.dv0 = 0;
            // work items of heads >= nh (a last, smaller group) are dropped
            int n_work = (int)pwork.size();
            if (nh < hg) {
                std::vector<int4> part_w;
                for (const int4 &w : pwork)
                    if (w.y < nh) part_w.push_back(w);
                void *dw;
                if ((rc = stage(c, part_w.data(), part_w.size() * sizeof(int4), &dw))) return rc;
                a.work = (const int4 *)dw;
                n_work = (int)part_w.size();
            }
            HIP_TRY(launch_prefill(c->stream, kSrcDense, dp, a, n_work, g == 0 ? e0 : nullptr,
                                   g == n_groups - 1 ? e1 : nullptr));
        }
        return RLX_OK;
    }
    // Decode / verify: one work-group covers at most 32 query rows (heads x
    // queries, query-major: row qi H + h) of a split of a sequence's context.
    // A sequence with more rows is cut into head groups of QRP rows, each a
    // plan row of its own (q0 = its first row, qn = its rows) that re-reads
    // the sequence's latent rows; the merge finds a row's group by index.
    // The host state of app's tokens is committed already: a failure before
    // the launch that carries them still writes them (and their table
    // patches) to the device, so host and device tables stay in agreement.
    auto bail = [&](int32_t r) -> int32_t {
        if (app)
            (void)launch_mla_append(c->stream, app->plan, app->tok_off, app->pool, app->table,
                                    app->patches, app->n_patch, app->toks, app->n_tok, app->c_src,
                                    app->kr_src, app->src_bf16, app->dc, app->dr, app->P);
        return r;
    };
    const int nqt = max_qr > 16 ? 2 : 1;
    const int QRP = 16 * nqt;
    std::vector<AttRow> rows;
    std::vector<int> rlen;
    int total_q = 0, row_nq = 0;
    for (int i = 0; i < n_seqs; i++) {
        const SeqState &st = ls.seqs[seq_ids[i]];
        const int nq = n_q ? n_q[i] : 1;
        if (st.len <= 0) return bail(fail(RLX_ERR_STATE, "sequence %d holds no tokens", seq_ids[i]));
        if (nq < 1 || nq > st.len)
            return bail(fail(RLX_ERR_INVALID, "n_q=%d must be in [1, len=%d]", nq, st.len));
        const int32_t tab = (int32_t)(c->row_base(layer, seq_ids[i]) + st.first);
        const int all = num_heads * nq;
        for (int q0 = 0; q0 < all; q0 += QRP) {
            AttRow r{};
            r.tab = tab;
            r.len = st.len;
            r.nq = nq;
            r.qrow = total_q;
            r.q0 = q0;
            r.qn = std::min(QRP, all - q0);
            rows.push_back(r);
            rlen.push_back(st.len);
        }
        row_nq = std::max(row_nq, nq);
        total_q += nq;
    }
    const int kmask = mask_mode;
    const std::vector<int> nsplit = mla_splits(rlen, (int64_t)c->cus * mla_decode_wgs_per_cu(nqt));
    std::vector<int2> work;
    int parts = 0;
    for (size_t r = 0; r < rows.size(); r++) {
        rows[r].nsplit = nsplit[r];
        rows[r].part = parts;
        parts += nsplit[r];
    }
    // The head groups of a sequence read the same latent rows (equal lengths,
    // equal splits).  Work-group b runs on XCD b mod 8, so split s of every
    // group is placed at the same position mod 8 of consecutive runs of 8
    // work-groups: the groups of a split run on one XCD at about the same
    // time and all but the first find its tiles in that XCD's L2.  (The
    // plan then travels staged: the kernel-argument form derives the work
    // list in row order.)
    const bool grouped = rows.size() > (size_t)n_seqs;
    if (!grouped) {
        for (size_t r = 0; r < rows.size(); r++)
            for (int sp = 0; sp < nsplit[r]; sp++) work.push_back(int2{(int)r, sp});
    } else {
        for (size_t r0 = 0; r0 < rows.size();) {
            size_t r1 = r0;
            while (r1 < rows.size() && rows[r1].qrow == rows[r0].qrow) r1++;  // one sequence's groups
            const int ns = rows[r0].nsplit;
            for (int s0 = 0; s0 < ns; s0 += 8) {
                const int m = std::min(8, ns - s0);
                for (size_t r = r0; r < r1; r++)
                    for (int j = 0; j < m; j++) work.push_back(int2{(int)r, s0 + j});
            }
            r0 = r1;
        }
    }
    if ((rc = flush_patches(c))) return bail(rc);
    const size_t ql_bytes = ((size_t)total_q * num_heads * kMlaRow * 2 + 255) & ~(size_t)255;
    const size_t po_bytes = ((size_t)parts * QRP * kMlaDc * sizeof(uint16_t) + 255) & ~(size_t)255;
    const size_t pm_bytes = ((size_t)parts * QRP * 2 * sizeof(float) + 255) & ~(size_t)255;
    if ((rc = ensure_ws(c, ql_bytes + po_bytes + pm_bytes))) return bail(rc);
    PlanArg plan_arg;
    const PlanArg *plan = nullptr;
    const AttRow *d_rows = nullptr;
    const int2 *d_work = nullptr;
    if (!grouped && rows.size() * sizeof(AttRow) <= sizeof(PlanArg)) {
        memcpy(plan_arg.b, rows.data(), rows.size() * sizeof(AttRow));
        plan = &plan_arg;
    } else {
        Blob b;
        size_t o_r = b.add(rows), o_w = b.add(work);
        void *dev;
        if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return bail(rc);
        d_rows = (const AttRow *)((char *)dev + o_r);
        d_work = (const int2 *)((char *)dev + o_w);
    }
    if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)(head_dim + c->dr)));
    const float qscale = scale * 1.4426950408889634f;
    char *ws = (char *)c->ws;
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1))) return bail(rc);
    HIP_TRY(launch_mla_decode(c->stream, plan, ls.pool0, c->d_table, d_rows, (int)rows.size(), d_work,
                              (int)work.size(), q_nope,
                              q_rope, q_dtype == RLX_BF16, (const uint16_t *)w_uk,
                              (const uint16_t *)w_uv, num_heads, head_dim, c->dc, c->dr, total_q,
                              row_nq, c->P, qscale, kmask, nqt, (uint16_t *)ws,
                              (uint16_t *)(ws + ql_bytes), (float *)(ws + ql_bytes + po_bytes), out,
                              out_dtype == RLX_BF16, c->cus, e0, e1, app));
    return RLX_OK;
}

static int32_t mla_append_attend_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                                      const int32_t *n_tok, const void *c_src, const void *kr_src,
                                      int32_t src_dtype, int32_t num_heads, int32_t head_dim,
                                      const void *q_nope, const void *q_rope, int32_t q_dtype,
                                      const void *w_uk, const void *w_uv, float scale, int32_t mask_mode,
                                      void *out, int32_t out_dtype);

}  // extern "C"

// An MLA attention call through adapter rows when head_dim is not a
// multiple of 8: q_nope [rows][H][D], W_UK and W_UV [d_c][H][D] and out
// cross at the next multiple of 8 (zero dims), with the default scale of
// the caller's head dim.  call(head_dim, q_nope, w_uk, w_uv, out, scale).
template <class F>
static int32_t mla_call_padded(Cache *c, int n_seqs, const int32_t *n_q, int num_heads, int head_dim,
                               const void *q_nope, int32_t q_dtype, const void *w_uk, const void *w_uv,
                               void *out, int32_t out_dtype, float scale, F call) {
    if (head_dim % 8 == 0) return call(head_dim, q_nope, w_uk, w_uv, out, scale);
    const int hp = (head_dim + 7) & ~7;
    if (scale <= 0.f) scale = (float)(1.0 / std::sqrt((double)(head_dim + c->dr)));
    int64_t rows = 0;
    for (int i = 0; i < n_seqs; i++) rows += n_q ? std::max(0, n_q[i]) : 1;
    rows *= num_heads;
    const int64_t wrows = (int64_t)c->dc * num_heads;
    const int qe = q_dtype == RLX_BF16 ? 2 : 4, oe = out_dtype == RLX_BF16 ? 2 : 4;
    const size_t sz[4] = {(size_t)rows * hp * qe, (size_t)wrows * hp * 2, (size_t)wrows * hp * 2,
                          (size_t)rows * hp * oe};
    char *p[4];
    int32_t rc = adapter_regions(c, sz, 4, p);
    if (rc) return rc;
    HIP_TRY(launch_repack_rows(c->stream, q_nope, head_dim, p[0], hp, rows, qe));
    HIP_TRY(launch_repack_rows(c->stream, w_uk, head_dim, p[1], hp, wrows, 2));
    HIP_TRY(launch_repack_rows(c->stream, w_uv, head_dim, p[2], hp, wrows, 2));
    if ((rc = call(hp, (const void *)p[0], (const void *)p[1], (const void *)p[2], (void *)p[3], scale)))
        return rc;
    HIP_TRY(launch_repack_rows(c->stream, p[3], hp, out, head_dim, rows, oe));
    return RLX_OK;
}

extern "C" {

int32_t rlx_mla_attend(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                       const int32_t *n_q, int32_t num_heads, int32_t head_dim, const void *q_nope,
                       const void *q_rope, int32_t q_dtype, const void *w_uk, const void *w_uv,
                       float scale, int32_t mask_mode, void *out, int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kMLA) return fail(RLX_ERR_INVALID, "rlx_mla_attend on a GQA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if ((rc = mla_attend_check(c, n_seqs, n_q, num_heads, head_dim, q_nope, q_rope, q_dtype, w_uk, w_uv,
                               mask_mode, out, out_dtype)))
        return rc;
    if (n_seqs == 0) return RLX_OK;
    const int hk = (head_dim + 7) & ~7;  // the kernels' head dim
    if ((rc = mla_prefill_check(c, layer, n_seqs, seq_ids, n_q, nullptr, num_heads, hk))) return rc;
    return mla_call_padded(c, n_seqs, n_q, num_heads, head_dim, q_nope, q_dtype, w_uk, w_uv, out, out_dtype,
                           scale, [&](int hd, const void *qn, const void *wk, const void *wv, void *o, float sc) {
                               return mla_attend_impl(c, layer, n_seqs, seq_ids, n_q, num_heads, hd, qn,
                                                      q_rope, q_dtype, wk, wv, sc, mask_mode, o, out_dtype,
                                                      nullptr);
                           });
}

int32_t rlx_mla_append_attend(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                              const int32_t *n_tok, const void *c_src, const void *kr_src,
                              int32_t src_dtype, int32_t num_heads, int32_t head_dim,
                              const void *q_nope, const void *q_rope, int32_t q_dtype,
                              const void *w_uk, const void *w_uv, float scale, int32_t mask_mode,
                              void *out, int32_t out_dtype) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (c->kind != kMLA) return fail(RLX_ERR_INVALID, "rlx_mla_append_attend on a GQA cache");
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (src_dtype != RLX_F32 && src_dtype != RLX_BF16) return fail(RLX_ERR_INVALID, "src_dtype");
    for (int i = 0; i < n_seqs; i++)
        if (!n_tok || n_tok[i] < 1)
            return fail(RLX_ERR_INVALID, "rlx_mla_append_attend: every sequence appends at least one token");
    if ((rc = mla_attend_check(c, n_seqs, n_tok, num_heads, head_dim, q_nope, q_rope, q_dtype, w_uk, w_uv,
                               mask_mode, out, out_dtype)))
        return rc;
    if (n_seqs == 0) return RLX_OK;
    if (!c_src || !kr_src) return fail(RLX_ERR_INVALID, "null latent source");
    const int hk = (head_dim + 7) & ~7;  // the kernels' head dim
    if ((rc = mla_prefill_check(c, layer, n_seqs, seq_ids, n_tok, n_tok, num_heads, hk))) return rc;
    return mla_call_padded(c, n_seqs, n_tok, num_heads, head_dim, q_nope, q_dtype, w_uk, w_uv, out,
                           out_dtype, scale,
                           [&](int hd, const void *qn, const void *wk, const void *wv, void *o, float sc) {
                               return mla_append_attend_impl(c, layer, n_seqs, seq_ids, n_tok, c_src, kr_src,
                                                             src_dtype, num_heads, hd, qn, q_rope, q_dtype,
                                                             wk, wv, sc, mask_mode, o, out_dtype);
                           });
}

// rlx_mla_append_attend after its checks: the append (rlx_mla_append), then
// attention of the appended tokens.
static int32_t mla_append_attend_impl(Cache *c, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                                      const int32_t *n_tok, const void *c_src, const void *kr_src,
                                      int32_t src_dtype, int32_t num_heads, int32_t head_dim,
                                      const void *q_nope, const void *q_rope, int32_t q_dtype,
                                      const void *w_uk, const void *w_uv, float scale, int32_t mask_mode,
                                      void *out, int32_t out_dtype) {
    int32_t rc;
    std::vector<AppendTok> toks;
    if ((rc = plan_append(c, layer, n_seqs, seq_ids, n_tok, toks))) return rc;
    std::vector<Patch> patches = take_pending(c);
    PlanArg plan_arg;
    MlaAppendJob job{};
    if ((rc = append_plan(c, patches, toks, &plan_arg, &job.plan, &job.tok_off, &job.patches, &job.toks)))
        return rc;
    job.pool = c->L[layer].pool0;
    job.table = c->d_table;
    job.n_patch = (int)patches.size();
    job.n_tok = (int)toks.size();
    job.c_src = c_src;
    job.kr_src = kr_src;
    job.src_bf16 = src_dtype == RLX_BF16;
    job.dc = c->dc;
    job.dr = c->dr;
    job.P = c->P;
    return mla_attend_impl(c, layer, n_seqs, seq_ids, n_tok, num_heads, head_dim, q_nope, q_rope, q_dtype,
                           w_uk, w_uv, scale, mask_mode, out, out_dtype, &job);
}

static int32_t layer_range(Cache *c, int layer, int *lo, int *hi) {
    int32_t rc = check_layer(c, layer, true);
    if (rc) return rc;
    *lo = layer < 0 ? 0 : layer;
    *hi = layer < 0 ? c->layers : layer + 1;
    return RLX_OK;
}

int32_t rlx_rollback(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                     const int32_t *n_tokens) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (n_seqs > 0 && !n_tokens) return fail(RLX_ERR_INVALID, "null token counts");
    for (int i = 0; i < n_seqs; i++) {
        if (n_tokens[i] < 0) return fail(RLX_ERR_INVALID, "negative rollback");
        for (int l = lo; l < hi; l++)
            if (n_tokens[i] > c->L[l].seqs[seq_ids[i]].len)
                return fail(RLX_ERR_STATE, "rollback of %d tokens of seq %d on layer %d holding %d",
                            n_tokens[i], seq_ids[i], l, c->L[l].seqs[seq_ids[i]].len);
    }
    for (int i = 0; i < n_seqs; i++) {
        const int seq = seq_ids[i];
        for (int l = lo; l < hi; l++) {
            LayerState &ls = c->L[l];
            SeqState &s = ls.seqs[seq];
            s.len -= n_tokens[i];
            for (int n = n_tokens[i]; n > 0;) {  // drop whole appends from the end
                if (s.chunks.empty() || s.chunks.back() > n) {
                    s.chunks_ok = false;
                    break;
                }
                n -= s.chunks.back();
                s.chunks.pop_back();
            }
            const int keep = (s.len + c->P - 1) / c->P;
            for (int k = s.pages - 1; k >= keep; k--) {
                ls.free_stack.push_back(c->entry(l, seq, s.first + k));
                c->set_entry(l, seq, s.first + k, -1);
            }
            s.pages = keep;
        }
    }
    return RLX_OK;
}

int32_t rlx_evict(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids,
                  const int32_t *n_pages) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (n_seqs > 0 && !n_pages) return fail(RLX_ERR_INVALID, "null page counts");
    for (int i = 0; i < n_seqs; i++) {
        if (n_pages[i] < 0) return fail(RLX_ERR_INVALID, "negative eviction");
        for (int l = lo; l < hi; l++)
            if (n_pages[i] > c->L[l].seqs[seq_ids[i]].len / c->P)
                return fail(RLX_ERR_STATE, "evicting %d pages of seq %d on layer %d with %d full pages",
                            n_pages[i], seq_ids[i], l, c->L[l].seqs[seq_ids[i]].len / c->P);
    }
    for (int i = 0; i < n_seqs; i++) {
        const int seq = seq_ids[i];
        for (int l = lo; l < hi; l++) {
            LayerState &ls = c->L[l];
            SeqState &s = ls.seqs[seq];
            // Spilled pages are older than every resident one: once the
            // oldest resident pages are dropped they can no longer be put
            // back in front of the sequence, so they go as well.
            if (n_pages[i] > 0) release_spilled(c, l, seq);
            for (int k = 0; k < n_pages[i]; k++) {
                ls.free_stack.push_back(c->entry(l, seq, s.first + k));
                c->set_entry(l, seq, s.first + k, -1);
            }
            s.first += n_pages[i];
            s.pages -= n_pages[i];
            s.len -= n_pages[i] * c->P;
            s.pos_offset += n_pages[i] * c->P;
        }
    }
    return RLX_OK;
}

int32_t rlx_compact(void *h, int32_t layer) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    for (int l = lo; l < hi; l++) {
        LayerState &ls = c->L[l];
        for (int seq = 0; seq < c->max_seqs; seq++) {
            SeqState &s = ls.seqs[seq];
            if (s.first == 0) continue;
            for (int k = 0; k < s.pages; k++) c->set_entry(l, seq, k, c->entry(l, seq, s.first + k));
            for (int k = s.pages; k < s.first + s.pages; k++) c->set_entry(l, seq, k, -1);
            s.first = 0;
        }
    }
    return RLX_OK;
}

int32_t rlx_spill_attach(void *h, const char *path, int64_t host_pages) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    SpillTier &t = c->spill;
    for (auto &per_layer : t.held)
        for (auto &v : per_layer)
            if (!v.empty()) return fail(RLX_ERR_STATE, "the spill tier still holds pages");
    if (host_pages < 0) return fail(RLX_ERR_INVALID, "host_pages=%lld", (long long)host_pages);
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (t.base) {
        if (t.map_bytes)
            munmap(t.base, t.map_bytes);
        else
            HIP_TRY(hipHostFree(t.base));
    }
    if (t.bounce) HIP_TRY(hipHostFree(t.bounce));
    t = SpillTier{};
    if (host_pages == 0) return RLX_OK;
    const size_t slot_bytes = page_bytes0(c) + page_bytes1(c);
    const size_t bytes = slot_bytes * (size_t)host_pages;
    if (path && *path) {
        const int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
        if (fd < 0) return fail(RLX_ERR_INVALID, "rlx_spill_attach: open %s failed", path);
        void *m = MAP_FAILED;
        if (ftruncate(fd, (off_t)bytes) == 0) m = mmap(nullptr, bytes, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
        close(fd);  // the mapping keeps the file; the caller owns its lifetime
        if (m == MAP_FAILED) return fail(RLX_ERR_INVALID, "rlx_spill_attach: cannot map %zu bytes of %s", bytes, path);
        t.base = (uint8_t *)m;
        t.map_bytes = bytes;
        // The copy kernel cannot address a file mapping: pages pass through
        // a pinned staging buffer of up to 64 MB.
        t.bounce_slots = std::max<int64_t>(1, std::min<int64_t>(host_pages, (64 << 20) / (int64_t)slot_bytes));
        void *b = nullptr;
        HIP_TRY(hipHostMalloc(&b, (size_t)t.bounce_slots * slot_bytes, hipHostMallocDefault));
        t.bounce = (uint8_t *)b;
        void *db = nullptr;
        HIP_TRY(hipHostGetDevicePointer(&db, b, 0));
        t.dev_bounce = (uint8_t *)db;
    } else {
        void *m = nullptr;
        HIP_TRY(hipHostMalloc(&m, bytes, hipHostMallocDefault));
        t.base = (uint8_t *)m;
        void *dm = nullptr;
        HIP_TRY(hipHostGetDevicePointer(&dm, m, 0));
        t.dev_base = (uint8_t *)dm;
    }
    t.slots = host_pages;
    t.slot_bytes = slot_bytes;
    reset_spill(c);
    return RLX_OK;
}

int32_t rlx_spill(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids, const int32_t *n_pages) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    SpillTier &t = c->spill;
    if (!t.base) return fail(RLX_ERR_STATE, "no spill tier attached");
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (n_seqs > 0 && !n_pages) return fail(RLX_ERR_INVALID, "null page counts");
    int64_t need = 0;
    for (int i = 0; i < n_seqs; i++) {
        if (n_pages[i] < 0) return fail(RLX_ERR_INVALID, "negative spill");
        for (int l = lo; l < hi; l++)
            if (n_pages[i] > c->L[l].seqs[seq_ids[i]].len / c->P)
                return fail(RLX_ERR_STATE, "spilling %d pages of seq %d on layer %d with %d full pages",
                            n_pages[i], seq_ids[i], l, c->L[l].seqs[seq_ids[i]].len / c->P);
        need += (int64_t)n_pages[i] * (hi - lo);
    }
    if (need > (int64_t)t.free_stack.size())
        return fail(RLX_ERR_POOL, "spill tier: %lld slots needed, %zu free", (long long)need, t.free_stack.size());
    std::vector<PageMove> mv;
    for (int i = 0; i < n_seqs; i++) {
        const int seq = seq_ids[i];
        for (int l = lo; l < hi; l++) {
            LayerState &ls = c->L[l];
            SeqState &s = ls.seqs[seq];
            for (int k = 0; k < n_pages[i]; k++) {
                const int32_t page = c->entry(l, seq, s.first + k);
                const int64_t slot = t.free_stack.back();
                t.free_stack.pop_back();
                mv.push_back(PageMove{l, page, slot});
                t.held[l][seq].push_back(slot);
                // The page is reused only by later work on this stream, which
                // runs after the copy.
                ls.free_stack.push_back(page);
                c->set_entry(l, seq, s.first + k, -1);
            }
            s.first += n_pages[i];
            s.pages -= n_pages[i];
            s.len -= n_pages[i] * c->P;
            s.pos_offset += n_pages[i] * c->P;
        }
    }
    // (A file tier holds the bytes once this returns: the copies synchronise.)
    return copy_spill_pages(c, mv, true);
}

int32_t rlx_restore(void *h, int32_t layer, int32_t n_seqs, const int32_t *seq_ids, const int32_t *n_pages) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    SpillTier &t = c->spill;
    if (!t.base) return fail(RLX_ERR_STATE, "no spill tier attached");
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    if ((rc = check_seqs(c, n_seqs, seq_ids))) return rc;
    if (n_seqs > 0 && !n_pages) return fail(RLX_ERR_INVALID, "null page counts");
    for (int l = lo; l < hi; l++) {
        int64_t need = 0;
        for (int i = 0; i < n_seqs; i++) {
            const int seq = seq_ids[i];
            const SeqState &s = c->L[l].seqs[seq];
            if (n_pages[i] < 0) return fail(RLX_ERR_INVALID, "negative restore");
            if (n_pages[i] > (int)t.held[l][seq].size())
                return fail(RLX_ERR_STATE, "restoring %d pages of seq %d on layer %d with %zu spilled",
                            n_pages[i], seq, l, t.held[l][seq].size());
            if (std::max(s.first, n_pages[i]) + s.pages > c->max_pages)
                return fail(RLX_ERR_OVERFLOW, "restore of seq %d on layer %d exceeds %d table entries", seq,
                            l, c->max_pages);
            need += n_pages[i];
        }
        for (int i = 0; i < n_seqs; i++)  // a sequence listed twice
            for (int j = 0; j < i; j++)
                if (seq_ids[i] == seq_ids[j]) return fail(RLX_ERR_INVALID, "seq %d listed twice", seq_ids[i]);
        if (need > (int64_t)c->L[l].free_stack.size())
            return fail(RLX_ERR_POOL, "restore needs %lld pages on layer %d, %zu free", (long long)need, l,
                        c->L[l].free_stack.size());
    }
    std::vector<PageMove> mv;
    for (int i = 0; i < n_seqs; i++) {
        const int seq = seq_ids[i], n = n_pages[i];
        if (n == 0) continue;
        for (int l = lo; l < hi; l++) {
            LayerState &ls = c->L[l];
            SeqState &s = ls.seqs[seq];
            if (s.first < n) {  // make room in front: live entries move to [n, n + pages)
                for (int k = s.pages - 1; k >= 0; k--) c->set_entry(l, seq, n + k, c->entry(l, seq, s.first + k));
                for (int k = s.first; k < n && k < s.first + s.pages; k++) c->set_entry(l, seq, k, -1);
                s.first = n;
            }
            auto &held = t.held[l][seq];
            for (int k = n - 1; k >= 0; k--) {  // the newest spilled page first
                const int64_t slot = held.back();
                held.pop_back();
                const int32_t page = ls.free_stack.back();
                ls.free_stack.pop_back();
                c->set_entry(l, seq, s.first - n + k, page);
                mv.push_back(PageMove{l, page, slot});
                t.free_stack.push_back(slot);
            }
            s.first -= n;
            s.pages += n;
            s.len += n * c->P;
            s.pos_offset -= n * c->P;
        }
    }
    // The slots may be handed out again by the next spill, whose copies
    // queue behind these on the same stream.
    return copy_spill_pages(c, mv, false);
}

int32_t rlx_spill_slots(void *h, int32_t layer, int32_t seq, int64_t *slots_out, int32_t cap, int32_t *n_out) {
    if (!h || !n_out) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if (seq < 0 || seq >= c->max_seqs) return fail(RLX_ERR_INVALID, "seq id %d", seq);
    const SpillTier &t = c->spill;
    const int n = t.held.empty() ? 0 : (int)t.held[layer][seq].size();
    *n_out = n;
    if (slots_out)
        for (int k = 0; k < n && k < cap; k++) slots_out[k] = t.held[layer][seq][k];
    return RLX_OK;
}

int32_t rlx_spill_info(void *h, int64_t *info) {
    if (!h || !info) return fail(RLX_ERR_INVALID, "null argument");
    const SpillTier &t = as_cache(h)->spill;
    info[0] = t.slots;
    info[1] = (int64_t)t.slot_bytes;
    info[2] = (int64_t)t.free_stack.size();
    info[3] = t.map_bytes ? 1 : 0;
    return RLX_OK;
}

int32_t rlx_seq_release(void *h, int32_t layer, int32_t seq) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int lo, hi;
    int32_t rc = layer_range(c, layer, &lo, &hi);
    if (rc) return rc;
    if (seq < 0 || seq >= c->max_seqs) return fail(RLX_ERR_INVALID, "seq id %d", seq);
    for (int l = lo; l < hi; l++) {
        LayerState &ls = c->L[l];
        SeqState &s = ls.seqs[seq];
        for (int k = s.pages - 1; k >= 0; k--) {
            ls.free_stack.push_back(c->entry(l, seq, s.first + k));
            c->set_entry(l, seq, s.first + k, -1);
        }
        release_spilled(c, l, seq);
        s = SeqState{};
    }
    return RLX_OK;
}

int32_t rlx_seq_len(void *h, int32_t layer, int32_t seq, int32_t *len_out) {
    if (!h || !len_out) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    // TotalLen returns 0 for an out-of-range layer (kvcache.go:383-388).
    if (layer < 0 || layer >= c->layers || seq < 0 || seq >= c->max_seqs) {
        *len_out = 0;
        return RLX_OK;
    }
    *len_out = c->L[layer].seqs[seq].len;
    return RLX_OK;
}

int32_t rlx_seq_state(void *h, int32_t layer, int32_t seq, int32_t *st) {
    if (!h || !st) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if (seq < 0 || seq >= c->max_seqs) return fail(RLX_ERR_INVALID, "seq id %d", seq);
    const SeqState &s = c->L[layer].seqs[seq];
    st[0] = s.len;
    st[1] = s.first;
    st[2] = s.pos_offset;
    st[3] = s.pages;
    return RLX_OK;
}

int32_t rlx_page_table(void *h, int32_t layer, int32_t seq, int32_t *row_out) {
    if (!h || !row_out) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if (seq < 0 || seq >= c->max_seqs) return fail(RLX_ERR_INVALID, "seq id %d", seq);
    if ((rc = flush_patches(c))) return rc;
    HIP_TRY(hipMemcpyAsync(row_out, c->d_table + c->row_base(layer, seq),
                           (size_t)c->max_pages * sizeof(int32_t), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return RLX_OK;
}

int32_t rlx_free_list(void *h, int32_t layer, int32_t *out, int32_t cap, int32_t *n_out) {
    if (!h || !n_out) return fail(RLX_ERR_INVALID, "null argument");
    Cache *c = as_cache(h);
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    const auto &fs = c->L[layer].free_stack;
    *n_out = (int32_t)fs.size();
    if (out) {
        const int n = std::min<int>(cap, (int)fs.size());
        for (int i = 0; i < n; i++) out[i] = fs[i];
    }
    return RLX_OK;
}

// ---- token selection ------------------------------------------------------

int32_t rlx_greedy(void *h, const float *logits, int32_t n_rows, int32_t vocab, int64_t row_stride,
                   int32_t *out_tokens) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (n_rows < 0 || vocab <= 0 || row_stride < vocab)
        return fail(RLX_ERR_INVALID, "rlx_greedy: n_rows=%d vocab=%d row_stride=%lld", n_rows, vocab,
                    (long long)row_stride);
    if (n_rows == 0) return RLX_OK;
    if (!logits || !out_tokens) return fail(RLX_ERR_INVALID, "rlx_greedy: null pointer");
    int32_t rc = ensure_ws(c, (size_t)n_rows * 4);
    if (rc) return rc;
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1, RLX_TIME_SELECT))) return rc;
    HIP_TRY(launch_greedy(c->stream, logits, row_stride, vocab, n_rows, (int32_t *)c->ws, e0, e1));
    HIP_TRY(hipMemcpyAsync(out_tokens, c->ws, (size_t)n_rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return RLX_OK;
}

int32_t rlx_sample(void *h, const float *logits, int32_t n_rows, int32_t vocab, int64_t row_stride,
                   const rlx_sampler_t *p, const int32_t *prev_tokens, const int32_t *prev_offsets,
                   const float *uniforms, int32_t *out_tokens) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (n_rows < 0 || vocab <= 0 || row_stride < vocab || !p)
        return fail(RLX_ERR_INVALID, "rlx_sample: n_rows=%d vocab=%d row_stride=%lld params=%p",
                    n_rows, vocab, (long long)row_stride, (const void *)p);
    if (n_rows == 0) return RLX_OK;
    if (!logits || !uniforms || !out_tokens) return fail(RLX_ERR_INVALID, "rlx_sample: null pointer");
    // Penalties touch only the distinct tokens of each row's window
    // (sampler.go:213-262): they are counted here and applied on the device.
    const bool pen = prev_offsets && prev_tokens &&
                     ((p->repeat_penalty != 1.f && p->repeat_penalty != 0.f) ||
                      p->frequency_penalty != 0.f || p->presence_penalty != 0.f);
    std::vector<int32_t> st, sf, so;
    if (pen) {
        if (vocab > kSampMaxVocab)
            return fail(RLX_ERR_UNSUPPORTED, "rlx_sample: penalties with vocab %d > %d", vocab,
                        kSampMaxVocab);
        so.push_back(0);
        std::vector<int32_t> w;
        for (int b = 0; b < n_rows; b++) {
            int32_t lo = prev_offsets[b], hi = prev_offsets[b + 1];
            if (lo < 0 || hi < lo) return fail(RLX_ERR_INVALID, "rlx_sample: prev_offsets row %d", b);
            if (p->repeat_window > 0 && hi - lo > p->repeat_window) lo = hi - p->repeat_window;
            w.clear();
            for (int32_t i = lo; i < hi; i++)
                if (prev_tokens[i] >= 0 && prev_tokens[i] < vocab) w.push_back(prev_tokens[i]);
            std::sort(w.begin(), w.end());
            for (size_t i = 0; i < w.size();) {
                size_t j = i;
                while (j < w.size() && w[j] == w[i]) j++;
                st.push_back(w[i]);
                sf.push_back((int32_t)(j - i));
                i = j;
            }
            if ((int)st.size() - so.back() > kSampMaxSeen)
                return fail(RLX_ERR_UNSUPPORTED, "rlx_sample: row %d has %d distinct window tokens (max %d)",
                            b, (int)st.size() - so.back(), kSampMaxSeen);
            so.push_back((int32_t)st.size());
        }
    }
    Blob b;
    const size_t o_u = b.add(std::vector<float>(uniforms, uniforms + n_rows));
    size_t o_t = 0, o_f = 0, o_o = 0;
    if (pen) {
        o_t = b.add(st);
        o_f = b.add(sf);
        o_o = b.add(so);
    }
    void *dev;
    SampleArgs a{};
    a.V = vocab;
    a.top_k = p->top_k;
    const size_t o_split = ((size_t)n_rows * 4 + 255) & ~(size_t)255;
    int32_t rc = ensure_ws(c, o_split + (size_t)plan_sample_split(a, n_rows, nullptr));
    if (rc) return rc;
    plan_sample_split(a, n_rows, (char *)c->ws + o_split);
    if ((rc = stage(c, b.bytes.data(), b.bytes.size(), &dev))) return rc;
    char *d = (char *)dev;
    a.logits = logits;
    a.stride = row_stride;
    a.V = vocab;
    a.temperature = p->temperature;
    a.top_k = p->top_k;
    a.top_p = p->top_p;
    a.min_p = p->min_p;
    a.rp = p->repeat_penalty;
    a.fp = p->frequency_penalty;
    a.pp = p->presence_penalty;
    a.seen_tok = pen ? (const int32_t *)(d + o_t) : nullptr;
    a.seen_freq = pen ? (const int32_t *)(d + o_f) : nullptr;
    a.seen_off = pen ? (const int32_t *)(d + o_o) : nullptr;
    a.u = (const float *)(d + o_u);
    a.out = (int32_t *)c->ws;
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1, RLX_TIME_SELECT))) return rc;
    HIP_TRY(launch_sample(c->stream, a, n_rows, e0, e1));
    HIP_TRY(hipMemcpyAsync(out_tokens, c->ws, (size_t)n_rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return RLX_OK;
}

int32_t rlx_sample_async(void *h, const float *logits, int32_t n_rows, int32_t vocab, int64_t row_stride,
                         const rlx_sampler_t *p, const int32_t *history, int64_t hist_stride,
                         const int32_t *hist_len, const float *uniforms, int32_t *out_tokens) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (n_rows < 0 || vocab <= 0 || row_stride < vocab || !p || hist_stride < 0)
        return fail(RLX_ERR_INVALID, "rlx_sample_async: n_rows=%d vocab=%d row_stride=%lld hist_stride=%lld",
                    n_rows, vocab, (long long)row_stride, (long long)hist_stride);
    if (n_rows == 0) return RLX_OK;
    if (!logits || !uniforms || !out_tokens)
        return fail(RLX_ERR_INVALID, "rlx_sample_async: null pointer");
    const bool pen = history && hist_len &&
                     ((p->repeat_penalty != 1.f && p->repeat_penalty != 0.f) ||
                      p->frequency_penalty != 0.f || p->presence_penalty != 0.f);
    if (pen) {
        if (vocab > kSampMaxVocab)
            return fail(RLX_ERR_UNSUPPORTED, "rlx_sample_async: penalties with vocab %d > %d", vocab,
                        kSampMaxVocab);
        // the longest window a row can have: the last repeat_window entries,
        // or the whole history row when repeat_window <= 0
        const int64_t wmax = p->repeat_window > 0 ? std::min<int64_t>(p->repeat_window, hist_stride)
                                                  : hist_stride;
        if (wmax > kSampMaxSeen)
            return fail(RLX_ERR_UNSUPPORTED,
                        "rlx_sample_async: windows of up to %lld tokens (repeat_window %d, history stride "
                        "%lld); the device count takes at most %d",
                        (long long)wmax, p->repeat_window, (long long)hist_stride, kSampMaxSeen);
    }
    SampleArgs a{};
    a.logits = logits;
    a.stride = row_stride;
    a.V = vocab;
    a.temperature = p->temperature;
    a.top_k = p->top_k;
    a.top_p = p->top_p;
    a.min_p = p->min_p;
    a.rp = p->repeat_penalty;
    a.fp = p->frequency_penalty;
    a.pp = p->presence_penalty;
    a.hist = pen ? history : nullptr;
    a.hist_stride = hist_stride;
    a.hist_len = pen ? hist_len : nullptr;
    a.window = p->repeat_window;
    a.u = uniforms;
    a.out = out_tokens;
    int32_t rc = ensure_ws(c, (size_t)plan_sample_split(a, n_rows, nullptr));
    if (rc) return rc;
    plan_sample_split(a, n_rows, (char *)c->ws);
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1, RLX_TIME_SELECT))) return rc;
    HIP_TRY(launch_sample(c->stream, a, n_rows, e0, e1));
    return RLX_OK;
}

int32_t rlx_spec_accept_async(void *h, const float *draft_logits, const float *target_logits,
                              const int32_t *draft_tokens, const int32_t *n_draft, int32_t n_rows,
                              int32_t max_k, int32_t vocab, const float *uniforms, const rlx_sampler_t *p,
                              int32_t *n_accepted, int32_t *next_token) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (n_rows < 0 || max_k < 0 || vocab <= 0 || !p)
        return fail(RLX_ERR_INVALID, "rlx_spec_accept_async: n_rows=%d max_k=%d vocab=%d", n_rows, max_k,
                    vocab);
    if (n_rows == 0) return RLX_OK;
    if (!target_logits || !n_draft || !uniforms || !n_accepted || !next_token ||
        (max_k > 0 && (!draft_logits || !draft_tokens)))
        return fail(RLX_ERR_INVALID, "rlx_spec_accept_async: null pointer");
    SpecArgs a{};
    a.d_logits = draft_logits;
    a.t_logits = target_logits;
    a.d_tok = draft_tokens;
    a.n_draft = n_draft;
    a.max_k = max_k;
    a.V = vocab;
    a.u = uniforms;
    a.temperature = p->temperature;
    a.top_k = p->top_k;
    a.top_p = p->top_p;
    a.min_p = p->min_p;
    a.n_acc = n_accepted;
    a.next = next_token;
    const int64_t ws_bytes = plan_spec_split(a, n_rows, nullptr);
    if (ws_bytes < 0)
        return fail(RLX_ERR_UNSUPPORTED, "rlx_spec_accept_async: max_k=%d at vocab %d exceeds the grid", max_k,
                    vocab);
    int32_t rc = ensure_ws(c, (size_t)ws_bytes);
    if (rc) return rc;
    plan_spec_split(a, n_rows, (char *)c->ws);
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1, RLX_TIME_SELECT))) return rc;
    HIP_TRY(launch_spec_accept(c->stream, a, n_rows, e0, e1));
    return RLX_OK;
}

int32_t rlx_spec_accept(void *h, const float *draft_logits, const float *target_logits,
                        const int32_t *draft_tokens, const int32_t *n_draft, int32_t n_rows,
                        int32_t max_k, int32_t vocab, const float *uniforms, const rlx_sampler_t *p,
                        int32_t *n_accepted, int32_t *next_token) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    if (n_rows < 0 || max_k < 0 || vocab <= 0 || !p)
        return fail(RLX_ERR_INVALID, "rlx_spec_accept: n_rows=%d max_k=%d vocab=%d", n_rows, max_k, vocab);
    if (n_rows == 0) return RLX_OK;
    if (!target_logits || !n_draft || !uniforms || !n_accepted || !next_token ||
        (max_k > 0 && (!draft_logits || !draft_tokens)))
        return fail(RLX_ERR_INVALID, "rlx_spec_accept: null pointer");
    // Token ids index the logit rows on the device: check them here.
    for (int b = 0; b < n_rows; b++) {
        if (n_draft[b] < 0 || n_draft[b] > max_k)
            return fail(RLX_ERR_INVALID, "rlx_spec_accept: n_draft[%d]=%d outside [0, %d]", b, n_draft[b], max_k);
        for (int i = 0; i < n_draft[b]; i++) {
            const int32_t t = draft_tokens[(int64_t)b * max_k + i];
            if (t < 0 || t >= vocab)
                return fail(RLX_ERR_INVALID, "rlx_spec_accept: draft token %d of row %d = %d outside [0, %d)",
                            i, b, t, vocab);
        }
    }
    Blob bl;
    const size_t o_d = bl.add(std::vector<int32_t>(draft_tokens, draft_tokens + (size_t)n_rows * max_k));
    const size_t o_n = bl.add(std::vector<int32_t>(n_draft, n_draft + n_rows));
    const size_t o_u = bl.add(std::vector<float>(uniforms, uniforms + (size_t)n_rows * (max_k + 1)));
    void *dev;
    SpecArgs a{};
    a.max_k = max_k;
    a.V = vocab;
    a.top_k = p->top_k;
    const size_t o_split = ((size_t)n_rows * 8 + 255) & ~(size_t)255;
    const int64_t split_bytes = plan_spec_split(a, n_rows, nullptr);
    if (split_bytes < 0)
        return fail(RLX_ERR_UNSUPPORTED, "rlx_spec_accept: max_k=%d at vocab %d exceeds the grid", max_k, vocab);
    int32_t rc = ensure_ws(c, o_split + (size_t)split_bytes);
    if (rc) return rc;
    plan_spec_split(a, n_rows, (char *)c->ws + o_split);
    if ((rc = stage(c, bl.bytes.data(), bl.bytes.size(), &dev))) return rc;
    char *d = (char *)dev;
    a.d_logits = draft_logits;
    a.t_logits = target_logits;
    a.d_tok = (const int32_t *)(d + o_d);
    a.n_draft = (const int32_t *)(d + o_n);
    a.max_k = max_k;
    a.V = vocab;
    a.u = (const float *)(d + o_u);
    a.temperature = p->temperature;
    a.top_k = p->top_k;
    a.top_p = p->top_p;
    a.min_p = p->min_p;
    a.n_acc = (int32_t *)c->ws;
    a.next = (int32_t *)c->ws + n_rows;
    hipEvent_t e0, e1;
    if ((rc = timing_events(c, &e0, &e1, RLX_TIME_SELECT))) return rc;
    HIP_TRY(launch_spec_accept(c->stream, a, n_rows, e0, e1));
    HIP_TRY(hipMemcpyAsync(n_accepted, a.n_acc, (size_t)n_rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(next_token, a.next, (size_t)n_rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return RLX_OK;
}

int32_t rlx_pool_ptr(void *h, int32_t layer, void **k_pool, void **v_pool) {
    if (!h) return fail(RLX_ERR_INVALID, "null cache");
    Cache *c = as_cache(h);
    int32_t rc = check_layer(c, layer, false);
    if (rc) return rc;
    if (k_pool) *k_pool = c->L[layer].pool0;
    if (v_pool) *v_pool = c->L[layer].pool1;
    return RLX_OK;
}

}  // extern "C"
