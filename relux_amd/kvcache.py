"""Host-side mirror of relux's cache interface over librelux_kv.

`KVCache` and `MLACache` keep the method names, argument meaning and panic
sites of the reference's Go types (internal/transformer/kvcache.go,
mla_cache.go) and add the paged operations the reference lacks (Rollback,
Evict, Compact, Release) plus the fused attention entry points that replace
the loops of MHA.forwardCached / MLA.forwardCached.  Tensors are torch tensors
on the GPU; the library runs on torch's current stream, so ordering against
torch work is implicit.  Every call goes to the HIP library: there is no CPU
path here.
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import check, i32_array

_MASKS = {"causal": _lib.RLX_MASK_CAUSAL, "ref": _lib.RLX_MASK_REF, "none": _lib.RLX_MASK_NONE}
_LAYOUTS = {"HSD": _lib.RLX_LAYOUT_HSD, "SHD": _lib.RLX_LAYOUT_SHD}
_ROPE = {"offset": _lib.RLX_ROPE_OFFSET, "ref": _lib.RLX_ROPE_REF, "none": _lib.RLX_ROPE_NONE}


def _dtype_code(t):
    if t.dtype == torch.float32:
        return _lib.RLX_F32
    if t.dtype == torch.bfloat16:
        return _lib.RLX_BF16
    raise TypeError(f"unsupported dtype {t.dtype}: use float32 or bfloat16")


def _as_lists(seq, n):
    if isinstance(seq, (list, tuple)):
        seqs = [int(s) for s in seq]
        ns = [int(v) for v in n] if isinstance(n, (list, tuple)) else [int(n)] * len(seqs)
        return seqs, ns
    return [int(seq)], [int(n)]


def _dev(t, what):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{what} must be a GPU torch tensor")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


class _PagedCache:
    def __init__(self, handle, num_layers, page_tokens, max_pages, max_seqs, device):
        self._h = handle
        self.num_layers = num_layers
        self.page_tokens = page_tokens
        self.max_pages = max_pages
        self.max_seqs = max_seqs
        self.device = torch.device("cuda", device)
        self._lib = _lib.load()
        self.use_stream(torch.cuda.current_stream(self.device))

    # -- lifetime ---------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            check(self._lib.rlx_cache_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def use_stream(self, stream):
        """Run this cache's work on `stream` (a torch.cuda.Stream)."""
        check(self._lib.rlx_cache_set_stream(self._h, ctypes.c_void_p(stream.cuda_stream)))

    def Sync(self):
        check(self._lib.rlx_cache_sync(self._h))

    def Reserve(self, workspace_bytes=0, staging_bytes=0, adapter_bytes=0):
        """Grow the device workspace, the plan staging slots and the adapter
        buffer now, so that later calls up to these sizes allocate nothing
        (rlx_cache_reserve)."""
        check(self._lib.rlx_cache_reserve(self._h, int(workspace_bytes), int(staging_bytes),
                                          int(adapter_bytes)))

    def MemoryStats(self):
        """Workspace, staging and adapter capacities and the largest requests
        so far: dict(workspace, workspace_peak, staging, staging_peak,
        adapter, adapter_peak) in bytes."""
        out = (ctypes.c_uint64 * 6)()
        check(self._lib.rlx_cache_memory(self._h, out))
        return dict(workspace=out[0], workspace_peak=out[1], staging=out[2], staging_peak=out[3],
                    adapter=out[4], adapter_peak=out[5])

    def Timing(self, enable=True, kernels="attend"):
        """Bracket every later attention kernel ("attend"), projection
        kernel ("project"), token-selection kernel ("select") or spill /
        restore page copy ("copy") with HIP events."""
        mask = {"attend": _lib.RLX_TIME_ATTEND, "project": _lib.RLX_TIME_PROJECT,
                "select": _lib.RLX_TIME_SELECT, "copy": _lib.RLX_TIME_COPY}[kernels]
        check(self._lib.rlx_cache_timing(self._h, mask if enable else 0))

    def KernelTime(self):
        """(total ms, launches) of the attention kernels timed since the last
        report; synchronises."""
        ms = ctypes.c_float()
        n = ctypes.c_int32()
        check(self._lib.rlx_cache_kernel_time(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    # -- reference method set ---------------------------------------------
    def Reset(self):
        """KVCache.Reset / MLACache.Reset (kvcache.go:174-202): drop every
        sequence, return every page."""
        check(self._lib.rlx_cache_reset(self._h))

    def TotalLen(self, layer_idx, seq=0):
        """Live tokens of `seq` on `layer_idx` (kvcache.go:383-388); 0 for an
        out-of-range layer, as the reference returns."""
        n = ctypes.c_int32()
        check(self._lib.rlx_seq_len(self._h, layer_idx, seq, ctypes.byref(n)))
        return n.value

    def DType(self):
        return "bf16"

    # -- paged operations (no reference counterpart) ------------------------
    def Rollback(self, seq, n_tokens, layer=-1):
        """Drop the last n_tokens of `seq` (int) or, with lists, of every
        listed sequence in one call."""
        seqs, ns = _as_lists(seq, n_tokens)
        check(self._lib.rlx_rollback(self._h, layer, len(seqs), i32_array(seqs), i32_array(ns)))

    def Evict(self, seq, n_pages, layer=-1):
        """Drop the oldest n_pages full pages of `seq` (int or list)."""
        seqs, ns = _as_lists(seq, n_pages)
        check(self._lib.rlx_evict(self._h, layer, len(seqs), i32_array(seqs), i32_array(ns)))

    def Compact(self, layer=-1):
        check(self._lib.rlx_compact(self._h, layer))

    def Release(self, seq, layer=-1):
        check(self._lib.rlx_seq_release(self._h, layer, seq))

    # -- host spill tier (no reference counterpart) --------------------------
    def AttachSpill(self, host_pages, path=None):
        """Attach a host tier of `host_pages` page slots below the HBM pool:
        pinned host memory, or -- with `path` -- a file created at that size
        and mapped MAP_SHARED, as the reference's NewKVCacheFile
        (kvcache.go:95-166) maps its whole cache.  The file is not deleted.
        host_pages 0 detaches."""
        check(self._lib.rlx_spill_attach(self._h, path.encode() if path else None, int(host_pages)))

    def Spill(self, seq, n_pages, layer=-1):
        """Move the oldest n_pages full pages of `seq` (int or list) to the
        host tier; the device state is that of Evict with the same
        arguments."""
        seqs, ns = _as_lists(seq, n_pages)
        check(self._lib.rlx_spill(self._h, layer, len(seqs), i32_array(seqs), i32_array(ns)))

    def Restore(self, seq, n_pages, layer=-1):
        """Put the n_pages most recently spilled pages of `seq` back in
        front of it (bytes and positions as before the spill)."""
        seqs, ns = _as_lists(seq, n_pages)
        check(self._lib.rlx_restore(self._h, layer, len(seqs), i32_array(seqs), i32_array(ns)))

    def SpilledSlots(self, layer, seq):
        """Tier slots of (layer, seq)'s spilled pages, oldest first."""
        n = ctypes.c_int32()
        check(self._lib.rlx_spill_slots(self._h, layer, seq, None, 0, ctypes.byref(n)))
        out = (ctypes.c_int64 * max(n.value, 1))()
        check(self._lib.rlx_spill_slots(self._h, layer, seq, out, n.value, ctypes.byref(n)))
        return list(out[:n.value])

    def SpillInfo(self):
        """{slots, slot_bytes, free, file} of the host tier."""
        info = (ctypes.c_int64 * 4)()
        check(self._lib.rlx_spill_info(self._h, info))
        return {"slots": info[0], "slot_bytes": info[1], "free": info[2], "file": bool(info[3])}

    # -- state dumps ---------------------------------------------------------
    def SeqState(self, layer, seq):
        st = (ctypes.c_int32 * 4)()
        check(self._lib.rlx_seq_state(self._h, layer, seq, st))
        return {"len": st[0], "first": st[1], "pos_offset": st[2], "pages": st[3]}

    def PageTable(self, layer, seq):
        row = (ctypes.c_int32 * self.max_pages)()
        check(self._lib.rlx_page_table(self._h, layer, seq, row))
        return list(row)

    def FreeList(self, layer):
        n = ctypes.c_int32()
        check(self._lib.rlx_free_list(self._h, layer, None, 0, ctypes.byref(n)))
        buf = (ctypes.c_int32 * max(1, n.value))()
        check(self._lib.rlx_free_list(self._h, layer, buf, n.value, ctypes.byref(n)))
        return list(buf)[: n.value]

    def OutProject(self, x, w_packed, n_out, residual=None, out=None, out_dtype=None):
        """The step after attention on this cache's stream: out = x . W
        (+ residual) -- the output projection (mha.go:356-360, mla.go:384-389)
        and the block's residual add.  x [rows][k_in] f32 or bf16 (device),
        w_packed from pack_out, residual None or [rows][n_out] in out's dtype."""
        rows, k_in = x.shape[0], x.shape[-1]
        if out is None:
            dt = out_dtype or (residual.dtype if residual is not None else torch.float32)
            out = torch.empty((rows, n_out), dtype=dt, device=x.device)
        if residual is not None and (residual.dtype != out.dtype or residual.shape[-1] != n_out):
            raise ValueError("residual must be [rows][n_out] in the output dtype")
        check(self._lib.rlx_out_project(self._h, rows, _dev(x, "x"), _dtype_code(x), k_in,
                                        _dev(w_packed, "w_packed"), n_out,
                                        _dev(residual, "residual") if residual is not None else None,
                                        _dev(out, "out"), _dtype_code(out)))
        return out

    def _lens(self, layer_idx, seq_ids):
        return [self.TotalLen(layer_idx, s) for s in seq_ids]


class KVCache(_PagedCache):
    """Paged bf16 GQA K/V cache.

    KVCache(num_layers, max_len, num_kv_heads, head_dim) mirrors
    NewKVCacheSized(numLayers, maxLen, numKVHeads, headDim, BFloat16)
    (kvcache.go:66-93): every sequence may hold max_len tokens.  Pages of
    `page_tokens` tokens come from a per-layer pool of `pool_pages` pages
    (default: enough for max_seqs full sequences).
    """

    def __init__(self, num_layers, max_len, num_kv_heads, head_dim, page_tokens=16, max_seqs=1,
                 pool_pages=None, device=0):
        _lib.init(device)
        if num_layers <= 0:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID,
                                  f"NewKVCacheSized: numLayers={num_layers}, must be > 0")
        if max_len <= 0:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID,
                                  f"NewKVCacheSized: maxLen={max_len}, must be > 0")
        max_pages = -(-max_len // page_tokens)
        if pool_pages is None:
            pool_pages = max_pages * max_seqs
        h = ctypes.c_void_p()
        check(_lib.load().rlx_kv_create(num_layers, num_kv_heads, head_dim, page_tokens, pool_pages,
                                        max_seqs, max_pages, ctypes.byref(h)))
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.pool_pages = pool_pages
        super().__init__(h, num_layers, page_tokens, max_pages, max_seqs, device)

    def Append(self, layer_idx, new_k, new_v, seq_ids=(0,), n_tok=None, layout="HSD"):
        """Append K/V rows (kvcache.go:240-316).  With one sequence and the
        reference's [1, KVH, n, D] tensors this is KVCache.Append; with
        several, n_tok[i] rows per sequence in `layout` order."""
        if new_k.shape != new_v.shape:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID,
                                  f"KVCache.Append: K and V shape mismatch: {tuple(new_k.shape)} vs {tuple(new_v.shape)}")
        if new_k.dtype != new_v.dtype:
            raise TypeError("K and V dtypes differ")
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [new_k.shape[-2] if layout == "HSD" else new_k.shape[-3]]
        total = sum(n_tok)
        if new_k.numel() != total * self.num_kv_heads * self.head_dim:
            raise ValueError(f"K holds {new_k.numel()} elements, expected "
                             f"{total}x{self.num_kv_heads}x{self.head_dim}")
        check(self._lib.rlx_kv_append(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                      i32_array(n_tok), _dev(new_k, "K"), _dev(new_v, "V"),
                                      _dtype_code(new_k), _LAYOUTS[layout]))

    def View(self, layer_idx, seq=0):
        """Dense bf16 (K, V) of one sequence, each [1, KVH, T, D], gathered
        through the page table (kvcache.go:363-380).  None, None when empty."""
        T = self.TotalLen(layer_idx, seq)
        if not 0 <= layer_idx < self.num_layers:
            raise _lib.ReluxPanic(_lib.RLX_ERR_LAYER, f"KVCache.View: layerIdx={layer_idx} out of range")
        if T == 0:
            return None, None
        k = torch.empty((1, self.num_kv_heads, T, self.head_dim), dtype=torch.bfloat16, device=self.device)
        v = torch.empty_like(k)
        check(self._lib.rlx_kv_gather(self._h, layer_idx, 1, i32_array([seq]), _dev(k, "k"), _dev(v, "v")))
        return k, v

    def Gather(self, layer_idx, seq_ids, k_out, v_out):
        """Gather several sequences into caller-owned dense buffers
        ([KVH][T_i][D] per sequence, concatenated)."""
        check(self._lib.rlx_kv_gather(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                      _dev(k_out, "k_out"), _dev(v_out, "v_out")))

    def Attend(self, layer_idx, q, num_heads, seq_ids=(0,), n_q=None, layout="SHD", scale=None,
               mask="causal", out=None, out_dtype=torch.float32):
        """Attention of n_q[i] query rows per sequence over its cached tokens
        (mha.go:291-348).  q: rows x num_heads x head_dim in `layout`."""
        seq_ids = list(seq_ids)
        if n_q is None:
            n_q = [1] * len(seq_ids)
        rows = sum(n_q)
        if q.numel() != rows * num_heads * self.head_dim:
            raise ValueError("q size does not match sum(n_q) x num_heads x head_dim")
        if out is None:
            out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
        check(self._lib.rlx_gqa_attend(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                       i32_array(n_q), num_heads, _dev(q, "q"), _dtype_code(q),
                                       _LAYOUTS[layout], float(scale or 0.0), _MASKS[mask],
                                       _dev(out, "out"), _dtype_code(out)))
        return out

    def AppendAttend(self, layer_idx, new_k, new_v, q, num_heads, seq_ids=(0,), n_tok=None,
                     kv_layout="SHD", layout="SHD", scale=None, mask="causal", out=None,
                     out_dtype=torch.float32):
        """The cache half of MHA.forwardCached (mha.go:283-348): Append the
        n_tok[i] new tokens' K/V rows (in `kv_layout`), then Attend with
        those tokens as the queries (n_q = n_tok), in one library call.  Same
        bytes and outputs as the two calls."""
        if new_k.shape != new_v.shape:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID,
                                  f"KVCache.Append: K and V shape mismatch: {tuple(new_k.shape)} vs {tuple(new_v.shape)}")
        if new_k.dtype != new_v.dtype:
            raise TypeError("K and V dtypes differ")
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [new_k.shape[-2] if kv_layout == "HSD" else new_k.shape[-3]]
        total = sum(n_tok)
        if new_k.numel() != total * self.num_kv_heads * self.head_dim:
            raise ValueError(f"K holds {new_k.numel()} elements, expected "
                             f"{total}x{self.num_kv_heads}x{self.head_dim}")
        if q.numel() != total * num_heads * self.head_dim:
            raise ValueError("q size does not match sum(n_tok) x num_heads x head_dim")
        if out is None:
            out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
        check(self._lib.rlx_gqa_append_attend(
            self._h, layer_idx, len(seq_ids), i32_array(seq_ids), i32_array(n_tok), _dev(new_k, "K"),
            _dev(new_v, "V"), _dtype_code(new_k), _LAYOUTS[kv_layout], num_heads, _dev(q, "q"),
            _dtype_code(q), _LAYOUTS[layout], float(scale or 0.0), _MASKS[mask], _dev(out, "out"),
            _dtype_code(out)))
        return out

    def AttendRefImage(self, layer_idx, q, num_heads, seq_ids=(0,), n_q=None, layout="SHD", scale=None,
                       mask="ref", out=None, out_dtype=torch.float32):
        """Attend over the keys and values as the reference KVCache holds
        them (rlx_gqa_attend_ref_image): each Append's [KVH, S, D] block laid
        out raw (kvcache.go:286-287, 407-423) and read head-major with stride
        totalLen (mha.go:305-310) -- relux's own decode outputs, mask rule
        RLX_MASK_REF by default.  Raises for sequences that were evicted or
        rolled back into the middle of an append."""
        seq_ids = list(seq_ids)
        if n_q is None:
            n_q = [1] * len(seq_ids)
        if q.numel() != sum(n_q) * num_heads * self.head_dim:
            raise ValueError("q size does not match sum(n_q) x num_heads x head_dim")
        if out is None:
            out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
        check(self._lib.rlx_gqa_attend_ref_image(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                                 i32_array(n_q), num_heads, _dev(q, "q"), _dtype_code(q),
                                                 _LAYOUTS[layout], float(scale or 0.0), _MASKS[mask],
                                                 _dev(out, "out"), _dtype_code(out)))
        return out

    def AttendNoAlloc(self, layer_idx, q, num_heads, out, seq_ids=(0,), n_q=None, layout="SHD",
                      scale=None, mask="causal"):
        """Attend for decode / verify calls through rlx_gqa_attend_noalloc:
        the library allocates nothing (split partials in its fixed per-device
        scratch).  The caller provides `out`.  Same results as Attend."""
        seq_ids = list(seq_ids)
        if n_q is None:
            n_q = [1] * len(seq_ids)
        if q.numel() != sum(n_q) * num_heads * self.head_dim or out.numel() != q.numel():
            raise ValueError("q / out size does not match sum(n_q) x num_heads x head_dim")
        check(self._lib.rlx_gqa_attend_noalloc(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                               i32_array(n_q), num_heads, _dev(q, "q"),
                                               _dtype_code(q), _LAYOUTS[layout],
                                               float(scale or 0.0), _MASKS[mask], _dev(out, "out"),
                                               _dtype_code(out)))
        return out


    def ProjectAppend(self, layer_idx, x, w_packed, num_heads, rope=None, seq_ids=(0,), n_tok=None,
                      rope_mode="offset", q_dtype=torch.float32):
        """Fused pre-attention step (mha.go:250-289): q/k/v projection of the
        new tokens' hidden states x [sum n][d_model] with weights packed by
        pack_qkv, RoPE of q and k (rope = (cos, sin) tables from rope_tables),
        append of k and v.  Returns the rotated q [sum n][num_heads][head_dim]."""
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [x.shape[0]]
        rows, d_model = x.shape[0], x.shape[-1]
        if rows != sum(n_tok):
            raise ValueError("x rows do not match sum(n_tok)")
        q = torch.empty((rows, num_heads, self.head_dim), dtype=q_dtype, device=x.device)
        if rope is None:
            rope_mode = "none"
            cos_t = sin_t = None
            rope_rows = 0
        else:
            cos_t, sin_t = rope
            rope_rows = cos_t.shape[0]
        check(self._lib.rlx_gqa_project_append(
            self._h, layer_idx, len(seq_ids), i32_array(seq_ids), i32_array(n_tok), _dev(x, "x"),
            _dtype_code(x), d_model, _dev(w_packed, "w_packed"), num_heads,
            _dev(cos_t, "rope_cos") if cos_t is not None else None,
            _dev(sin_t, "rope_sin") if sin_t is not None else None, rope_rows, _ROPE[rope_mode],
            _dev(q, "q_out"), _dtype_code(q)))
        return q


def gqa_pack_width(num_heads, kv_heads, head_dim):
    """Packed features per head of pack_qkv: head_dim when H*D and KVH*D are
    multiples of 16, else head_dim rounded up to 16 (zero weights past it)."""
    if (num_heads * head_dim) % 16 == 0 and (kv_heads * head_dim) % 16 == 0:
        return head_dim
    return -(-head_dim // 16) * 16


def pack_qkv(w_q, w_k, w_v, num_heads, kv_heads, head_dim):
    """W_q [d_model][H*D], W_k/W_v [d_model][KVH*D] (bf16 or f32, device) ->
    packed bf16 weights for KVCache.ProjectAppend: N = (H + 2 KVH) * W
    features (W = gqa_pack_width) in 16-feature x 32-k fragments
    (rlx_pack_qkv)."""
    d_model = w_q.shape[0]
    W = gqa_pack_width(num_heads, kv_heads, head_dim)
    out = torch.empty(((num_heads + 2 * kv_heads) * W, -(-d_model // 32) * 32), dtype=torch.bfloat16,
                      device=w_q.device)
    check(_lib.load().rlx_pack_qkv(_dev(w_q, "w_q"), _dev(w_k, "w_k"), _dev(w_v, "w_v"),
                                   _dtype_code(w_q), d_model, num_heads, kv_heads, head_dim,
                                   _dev(out, "out")))
    return out


def pack_out(w, k_in=None, n_out=None):
    """W [k_in][n_out] (bf16 or f32, device; e.g. W_O [H*D][d_model]) ->
    packed bf16 weights for OutProject (rlx_pack_out)."""
    k_in = k_in or w.shape[0]
    n_out = n_out or w.shape[1]
    out = torch.empty((-(-n_out // 16) * 16, -(-k_in // 32) * 32), dtype=torch.bfloat16, device=w.device)
    check(_lib.load().rlx_pack_out(_dev(w, "w"), _dtype_code(w), k_in, n_out, _dev(out, "out")))
    return out


def rope_tables(head_dim, base, max_seq, device):
    """RotaryEmbedding tables (rope.go:50-75): theta_i = f32(1/f32(base^(2i/d))),
    angle = f32(pos * theta) in f64, cos/sin in f64 rounded to f32.  Returns
    device f32 (cos, sin), each [max_seq][head_dim/2]."""
    import numpy as np
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    p = np.power(np.float64(np.float32(base)), 2.0 * i / head_dim).astype(np.float32)
    theta = (np.float32(1.0) / p).astype(np.float32)
    pos = np.arange(max_seq, dtype=np.float64)[:, None]
    angle = (pos * theta.astype(np.float64)[None, :]).astype(np.float32)
    cos_t = np.cos(angle.astype(np.float64)).astype(np.float32)
    sin_t = np.sin(angle.astype(np.float64)).astype(np.float32)
    return (torch.from_numpy(cos_t).to(device), torch.from_numpy(sin_t).to(device))


class MLACache(_PagedCache):
    """Paged bf16 MLA latent cache (c^KV | k^R per token).

    MLACache(num_layers, max_len, d_c, d_r) mirrors NewMLACache(numLayers,
    maxLen, dC, dHR) (mla_cache.go:38-59); storage is bf16 instead of f32.
    """

    def __init__(self, num_layers, max_len, d_c=512, d_r=64, page_tokens=64, max_seqs=1,
                 pool_pages=None, device=0):
        _lib.init(device)
        if num_layers <= 0:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID, f"NewMLACache: numLayers={num_layers}, must be > 0")
        if max_len <= 0:
            raise _lib.ReluxPanic(_lib.RLX_ERR_INVALID, f"NewMLACache: maxLen={max_len}, must be > 0")
        max_pages = -(-max_len // page_tokens)
        if pool_pages is None:
            pool_pages = max_pages * max_seqs
        h = ctypes.c_void_p()
        check(_lib.load().rlx_mla_create(num_layers, d_c, d_r, page_tokens, pool_pages, max_seqs,
                                         max_pages, ctypes.byref(h)))
        self.d_c = d_c
        self.d_r = d_r
        self.pool_pages = pool_pages
        super().__init__(h, num_layers, page_tokens, max_pages, max_seqs, device)

    def Append(self, layer_idx, new_c, new_kr, seq_ids=(0,), n_tok=None):
        """Append latent rows (mla_cache.go:152-182): new_c [.., n, d_c],
        new_kr [.., n, d_r] (post-RoPE)."""
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [new_c.shape[-2]]
        total = sum(n_tok)
        if new_c.numel() != total * self.d_c or new_kr.numel() != total * self.d_r:
            raise ValueError("latent / rope-key sizes do not match sum(n_tok)")
        if new_c.dtype != new_kr.dtype:
            raise TypeError("c and kr dtypes differ")
        check(self._lib.rlx_mla_append(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                       i32_array(n_tok), _dev(new_c, "c"), _dev(new_kr, "kr"),
                                       _dtype_code(new_c)))

    def ProjectAppend(self, layer_idx, x, w_packed, num_heads, head_dim, rope=None, seq_ids=(0,),
                      n_tok=None, rope_mode="offset", q_dtype=torch.float32):
        """Fused pre-attention step of an MLA layer (mla.go:279-314): q_c, q_r,
        c^KV, k^R projections of x [sum n][d_model] with weights packed by
        pack_mla_proj, RoPE of q_r and k^R (rope = (cos, sin) tables for
        d_r), append of the latent rows.  Returns (q_nope [sum n][H][D],
        q_rope [sum n][H][d_r]) for Attend."""
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [x.shape[0]]
        rows, d_model = x.shape[0], x.shape[-1]
        if rows != sum(n_tok):
            raise ValueError("x rows do not match sum(n_tok)")
        qn = torch.empty((rows, num_heads, head_dim), dtype=q_dtype, device=x.device)
        qr = torch.empty((rows, num_heads, self.d_r), dtype=q_dtype, device=x.device)
        if rope is None:
            rope_mode, cos_t, sin_t, rope_rows = "none", None, None, 0
        else:
            cos_t, sin_t = rope
            rope_rows = cos_t.shape[0]
        check(self._lib.rlx_mla_project_append(
            self._h, layer_idx, len(seq_ids), i32_array(seq_ids), i32_array(n_tok), _dev(x, "x"),
            _dtype_code(x), d_model, _dev(w_packed, "w_packed"), num_heads, head_dim,
            _dev(cos_t, "rope_cos") if cos_t is not None else None,
            _dev(sin_t, "rope_sin") if sin_t is not None else None, rope_rows, _ROPE[rope_mode],
            _dev(qn, "q_nope"), _dev(qr, "q_rope"), _dtype_code(qn)))
        return qn, qr

    def View(self, layer_idx, seq=0):
        """Dense bf16 (c [1, T, d_c], kr [1, T, d_r]) (mla_cache.go:222-233)."""
        if not 0 <= layer_idx < self.num_layers:
            raise _lib.ReluxPanic(_lib.RLX_ERR_LAYER, f"MLACache.View: layerIdx={layer_idx} out of range")
        T = self.TotalLen(layer_idx, seq)
        if T == 0:
            return None, None
        c = torch.empty((1, T, self.d_c), dtype=torch.bfloat16, device=self.device)
        kr = torch.empty((1, T, self.d_r), dtype=torch.bfloat16, device=self.device)
        check(self._lib.rlx_mla_gather(self._h, layer_idx, 1, i32_array([seq]), _dev(c, "c"), _dev(kr, "kr")))
        return c, kr

    def Attend(self, layer_idx, q_nope, q_rope, w_uk, w_uv, num_heads, head_dim, seq_ids=(0,),
               n_q=None, scale=None, mask="causal", out=None, out_dtype=torch.float32):
        """Absorbed MLA attention of n_q[i] query rows per sequence
        (mla.go:316-377).  q_nope [rows, H, D], q_rope [rows, H, d_r],
        w_uk / w_uv bf16 [d_c, H*D]; returns [rows, H, D]."""
        seq_ids = list(seq_ids)
        if n_q is None:
            n_q = [1] * len(seq_ids)
        rows = sum(n_q)
        if q_nope.numel() != rows * num_heads * head_dim or q_rope.numel() != rows * num_heads * self.d_r:
            raise ValueError("query sizes do not match sum(n_q) x heads")
        if w_uk.dtype != torch.bfloat16 or w_uv.dtype != torch.bfloat16:
            raise TypeError("W_UK / W_UV must be bf16 (optim.Param.Data is bf16)")
        if w_uk.numel() != self.d_c * num_heads * head_dim or w_uv.numel() != w_uk.numel():
            raise ValueError("W_UK / W_UV must be [d_c, num_heads*head_dim]")
        if out is None:
            out = torch.empty((rows, num_heads, head_dim), dtype=out_dtype, device=q_nope.device)
        if q_nope.dtype != q_rope.dtype:
            raise TypeError("q_nope and q_rope dtypes differ")
        check(self._lib.rlx_mla_attend(self._h, layer_idx, len(seq_ids), i32_array(seq_ids),
                                       i32_array(n_q), num_heads, head_dim, _dev(q_nope, "q_nope"),
                                       _dev(q_rope, "q_rope"), _dtype_code(q_nope),
                                       _dev(w_uk, "w_uk"), _dev(w_uv, "w_uv"), float(scale or 0.0),
                                       _MASKS[mask], _dev(out, "out"), _dtype_code(out)))
        return out

    def AppendAttend(self, layer_idx, new_c, new_kr, q_nope, q_rope, w_uk, w_uv, num_heads,
                     head_dim, seq_ids=(0,), n_tok=None, scale=None, mask="causal", out=None,
                     out_dtype=torch.float32):
        """The cache half of MLA.forwardCached (mla.go:308-377): Append the
        n_tok[i] new tokens' latent rows, then Attend with those tokens as the
        queries (n_q = n_tok).  Same bytes and outputs as the two calls; on
        the decode path the append rides in the attention's first launch."""
        seq_ids = list(seq_ids)
        if n_tok is None:
            if len(seq_ids) != 1:
                raise ValueError("n_tok is required for several sequences")
            n_tok = [new_c.shape[-2]]
        total = sum(n_tok)
        if new_c.numel() != total * self.d_c or new_kr.numel() != total * self.d_r:
            raise ValueError("latent / rope-key sizes do not match sum(n_tok)")
        if new_c.dtype != new_kr.dtype:
            raise TypeError("c and kr dtypes differ")
        if q_nope.numel() != total * num_heads * head_dim or q_rope.numel() != total * num_heads * self.d_r:
            raise ValueError("query sizes do not match sum(n_tok) x heads")
        if w_uk.dtype != torch.bfloat16 or w_uv.dtype != torch.bfloat16:
            raise TypeError("W_UK / W_UV must be bf16 (optim.Param.Data is bf16)")
        if w_uk.numel() != self.d_c * num_heads * head_dim or w_uv.numel() != w_uk.numel():
            raise ValueError("W_UK / W_UV must be [d_c, num_heads*head_dim]")
        if q_nope.dtype != q_rope.dtype:
            raise TypeError("q_nope and q_rope dtypes differ")
        if out is None:
            out = torch.empty((total, num_heads, head_dim), dtype=out_dtype, device=q_nope.device)
        check(self._lib.rlx_mla_append_attend(
            self._h, layer_idx, len(seq_ids), i32_array(seq_ids), i32_array(n_tok), _dev(new_c, "c"),
            _dev(new_kr, "kr"), _dtype_code(new_c), num_heads, head_dim, _dev(q_nope, "q_nope"),
            _dev(q_rope, "q_rope"), _dtype_code(q_nope), _dev(w_uk, "w_uk"), _dev(w_uv, "w_uv"),
            float(scale or 0.0), _MASKS[mask], _dev(out, "out"), _dtype_code(out)))
        return out


def pack_mla_proj(w_q, w_qr, w_dkv, w_kr, num_heads, head_dim):
    """W_Q [d_model][H*D], W_QR [d_model][H*d_r], W_DKV [d_model][d_c], W_KR
    [d_model][d_r] (bf16 or f32, device) -> packed bf16 weights for
    MLACache.ProjectAppend (rlx_pack_mla_proj); d_r and d_c features are
    padded to multiples of 16 with zero columns, and the q_c heads too when
    H*D is not one."""
    d_model = w_q.shape[0]
    d_c, d_r = w_dkv.shape[1], w_kr.shape[1]
    drp, dcp = -(-d_r // 16) * 16, -(-d_c // 16) * 16
    qw = head_dim if (num_heads * head_dim) % 16 == 0 else -(-head_dim // 16) * 16
    n = num_heads * (qw + drp) + dcp + drp
    out = torch.empty((n, -(-d_model // 32) * 32), dtype=torch.bfloat16, device=w_q.device)
    check(_lib.load().rlx_pack_mla_proj(_dev(w_q, "w_q"), _dev(w_qr, "w_qr"), _dev(w_dkv, "w_dkv"),
                                        _dev(w_kr, "w_kr"), _dtype_code(w_q), d_model, num_heads,
                                        head_dim, d_c, d_r, _dev(out, "out")))
    return out


def default_scale(head_dim, d_r=0):
    """f32(1/sqrt(f64(D + dR))) as the reference computes it (mha.go:319,
    mla.go:339-340)."""
    return float(torch.tensor(1.0 / math.sqrt(head_dim + d_r), dtype=torch.float32))
