"""ctypes binding of librelux_kv.so (the C ABI declared in include/relux_kv.h).

The library is loaded from this package directory.  There is no fallback:
if it is missing the import fails with instructions to build it.  torch is
imported first so that the library binds to the HIP runtime torch already
loaded (both carry the soname libamdhip64.so.7): device pointers and streams
are then shared between torch tensors and the library.
"""
import ctypes
import os

try:  # torch provides device memory and streams to the Python host layer
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - the C ABI itself does not need torch
    torch = None

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librelux_kv.so")

RLX_OK = 0
RLX_ERR_INVALID = -1
RLX_ERR_OVERFLOW = -2
RLX_ERR_POOL = -3
RLX_ERR_LAYER = -4
RLX_ERR_HIP = -5
RLX_ERR_UNSUPPORTED = -6
RLX_ERR_STATE = -7

RLX_F32 = 0
RLX_BF16 = 1
RLX_LAYOUT_HSD = 0
RLX_LAYOUT_SHD = 1
RLX_MASK_CAUSAL = 0
RLX_MASK_REF = 1
RLX_MASK_NONE = 2
RLX_ROPE_OFFSET = 0
RLX_ROPE_REF = 1
RLX_ROPE_NONE = 2
RLX_TIME_ATTEND = 1
RLX_TIME_PROJECT = 2
RLX_TIME_SELECT = 4
RLX_TIME_COPY = 8

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_pi32 = ctypes.POINTER(ctypes.c_int32)
_f32 = ctypes.c_float

class SamplerParams(ctypes.Structure):
    """rlx_sampler_t: Sampler (sampler.go:33-43) without Rand."""
    _fields_ = [("temperature", _f32), ("top_k", _i32), ("top_p", _f32), ("min_p", _f32),
                ("repeat_penalty", _f32), ("frequency_penalty", _f32),
                ("presence_penalty", _f32), ("repeat_window", _i32)]


_psp = ctypes.POINTER(SamplerParams)

# name -> argument types; every entry returns int32.  Kept in the order of
# include/relux_kv.h.
SIGNATURES = {
    "rlx_init": [_i32],
    "rlx_last_error": [ctypes.c_char_p, _i64],
    "rlx_version": [ctypes.c_char_p, _i64],
    "rlx_dev_alloc": [_i64, ctypes.POINTER(_vp)],
    "rlx_dev_free": [_vp],
    "rlx_h2d": [_vp, _vp, _i64],
    "rlx_d2h": [_vp, _vp, _i64],
    "rlx_device_sync": [],
    "rlx_cache_timing": [_vp, _i32],
    "rlx_cache_kernel_time": [_vp, ctypes.POINTER(_f32), _pi32],
    "rlx_kv_create": [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    "rlx_mla_create": [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    "rlx_cache_destroy": [_vp],
    "rlx_cache_reset": [_vp],
    "rlx_cache_sync": [_vp],
    "rlx_cache_set_stream": [_vp, _vp],
    "rlx_cache_reserve": [_vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64],
    "rlx_cache_memory": [_vp, ctypes.POINTER(ctypes.c_uint64)],
    "rlx_kv_append": [_vp, _i32, _i32, _pi32, _pi32, _vp, _vp, _i32, _i32],
    "rlx_pack_qkv": [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp],
    "rlx_gqa_project_append": [_vp, _i32, _i32, _pi32, _pi32, _vp, _i32, _i32, _vp, _i32, _vp, _vp,
                               _i32, _i32, _vp, _i32],
    "rlx_pack_mla_proj": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    "rlx_mla_project_append": [_vp, _i32, _i32, _pi32, _pi32, _vp, _i32, _i32, _vp, _i32, _i32, _vp,
                               _vp, _i32, _i32, _vp, _vp, _i32],
    "rlx_pack_out": [_vp, _i32, _i32, _i32, _vp],
    "rlx_out_project": [_vp, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _i32],
    "rlx_mla_append": [_vp, _i32, _i32, _pi32, _pi32, _vp, _vp, _i32],
    "rlx_kv_gather": [_vp, _i32, _i32, _pi32, _vp, _vp],
    "rlx_mla_gather": [_vp, _i32, _i32, _pi32, _vp, _vp],
    "rlx_gqa_attend": [_vp, _i32, _i32, _pi32, _pi32, _i32, _vp, _i32, _i32, _f32, _i32, _vp, _i32],
    "rlx_gqa_attend_noalloc": [_vp, _i32, _i32, _pi32, _pi32, _i32, _vp, _i32, _i32, _f32, _i32,
                               _vp, _i32],
    "rlx_gqa_append_attend": [_vp, _i32, _i32, _pi32, _pi32, _vp, _vp, _i32, _i32, _i32, _vp, _i32,
                              _i32, _f32, _i32, _vp, _i32],
    "rlx_mla_attend": [_vp, _i32, _i32, _pi32, _pi32, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _f32,
                       _i32, _vp, _i32],
    "rlx_mla_append_attend": [_vp, _i32, _i32, _pi32, _pi32, _vp, _vp, _i32, _i32, _i32, _vp, _vp,
                              _i32, _vp, _vp, _f32, _i32, _vp, _i32],
    "rlx_rollback": [_vp, _i32, _i32, _pi32, _pi32],
    "rlx_evict": [_vp, _i32, _i32, _pi32, _pi32],
    "rlx_compact": [_vp, _i32],
    "rlx_seq_release": [_vp, _i32, _i32],
    "rlx_spill_attach": [_vp, ctypes.c_char_p, _i64],
    "rlx_spill": [_vp, _i32, _i32, _pi32, _pi32],
    "rlx_restore": [_vp, _i32, _i32, _pi32, _pi32],
    "rlx_spill_slots": [_vp, _i32, _i32, ctypes.POINTER(ctypes.c_int64), _i32, _pi32],
    "rlx_spill_info": [_vp, ctypes.POINTER(ctypes.c_int64)],
    "rlx_greedy": [_vp, _vp, _i32, _i32, _i64, _pi32],
    "rlx_sample": [_vp, _vp, _i32, _i32, _i64, _psp, _pi32, _pi32, ctypes.POINTER(_f32), _pi32],
    "rlx_sample_async": [_vp, _vp, _i32, _i32, _i64, _psp, _vp, _i64, _vp, _vp, _vp],
    "rlx_gqa_attend_ref_image": [_vp, _i32, _i32, _pi32, _pi32, _i32, _vp, _i32, _i32, _f32, _i32,
                                 _vp, _i32],
    "rlx_spec_accept_async": [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _psp, _vp, _vp],
    "rlx_spec_accept": [_vp, _vp, _vp, _pi32, _pi32, _i32, _i32, _i32, ctypes.POINTER(_f32), _psp,
                        _pi32, _pi32],
    "rlx_seq_len": [_vp, _i32, _i32, _pi32],
    "rlx_seq_state": [_vp, _i32, _i32, _pi32],
    "rlx_page_table": [_vp, _i32, _i32, _pi32],
    "rlx_free_list": [_vp, _i32, _pi32, _i32, _pi32],
    "rlx_pool_ptr": [_vp, _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
}


class ReluxError(RuntimeError):
    """A librelux_kv call returned an error code."""

    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ReluxPanic(ReluxError):
    """Raised where the reference Go code panics (cache overflow, layer index
    out of range: kvcache.go:241-243, 282-285; mla_cache.go:153-167)."""


_lib = None


def load(path=LIB_PATH):
    """Load librelux_kv.so once and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the HIP library first "
            "(python -m relux_amd.build, or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _i32
    _lib = lib
    return lib


def last_error():
    buf = ctypes.create_string_buffer(1024)
    load().rlx_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(code):
    """Raise on a negative status, mirroring the reference's panic sites."""
    if code == RLX_OK:
        return
    msg = last_error()
    if code in (RLX_ERR_OVERFLOW, RLX_ERR_LAYER):
        raise ReluxPanic(code, msg)
    raise ReluxError(code, msg)


def i32_array(values):
    vals = [int(v) for v in values]
    return (ctypes.c_int32 * max(1, len(vals)))(*vals)


_initialised = {}


def init(device=0):
    """Select a gfx950 device (once per device)."""
    if not _initialised.get(device):
        check(load().rlx_init(device))
        _initialised[device] = True
