"""relux_amd -- MI355X (gfx950) KV-cache hot path for relux.

librelux_kv.so (HIP, built in-tree by relux_amd.build) implements paged GQA
and MLA caches, append, gather, rollback/evict/compact, and decode /
verify / chunked-prefill attention over the paged cache, and the fused
Q/K/V projection + RoPE + append step, and token selection (greedy,
sampling, speculative acceptance) on logits that stay on the device.  `KVCache` and `MLACache` mirror the
reference's Go cache types (internal/transformer/kvcache.go, mla_cache.go).
"""
from ._lib import ReluxError, ReluxPanic, load  # noqa: F401

__all__ = ["KVCache", "MLACache", "ReluxError", "ReluxPanic", "load", "pack_qkv", "gqa_pack_width", "pack_mla_proj", "pack_out", "rope_tables",
           "Sampler", "SpeculativeDecoder", "Draws", "spec_accept", "spec_accept_async"]


def __getattr__(name):
    # Lazy: importing the package must not touch the GPU or require torch.
    if name in ("KVCache", "MLACache", "default_scale", "pack_qkv", "gqa_pack_width", "pack_mla_proj", "pack_out",
                "rope_tables"):
        from . import kvcache
        return getattr(kvcache, name)
    if name in ("Sampler", "SpeculativeDecoder", "Draws", "spec_accept", "spec_accept_async"):
        from . import sampling
        return getattr(sampling, name)
    raise AttributeError(name)
