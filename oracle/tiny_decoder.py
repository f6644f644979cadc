"""Config-1 tiny decoders on the CPU -- TEST INFRASTRUCTURE ONLY.

The README decoder (vocab 100, d_model 64, 4 query heads, 2 KV heads,
head_dim 16, 2 layers, DFF 128 GELU, MaxSeqLen 64, causal, RoPE base 10000)
restated from the reference's inference path:

  Transformer.Forward     transformer.go:269-280  embed, blocks, final norm, lm head
  Transformer.Generate    transformer.go:887-966  prefill Forward(prompt), then
                                                  maxNew-1 single-token steps
  Block.Forward           transformer_block.go:119-142
  MHA.forwardCached       mha.go:245-369          projections, RoPE at cacheLen,
                                                  Append, View, attention, Wo
  RMSNorm.Forward         rmsnorm.go:69-116
  MLP.forwardGELU         mlp.go:103-140, geluExact mlp.go:448-451
  Linear.Forward          linear.go:65-106        (lm head, with bias)
  Sampler.Sample          sampler.go:73+          temperature 0 and topK 1 keep
                                                  only the largest logit: greedy
                                                  argmax (ties would need the
                                                  RNG; the tests check none occur)

The attention cache is pluggable, so the same model runs over
  RefCache      -- the reference KVCache byte image: rows of KVH*D bf16 written
                   by copyInto in [KVH,S,D] order (kvcache.go:286-287,407-423)
                   and read head-major with stride totalLen (mha.go:305-310);
                   mask only when seqQ == totalLen (mha.go:340).  This is the
                   reference's own (scrambled for KVH > 1) behaviour.
  LogicalCache  -- the corrected semantics: K/V per kv head in token order,
                   bf16 like the reference cache (or f32 for the uncached
                   forward), causal mask offset by the cached length.
  any object with the same three methods (the GPU paged cache in tests).

Weights: the reference's own constructors use fixed LCG initialisers; the
configuration asks for N(0, 0.02) bf16 matrices from seed 0 with gammas 1 and
biases 0, drawn here with numpy's PCG64 (Go's math/rand stream is not
available without the Go toolchain; the seed fixes the test case, not a
reference output).
"""
import numpy as np

from . import (add_bias, bf16_from_f32, f32_from_bf16, gelu, gqa_attend, kv_copy_into,
               matmul_bf16w, mla_attend, rmsnorm, rope_apply, rope_tables)

CFG1 = dict(vocab=100, d_model=64, heads=4, kv_heads=2, layers=2, dff=128, max_seq=64,
            rope_base=10000.0, eps=1e-5)

# TestTransformer_MLA's configuration (transformer_test.go:1012-1027):
# head_dim 8, d_c = 4 head_dim, d_r = head_dim / 2.
CFG_MLA = dict(vocab=100, d_model=32, heads=4, kv_heads=4, layers=2, dff=64, max_seq=32,
               rope_base=10000.0, eps=1e-5, d_c=32, d_r=4)


def make_weights(cfg, seed=0, std=0.02):
    """bf16 (uint16) parameters of the decoder, [in, out] matrix layout."""
    rng = np.random.default_rng(seed)
    d, H, KVH = cfg["d_model"], cfg["heads"], cfg["kv_heads"]
    D = d // H

    def mat(r, c):
        return bf16_from_f32(rng.normal(0.0, std, (r, c)).astype(np.float32))

    def ones(n):
        return np.full(n, 0x3F80, np.uint16)

    def zeros(n):
        return np.zeros(n, np.uint16)

    W = {"embed": mat(cfg["vocab"], d), "layers": []}
    for _ in range(cfg["layers"]):
        W["layers"].append(dict(
            norm1=ones(d), wq=mat(d, H * D), wk=mat(d, KVH * D), wv=mat(d, KVH * D),
            wo=mat(H * D, d), norm2=ones(d), w1=mat(d, cfg["dff"]), b1=zeros(cfg["dff"]),
            w2=mat(cfg["dff"], d), b2=zeros(d)))
    W["norm_f"] = ones(d)
    W["lm_w"] = mat(d, cfg["vocab"])
    W["lm_b"] = zeros(cfg["vocab"])
    return W


def mla_dims(cfg):
    """(head_dim, d_c, d_r): unset latent dims default to 4 head_dim and
    head_dim / 2 (transformer.go:223-233)."""
    D = cfg["d_model"] // cfg["heads"]
    return D, cfg.get("d_c") or 4 * D, cfg.get("d_r") or D // 2


def make_mla_weights(cfg, seed=0, std=0.02):
    """make_weights' embedding, norms, MLP and head, with each block's
    attention replaced by the seven MLA matrices of NewMLA (mla.go:110-118),
    [in, out] layout.  Their values follow NewMLA's initialiser's
    distribution -- uniform in [-1, 1) scaled by 1/sqrt(rows) (mla.go:84-93)
    -- drawn from PCG64, so W_UK and W_UV differ (the reference's LCG
    restarts per matrix, which would make them equal)."""
    W = make_weights(dict(cfg, kv_heads=cfg["heads"]), seed, std)
    rng = np.random.default_rng(seed + 1)
    d, H = cfg["d_model"], cfg["heads"]
    D, dC, dR = mla_dims(cfg)

    def lin(r, c):
        return bf16_from_f32((rng.uniform(-1.0, 1.0, (r, c)) / np.sqrt(r)).astype(np.float32))

    for Wl in W["layers"]:
        for k in ("wq", "wk", "wv", "wo"):
            del Wl[k]
        Wl.update(w_q=lin(d, H * D), w_dkv=lin(d, dC), w_uk=lin(dC, H * D), w_uv=lin(dC, H * D),
                  w_kr=lin(d, dR), w_qr=lin(d, H * dR), w_o=lin(H * D, d))
    return W


class MLARefCache:
    """The reference MLACache and forwardCached's attention: f32 latent rows
    (mla_cache.go:171-172), K_c / V decompressed token-major and read
    head-major (mla.go:326-356, head_major_compat), mask only when
    seqQ == totalLen (mla.go:368)."""

    def __init__(self, cfg):
        self.cap = cfg["max_seq"]
        self.c = [np.zeros((0, mla_dims(cfg)[1]), np.float32) for _ in range(cfg["layers"])]
        self.kr = [np.zeros((0, mla_dims(cfg)[2]), np.float32) for _ in range(cfg["layers"])]

    def total_len(self, layer):
        return self.c[layer].shape[0]

    def append(self, layer, c, kr):
        if self.total_len(layer) + c.shape[0] > self.cap:
            raise OverflowError("MLACache.Append: overflow")
        self.c[layer] = np.concatenate([self.c[layer], np.asarray(c, np.float32)])
        self.kr[layer] = np.concatenate([self.kr[layer], np.asarray(kr, np.float32)])

    def attend(self, layer, qc, qr, w_uk, w_uv):
        return mla_attend(qc, qr, self.c[layer], self.kr[layer], w_uk, w_uv, mask="ref",
                          head_major_compat=True)


class MLALogicalCache(MLARefCache):
    """Corrected MLA semantics: head h reads its own slice of the
    decompressed rows (as the uncached path does, mla.go:159-161), the causal
    mask is offset by the cached length, and rows are stored bf16 like the
    device cache (or f32, store_bf16=False)."""

    def __init__(self, cfg, store_bf16=True):
        super().__init__(cfg)
        self.store_bf16 = store_bf16

    def append(self, layer, c, kr):
        if self.store_bf16:
            c, kr = f32_from_bf16(bf16_from_f32(c)), f32_from_bf16(bf16_from_f32(kr))
        super().append(layer, c, kr)

    def attend(self, layer, qc, qr, w_uk, w_uv):
        return mla_attend(qc, qr, self.c[layer], self.kr[layer], w_uk, w_uv, mask="causal")


class RefCache:
    """Reference KVCache byte image (bf16), one [cap][KVH*D] buffer per layer."""

    def __init__(self, cfg):
        self.KVH = cfg["kv_heads"]
        self.D = cfg["d_model"] // cfg["heads"]
        self.cap = cfg["max_seq"]
        row = self.KVH * self.D
        self.k = [np.zeros(self.cap * row, np.uint16) for _ in range(cfg["layers"])]
        self.v = [np.zeros(self.cap * row, np.uint16) for _ in range(cfg["layers"])]
        self.len = [0] * cfg["layers"]

    def total_len(self, layer):
        return self.len[layer]

    def append(self, layer, k, v):
        """k, v: f32 [KVH, S, D] (the rearranged, rotated projections)."""
        S = k.shape[1]
        if self.len[layer] + S > self.cap:
            raise OverflowError("KVCache.Append: overflow")
        kv_copy_into(self.k[layer], k, self.len[layer], S, self.KVH * self.D)
        kv_copy_into(self.v[layer], v, self.len[layer], S, self.KVH * self.D)
        self.len[layer] += S

    def attend(self, layer, q):
        T = self.len[layer]
        n = self.KVH * T * self.D
        kw = f32_from_bf16(self.k[layer][:n]).reshape(self.KVH, T, self.D)
        vw = f32_from_bf16(self.v[layer][:n]).reshape(self.KVH, T, self.D)
        return gqa_attend(q, kw, vw, mask="ref")


class LogicalCache:
    """Corrected cache semantics: [KVH, T, D] per layer, causal mask."""

    def __init__(self, cfg, store_bf16=True):
        self.store_bf16 = store_bf16
        self.k = [None] * cfg["layers"]
        self.v = [None] * cfg["layers"]

    def total_len(self, layer):
        return 0 if self.k[layer] is None else self.k[layer].shape[1]

    def append(self, layer, k, v):
        if self.store_bf16:
            k, v = f32_from_bf16(bf16_from_f32(k)), f32_from_bf16(bf16_from_f32(v))
        if self.k[layer] is None:
            self.k[layer], self.v[layer] = k.copy(), v.copy()
        else:
            self.k[layer] = np.concatenate([self.k[layer], k], axis=1)
            self.v[layer] = np.concatenate([self.v[layer], v], axis=1)

    def attend(self, layer, q):
        return gqa_attend(q, self.k[layer], self.v[layer], mask="causal")

    def rollback(self, layer, n):
        """Drop the newest n tokens (the device cache's rlx_rollback)."""
        if n:
            T = self.total_len(layer)
            assert 0 <= n <= T
            self.k[layer] = self.k[layer][:, :T - n]
            self.v[layer] = self.v[layer][:, :T - n]


class TinyDecoder:
    def __init__(self, cfg=CFG1, weights=None, seed=0, rope_rule="ref"):
        """rope_rule "ref": RotaryEmbedding.Apply's rule (rope.go:152-153:
        with startPos > 0 every row of a call takes position startPos, which
        Generate's one-token steps never trigger); "offset": row j of a call
        takes position start + j (the positions a chunked verify needs)."""
        self.rope_rule = rope_rule
        self.cfg = dict(cfg)
        self.W = weights if weights is not None else make_weights(self.cfg, seed)
        self.H, self.KVH = cfg["heads"], cfg["kv_heads"]
        self.D = cfg["d_model"] // cfg["heads"]
        self.rope = rope_tables(self.D, cfg["rope_base"], cfg["max_seq"])

    def _attention(self, layer, x, cache):
        """MHA.forwardCached (mha.go:245-369) for batch 1; x [S, d_model]."""
        Wl = self.W["layers"][layer]
        S = x.shape[0]
        H, KVH, D = self.H, self.KVH, self.D
        q = matmul_bf16w(x, Wl["wq"]).reshape(S, H, D).transpose(1, 0, 2)
        k = matmul_bf16w(x, Wl["wk"]).reshape(S, KVH, D).transpose(1, 0, 2)
        v = matmul_bf16w(x, Wl["wv"]).reshape(S, KVH, D).transpose(1, 0, 2)
        start = cache.total_len(layer)
        q = self._rope(np.ascontiguousarray(q), start)
        k = self._rope(np.ascontiguousarray(k), start)
        v = np.ascontiguousarray(v, np.float32)
        cache.append(layer, k, v)
        o = cache.attend(layer, q)  # [H, S, D]
        o = np.ascontiguousarray(np.asarray(o, np.float32).transpose(1, 0, 2)).reshape(S, H * D)
        return matmul_bf16w(o, Wl["wo"])

    def _rope(self, x, start, tables=None):
        """x [heads, S, dim] at cache position start."""
        tables = self.rope if tables is None else tables
        if self.rope_rule == "ref" or start == 0:
            return rope_apply(x, start, tables, self.cfg["max_seq"])
        return np.concatenate([rope_apply(np.ascontiguousarray(x[:, j:j + 1]), start + j, tables,
                                          self.cfg["max_seq"]) for j in range(x.shape[1])], axis=1)

    def forward(self, ids, cache):
        """Transformer.Forward(ids, 1) with the caches wired in: logits [S, vocab]."""
        eps = np.float32(self.cfg["eps"])
        x = f32_from_bf16(self.W["embed"][np.asarray(ids)])
        for layer, Wl in enumerate(self.W["layers"]):
            h = rmsnorm(x, Wl["norm1"], eps)
            x = (x + self._attention(layer, h, cache)).astype(np.float32)
            h = rmsnorm(x, Wl["norm2"], eps)
            m = gelu(add_bias(matmul_bf16w(h, Wl["w1"]), Wl["b1"]))
            x = (x + add_bias(matmul_bf16w(m, Wl["w2"]), Wl["b2"])).astype(np.float32)
        x = rmsnorm(x, self.W["norm_f"], eps)
        return add_bias(matmul_bf16w(x, self.W["lm_w"]), self.W["lm_b"])

    def forward_uncached(self, ids):
        """MHA.Forward without a cache (mha.go:119-238): the whole sequence
        at positions 0..S-1, causal, f32 K/V -- the semantic oracle (row t is
        the exact decode of step t)."""
        return self.forward(ids, LogicalCache(self.cfg, store_bf16=False))

    def generate(self, prompt, max_new, cache):
        """Transformer.Generate(prompt, max_new, 0, 1, rng) greedy: returns
        (tokens, logits of every forward call's last row, smallest top-2 gap)."""
        logits = self.forward(prompt, cache)
        steps = [logits[-1].copy()]
        out = list(prompt)
        for i in range(max_new):
            if i > 0:
                logits = self.forward([out[-1]], cache)
                steps.append(logits[-1].copy())
            out.append(int(np.argmax(steps[-1])))
        gap = min(float(np.diff(np.sort(s)[-2:])[0]) for s in steps)
        return out, np.stack(steps), gap


class MLATinyDecoder(TinyDecoder):
    """The same decoder with AttnType "mla" blocks (transformer_block.go:
    69-77): each block's attention is MLA.forwardCached (mla.go:272-397) for
    batch 1 over a pluggable latent cache (MLARefCache, MLALogicalCache or
    the GPU paged cache in tests, with total_len / append / attend)."""

    def __init__(self, cfg=CFG_MLA, weights=None, seed=0, rope_rule="ref"):
        cfg = dict(cfg)
        self.D, self.dC, self.dR = mla_dims(cfg)
        super().__init__(cfg, weights if weights is not None else make_mla_weights(cfg, seed),
                         seed, rope_rule)
        # MLA's own RoPE over d_r dims, base and length of the model's
        # (NewBlock, transformer_block.go:69-75; NewMLA mla.go:83)
        self.rope_r = rope_tables(self.dR, cfg["rope_base"], cfg["max_seq"])

    def _attention(self, layer, x, cache):
        """forwardCached for batch 1; x [S, d_model] -> [S, d_model]."""
        Wl = self.W["layers"][layer]
        S = x.shape[0]
        H, D, dR = self.H, self.D, self.dR
        # 1. projections (mla.go:286-289)
        qc = matmul_bf16w(x, Wl["w_q"]).reshape(S, H, D).transpose(1, 0, 2)
        qr = matmul_bf16w(x, Wl["w_qr"]).reshape(S, H, dR).transpose(1, 0, 2)
        ckv = matmul_bf16w(x, Wl["w_dkv"])
        kr = matmul_bf16w(x, Wl["w_kr"])
        # 3. RoPE of q^R [H, S, dR] and k^R [S, dR] at the cached length
        # (mla.go:297-310; a rank-2 k^R takes rows as positions)
        start = cache.total_len(layer)
        qr = self._rope(np.ascontiguousarray(qr), start, self.rope_r)
        kr = self._rope(np.ascontiguousarray(kr)[None], start, self.rope_r)[0]
        # 4-6. append, attention over every cached row (mla.go:312-377)
        cache.append(layer, np.ascontiguousarray(ckv, np.float32), kr)
        o = cache.attend(layer, np.ascontiguousarray(qc), qr, Wl["w_uk"], Wl["w_uv"])  # [H, S, D]
        # 7. back to [S, H*D], W_O (mla.go:385-389)
        o = np.ascontiguousarray(np.asarray(o, np.float32).transpose(1, 0, 2)).reshape(S, H * D)
        return matmul_bf16w(o, Wl["w_o"])

    def forward_uncached(self, ids):
        """The whole sequence in one call at positions 0..S-1 over an f32
        corrected cache: row t is the exact decode of step t."""
        return self.forward(ids, MLALogicalCache(self.cfg, store_bf16=False))


def ref_byte_image(k_logical, chunks, cap):
    """Reference cache bytes from logical ones: k_logical [KVH, T, D] (any
    dtype) appended in `chunks` (rows per Append call, in order).  Append
    copies each [KVH, S, D] block raw into rows r..r+S-1 of a [cap][KVH*D]
    buffer (kvcache.go:286-287, copyInto 407-423), so element (kvh, r+s, d)
    lands at flat (r*KVH + kvh*S + s)*D + d.  Unwritten rows stay zero."""
    KVH, T, D = k_logical.shape
    img = np.zeros(cap * KVH * D, k_logical.dtype)
    r = 0
    for S in chunks:
        blk = k_logical[:, r:r + S, :]  # [KVH, S, D]
        img[r * KVH * D:(r + S) * KVH * D] = blk.reshape(-1)
        r += S
    assert r == T
    return img


def prompt_ids(cfg=CFG1, n=8, seed=0):
    """8 prompt ids uniform in [0, vocab) from seed 0."""
    return [int(t) for t in np.random.default_rng(seed).integers(0, cfg["vocab"], n)]
