"""Fused pre-attention step (rlx_pack_qkv + rlx_gqa_project_append):
projection of the new tokens' hidden states, RoPE of q and k, paged append
of k and v, checked against the oracle's restatement of mha.go:250-289
(matmul_bf16w, rope_apply, BF16FromF32); and the step after attention
(rlx_pack_out + rlx_out_project: W_O, mha.go:356-360, plus the residual).

f32 activations enter the MFMA products as hi + lo bf16 pairs, so the
checks compare with the oracle on the same f32 activations: only the f32
summation order (and the ~2^-17 of the lo part) differ."""
import numpy as np
import pytest
import torch

import oracle
from oracle import tiny_decoder as td

pytestmark = pytest.mark.gpu


def _bf16_tensor(u16, gpu):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).to(gpu).view(torch.bfloat16)


def _oracle_qkv(x, wq, wk, wv, H, KVH, D, tables, max_seq, positions):
    """Per-row reference step: projections, then RoPE of each head row at its
    position (positions[r] = -1: no rotation).  Returns q [R,H,D], k, v [R,KVH,D]."""
    R = x.shape[0]
    q = oracle.matmul_bf16w(x, wq).reshape(R, H, D)
    k = oracle.matmul_bf16w(x, wk).reshape(R, KVH, D)
    v = oracle.matmul_bf16w(x, wv).reshape(R, KVH, D)
    for r in range(R):
        if positions[r] >= 0:
            # [heads, 1, D]: every head row of token r at positions[r]
            q[r] = oracle.rope_apply(q[r][:, None, :], positions[r], tables, max_seq)[:, 0, :]
            k[r] = oracle.rope_apply(k[r][:, None, :], positions[r], tables, max_seq)[:, 0, :]
    return q, k, v


@pytest.mark.parametrize("d_model,H,KVH,D,lens,ntok,x_dtype,mode", [
    (256, 8, 2, 64, [0, 5, 40], [3, 1, 70], torch.float32, "offset"),   # > 64 rows: two launches
    (512, 16, 4, 128, [17, 0], [1, 9], torch.bfloat16, "offset"),
    (64, 4, 2, 16, [0], [8], torch.float32, "offset"),                   # config-1 shapes
    (128, 4, 4, 32, [6, 3], [4, 2], torch.float32, "ref"),               # reference RoPE rule
    # the 8k block's shapes: 16 decode rows through d_model 4096
    (4096, 32, 8, 128, [40] * 16, [1] * 16, torch.bfloat16, "offset"),
    (4096, 32, 8, 128, [40] * 16, [1] * 16, torch.float32, "offset"),
    # decode-size kernel: 20 rows (two row tiles), d_model 2048
    (2048, 8, 2, 128, [10] * 20, [1] * 20, torch.bfloat16, "offset"),
    # 261 16-feature tiles (more than the CUs) at d_model 512: two tiles per
    # work-group, the last work-group's second tile empty
    (512, 259, 1, 16, [5, 0, 3], [1, 1, 1], torch.bfloat16, "offset"),
    # ... and at d_model 256, whose one-wave work-groups take one tile
    (256, 259, 1, 16, [5, 0, 3], [1, 1, 1], torch.bfloat16, "offset"),
    # 20 rows (two row tiles) at d_model 256 (one wave per work-group): the
    # chunked kernel
    (256, 8, 2, 64, [3] * 20, [1] * 20, torch.bfloat16, "offset"),
    # head_dim 80 stored in 96-dim pages (the new rows' padding is zeroed),
    # decode-size and chunked kernels
    (512, 8, 2, 80, [7, 30], [1, 1], torch.bfloat16, "offset"),
    (256, 4, 2, 80, [0, 12], [40, 30], torch.float32, "offset"),
    # the reference tests' tiny layers (heads packed 16 features wide, x
    # rows padded to 32): mha_test.go:86 (dModel 4, 2 heads over 1 kv head)
    # and NewMHA(8, 4, 2), then H x head_dim 36 and d_model 40
    (4, 2, 1, 2, [0, 3], [4, 2], torch.float32, "offset"),
    (8, 4, 2, 2, [5], [3], torch.float32, "ref"),
    (96, 3, 1, 12, [0, 20], [5, 1], torch.bfloat16, "offset"),
    (40, 2, 2, 20, [7, 0], [1, 33], torch.float32, "offset"),
])
def test_project_append_matches_oracle(gpu, d_model, H, KVH, D, lens, ntok, x_dtype, mode):
    from relux_amd import KVCache, pack_qkv, rope_tables
    rng = np.random.default_rng(d_model + H + D)
    S = len(lens)
    max_seq = 256
    c = KVCache(num_layers=1, max_len=max_seq, num_kv_heads=KVH, head_dim=D, max_seqs=S,
                device=gpu.index)
    wq = oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, H * D)).astype(np.float32))
    wk = oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, KVH * D)).astype(np.float32))
    wv = oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, KVH * D)).astype(np.float32))
    wp = pack_qkv(_bf16_tensor(wq, gpu), _bf16_tensor(wk, gpu), _bf16_tensor(wv, gpu), H, KVH, D)
    # packed layout: (16-feature x 32-k) fragments of W^T, fragment-major;
    # heads W features wide and k rows padded to 32, zeros in the padding
    from relux_amd import gqa_pack_width
    W, Kp = gqa_pack_width(H, KVH, D), -(-d_model // 32) * 32
    heads = lambda w, nh: np.pad(w.reshape(d_model, nh, D), ((0, 0), (0, 0), (0, W - D))).reshape(d_model, nh * W)
    wt = np.pad(np.concatenate([heads(wq, H), heads(wk, KVH), heads(wv, KVH)], axis=1),
                ((0, Kp - d_model), (0, 0))).T  # [N][Kp]
    N = wt.shape[0]
    blk = wt.reshape(N // 16, 16, Kp // 32, 32).transpose(0, 2, 1, 3).reshape(N, Kp)
    np.testing.assert_array_equal(wp.view(torch.int16).cpu().numpy().view(np.uint16).reshape(N, Kp), blk)
    rope = rope_tables(D, 10000.0, max_seq, gpu)
    tables = oracle.rope_tables(D, 10000.0, max_seq)
    # existing context through the plain append
    for i, L in enumerate(lens):
        if L:
            kv = torch.from_numpy(rng.standard_normal((L, KVH, D), dtype=np.float32)).to(gpu)
            c.Append(0, kv, kv, seq_ids=[i], n_tok=[L], layout="SHD")
    R = sum(ntok)
    x = rng.standard_normal((R, d_model), dtype=np.float32)
    xt = torch.from_numpy(x).to(gpu).to(x_dtype)
    q = c.ProjectAppend(0, xt, wp, H, rope=rope, seq_ids=list(range(S)), n_tok=ntok,
                        rope_mode=mode).cpu().numpy()
    pos = []
    for L, n in zip(lens, ntok):
        pos += [L + j for j in range(n)] if mode == "offset" else [L if L > 0 else j for j in range(n)]
    xr = xt.float().cpu().numpy()  # the activations the device saw (bf16 inputs exactly)
    q_o, k_o, v_o = _oracle_qkv(xr, wq, wk, wv, H, KVH, D, tables, max_seq, pos)
    np.testing.assert_allclose(q, q_o, atol=2e-4, rtol=1e-4)
    # cache bytes of the new tokens
    off = 0
    for i, (L, n) in enumerate(zip(lens, ntok)):
        kg, vg = c.View(0, i)
        kg = kg[0].view(torch.int16).cpu().numpy().view(np.uint16)[:, L:, :]  # [KVH, n, D]
        vg = vg[0].view(torch.int16).cpu().numpy().view(np.uint16)[:, L:, :]
        kw = oracle.bf16_from_f32(k_o[off:off + n].transpose(1, 0, 2))
        vw = oracle.bf16_from_f32(v_o[off:off + n].transpose(1, 0, 2))
        for got, want in ((kg, kw), (vg, vw)):
            same = (got == want).mean()
            assert same > 0.99, same
            np.testing.assert_allclose(oracle.f32_from_bf16(got), oracle.f32_from_bf16(want),
                                       atol=1e-2, rtol=1e-2)
        off += n
    assert [c.TotalLen(0, i) for i in range(S)] == [L + n for L, n in zip(lens, ntok)]


@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_project_append_with_staged_plan_equals_kernel_argument_plan(gpu, x_dtype):
    """A compaction leaves table writes pending for every moved page; the
    next ProjectAppend carries them, and with 32 decode rows its plan no
    longer fits the kernel arguments, so it is staged in device memory.
    Against a twin cache that evicted the same pages without compacting
    (plan in the kernel arguments): rotated q, every cached K/V byte and
    the lengths identical, bit for bit."""
    from relux_amd import KVCache, pack_qkv, rope_tables
    rng = np.random.default_rng(11)
    S, H, KVH, D, d_model, L = 32, 16, 4, 64, 1024, 120
    caches = [KVCache(num_layers=1, max_len=256, num_kv_heads=KVH, head_dim=D, max_seqs=S,
                      device=gpu.index) for _ in range(2)]
    w = [oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, n * D)).astype(np.float32)) for n in (H, KVH, KVH)]
    wp = pack_qkv(*[_bf16_tensor(m, gpu) for m in w], H, KVH, D)
    rope = rope_tables(D, 10000.0, 256, gpu)
    for i in range(S):  # interleaved fills: the pages of a sequence are scattered
        kv = torch.from_numpy(rng.standard_normal((L, KVH, D), dtype=np.float32)).to(gpu)
        for c in caches:
            c.Append(0, kv, kv, seq_ids=[i], n_tok=[L], layout="SHD")
    for c in caches:
        c.Evict(list(range(S)), [2] * S)
    # every sequence's table row shifts: ~8 pending writes per sequence, 256
    # in all (2 KB of patches), past the 2 KB of kernel-argument plan
    caches[0].Compact()
    x = torch.from_numpy(rng.standard_normal((S, d_model), dtype=np.float32)).to(gpu).to(x_dtype)
    qs = [c.ProjectAppend(0, x, wp, H, rope=rope, seq_ids=list(range(S)), n_tok=[1] * S).cpu()
          for c in caches]
    assert torch.equal(qs[0], qs[1])
    for i in range(S):
        assert caches[0].TotalLen(0, i) == caches[1].TotalLen(0, i)
        k0, v0 = caches[0].View(0, i)
        k1, v1 = caches[1].View(0, i)
        assert torch.equal(k0.view(torch.int16), k1.view(torch.int16))
        assert torch.equal(v0.view(torch.int16), v1.view(torch.int16))


def test_rope_position_overflow_panics(gpu):
    from relux_amd import KVCache, ReluxPanic, pack_qkv, rope_tables
    c = KVCache(num_layers=1, max_len=64, num_kv_heads=1, head_dim=16, device=gpu.index)
    w = torch.zeros((64, 16), dtype=torch.bfloat16, device=gpu)
    wp = pack_qkv(w, w, w, 1, 1, 16)
    rope = rope_tables(16, 10000.0, 8, gpu)  # positions 0..7 only
    x = torch.zeros((9, 64), device=gpu)
    with pytest.raises(ReluxPanic):
        c.ProjectAppend(0, x, wp, 1, rope=rope)
    assert c.TotalLen(0) == 0  # nothing appended


@pytest.mark.parametrize("rows,k_in,n_out,x_dtype,out_dtype,resid", [
    (3, 512, 256, torch.float32, torch.float32, False),
    (64, 256, 128, torch.float32, torch.float32, True),
    (70, 128, 64, torch.bfloat16, torch.float32, True),     # two launches
    (17, 4096, 4096, torch.float32, torch.bfloat16, True),  # the 8k block's W_O
    (16, 4096, 4096, torch.bfloat16, torch.float32, True),  # ... with bf16 activations
    (40, 1024, 512, torch.bfloat16, torch.bfloat16, False),  # 3 row tiles
    (20, 2048, 512, torch.bfloat16, torch.float32, True),    # decode-size kernel, two row tiles
    (8, 512, 4608, torch.bfloat16, torch.bfloat16, True),    # 288 tiles: two per work-group
    # the reference tests' tiny layers: W_O of dModel 4 (k_in 4, n_out 4), and
    # k_in / n_out that are not multiples of 32 / 16 (zero-padded packing)
    (5, 4, 4, torch.float32, torch.float32, True),
    (33, 40, 24, torch.bfloat16, torch.float32, True),
])
def test_out_project_matches_oracle(gpu, rows, k_in, n_out, x_dtype, out_dtype, resid):
    """out = x . W_O (+ residual): mha.go:356-360 matmulBatched3D (bf16
    weights widened, f32 sums) and the block's f32 residual add."""
    from relux_amd import KVCache, pack_out
    rng = np.random.default_rng(rows + k_in)
    c = KVCache(num_layers=1, max_len=16, num_kv_heads=1, head_dim=64, device=gpu.index)
    w = oracle.bf16_from_f32(rng.normal(0, 0.02, (k_in, n_out)).astype(np.float32))
    wp = pack_out(_bf16_tensor(w, gpu))
    x = rng.standard_normal((rows, k_in), dtype=np.float32)
    xt = torch.from_numpy(x).to(gpu).to(x_dtype)
    r = torch.from_numpy(rng.standard_normal((rows, n_out), dtype=np.float32)).to(gpu).to(out_dtype) if resid else None
    y = c.OutProject(xt, wp, n_out, residual=r, out_dtype=out_dtype).float().cpu().numpy()
    want = oracle.matmul_bf16w(xt.float().cpu().numpy(), w)
    if resid:
        want = (want + r.float().cpu().numpy()).astype(np.float32)
    if out_dtype == torch.float32:
        np.testing.assert_allclose(y, want, atol=2e-5 * np.sqrt(k_in), rtol=1e-4)
    else:  # bf16 out: the rounding of the same f32 value, or one ulp off at a tie
        wb = oracle.f32_from_bf16(oracle.bf16_from_f32(want))
        assert (y == wb).mean() > 0.98
        np.testing.assert_allclose(y, wb, atol=1e-2, rtol=1e-2)


class FusedGpuDecoder(td.TinyDecoder):
    """Config-1 decoder whose attention layers run the fused device step:
    ProjectAppend (projection, RoPE, append) then Attend."""

    def __init__(self, device):
        super().__init__(td.CFG1, seed=0)
        from relux_amd import KVCache, pack_qkv, rope_tables
        cfg = self.cfg
        self.dev = device
        self.cache = KVCache(num_layers=cfg["layers"], max_len=cfg["max_seq"],
                             num_kv_heads=self.KVH, head_dim=self.D, device=device.index)
        self.wp = [pack_qkv(_bf16_tensor(Wl["wq"], device), _bf16_tensor(Wl["wk"], device),
                            _bf16_tensor(Wl["wv"], device), self.H, self.KVH, self.D)
                   for Wl in self.W["layers"]]
        self.rope_dev = rope_tables(self.D, cfg["rope_base"], cfg["max_seq"], device)
        from relux_amd import pack_out
        self.wo = [pack_out(_bf16_tensor(Wl["wo"], device)) for Wl in self.W["layers"]]

    def _attention(self, layer, x, cache):
        S = x.shape[0]
        q = self.cache.ProjectAppend(layer, torch.from_numpy(np.ascontiguousarray(x)).to(self.dev),
                                     self.wp[layer], self.H, rope=self.rope_dev)
        o = self.cache.Attend(layer, q, self.H, n_q=[S], layout="SHD", mask="causal")
        # W_O on the device too: the whole attention block runs there
        y = self.cache.OutProject(o.reshape(S, self.H * self.D), self.wo[layer], self.cfg["d_model"])
        return y.cpu().numpy()


def test_cfg1_generate_with_fused_step(gpu):
    """Config 1 end to end with the attention block on the GPU (projection,
    RoPE, append, attention, W_O): logits within 2e-2 / 2e-3 of the oracle
    over the same tokens."""
    m = FusedGpuDecoder(gpu)
    prompt = td.prompt_ids(td.CFG1)
    toks, logits, _ = m.generate(prompt, 16, None)
    ref = td.TinyDecoder(td.CFG1, seed=0)
    logical = td.LogicalCache(ref.cfg)
    want = [ref.forward(prompt, logical)[-1]]
    for t in toks[len(prompt):-1]:
        want.append(ref.forward([t], logical)[-1])
    d = np.abs(logits - np.stack(want))
    print(f"cfg1 fused logits max {d.max():.3e} mean {d.mean():.3e}")
    assert d.max() < 2e-2 and d.mean() < 2e-3
    assert m.cache.TotalLen(0) == len(toks) - 1


@pytest.mark.parametrize("d_model,H,D,lens,ntok,mode,x_dtype,dC,dR", [
    (256, 4, 128, [0, 70], [5, 2], "offset", torch.float32, 512, 64),
    (512, 16, 128, [9], [66], "offset", torch.float32, 512, 64),     # > 64 rows: two launches
    (128, 2, 64, [3, 0], [3, 4], "ref", torch.float32, 512, 64),
    (2048, 16, 128, [20] * 32, [1] * 32, "offset", torch.bfloat16, 512, 64),  # config 3's decode rows
    (512, 16, 128, [9], [66], "offset", torch.bfloat16, 512, 64),
    (4096, 8, 128, [12] * 16, [1] * 16, "offset", torch.bfloat16, 512, 64),   # decode-size kernel, 16 waves
    (4096, 8, 128, [12] * 20, [1] * 20, "offset", torch.bfloat16, 512, 64),   # 2 row tiles at 16 waves: chunked
    # the reference's default latent dims (dC = 4 headDim, dHR = headDim/2,
    # transformer.go:223-233): packed widths rounded up to 16, zero padded
    (512, 8, 32, [5, 40], [1, 1], "offset", torch.bfloat16, 128, 16),
    (256, 4, 64, [0, 20], [9, 3], "offset", torch.float32, 256, 32),
    (256, 4, 16, [3, 0], [2, 5], "ref", torch.float32, 64, 8),      # config-1-sized MLA layer
    # mla_test.go's layer (dModel 8, 2 heads, headDim 4, dC 16, dHR 2: q_c
    # heads packed 16 wide, x rows padded to 32) and H x head_dim 60 at d_model 40
    (8, 2, 4, [0, 5], [3, 2], "offset", torch.float32, 16, 2),
    (40, 3, 20, [4, 0], [1, 6], "ref", torch.bfloat16, 80, 10),
])
def test_mla_project_append_matches_oracle(gpu, d_model, H, D, lens, ntok, mode, x_dtype, dC, dR):
    """mla.go:279-314: q_c = x.W_Q, q_r = RoPE(x.W_QR), c = x.W_DKV,
    k^R = RoPE(x.W_KR) appended as latent rows."""
    from relux_amd import MLACache, pack_mla_proj, rope_tables
    rng = np.random.default_rng(7 + d_model + H + dC)
    S = len(lens)
    max_seq = 256
    c = MLACache(num_layers=1, max_len=max_seq, d_c=dC, d_r=dR, max_seqs=S, device=gpu.index)
    mats = [oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, w)).astype(np.float32))
            for w in (H * D, H * dR, dC, dR)]
    wp = pack_mla_proj(*[_bf16_tensor(m, gpu) for m in mats], H, D)
    rope = rope_tables(dR, 10000.0, max_seq, gpu)
    tables = oracle.rope_tables(dR, 10000.0, max_seq)
    for i, L in enumerate(lens):
        if L:
            cc = torch.from_numpy(rng.standard_normal((L, dC), dtype=np.float32)).to(gpu)
            kr = torch.from_numpy(rng.standard_normal((L, dR), dtype=np.float32)).to(gpu)
            c.Append(0, cc, kr, seq_ids=[i], n_tok=[L])
    R = sum(ntok)
    x = rng.standard_normal((R, d_model), dtype=np.float32)
    xt = torch.from_numpy(x).to(gpu).to(x_dtype)
    x = xt.float().cpu().numpy()  # the activations the device saw (bf16 inputs exactly)
    qn, qr = c.ProjectAppend(0, xt, wp, H, D, rope=rope,
                             seq_ids=list(range(S)), n_tok=ntok, rope_mode=mode)
    qn, qr = qn.cpu().numpy(), qr.cpu().numpy()
    pos = []
    for L, n in zip(lens, ntok):
        pos += [L + j for j in range(n)] if mode == "offset" else [L if L > 0 else j for j in range(n)]
    xr = x  # f32 activations: the device uses them at f32 precision (hi + lo)
    qc_o = oracle.matmul_bf16w(xr, mats[0]).reshape(R, H, D)
    qr_o = oracle.matmul_bf16w(xr, mats[1]).reshape(R, H, dR)
    c_o = oracle.matmul_bf16w(xr, mats[2])
    kr_o = oracle.matmul_bf16w(xr, mats[3])
    for r in range(R):
        qr_o[r] = oracle.rope_apply(qr_o[r][:, None, :], pos[r], tables, max_seq)[:, 0, :]
        kr_o[r] = oracle.rope_apply(kr_o[r][None, None, :], pos[r], tables, max_seq)[0, 0, :]
    np.testing.assert_allclose(qn, qc_o, atol=2e-4, rtol=1e-4)
    np.testing.assert_allclose(qr, qr_o, atol=2e-4, rtol=1e-4)
    # Sum order differs from the oracle's sequential one by a few f32 ulp,
    # which flips a bf16 rounding now and then: bit-equality is counted over
    # all new rows together (one decode row holds only 64 rope-key values).
    off = 0
    same = []
    for i, (L, n) in enumerate(zip(lens, ntok)):
        cg, krg = c.View(0, i)
        cg = cg[0].view(torch.int16).cpu().numpy().view(np.uint16)[L:]
        krg = krg[0].view(torch.int16).cpu().numpy().view(np.uint16)[L:]
        for got, want in ((cg, oracle.bf16_from_f32(c_o[off:off + n])),
                          (krg, oracle.bf16_from_f32(kr_o[off:off + n]))):
            same.append((got == want).ravel())
            np.testing.assert_allclose(oracle.f32_from_bf16(got), oracle.f32_from_bf16(want),
                                       atol=1e-2, rtol=1e-2)
        off += n
    assert np.concatenate(same).mean() > 0.99


def _check_gqa_step(c, q, x, wq, wk, wv, H, KVH, D, tables, max_seq, seqs, ntok, live_before, pos):
    """q and the appended K/V rows of one ProjectAppend against the oracle
    step at the given absolute RoPE positions (one per new row)."""
    q_o, k_o, v_o = _oracle_qkv(x, wq, wk, wv, H, KVH, D, tables, max_seq, pos)
    np.testing.assert_allclose(q, q_o, atol=2e-4, rtol=1e-4)
    off = 0
    same = []
    for s, n, L in zip(seqs, ntok, live_before):
        kg, vg = c.View(0, s)
        kg = kg[0].view(torch.int16).cpu().numpy().view(np.uint16)[:, L:, :]
        vg = vg[0].view(torch.int16).cpu().numpy().view(np.uint16)[:, L:, :]
        assert kg.shape[1] == n
        for got, want in ((kg, oracle.bf16_from_f32(k_o[off:off + n].transpose(1, 0, 2))),
                          (vg, oracle.bf16_from_f32(v_o[off:off + n].transpose(1, 0, 2)))):
            same.append((got == want).ravel())
            np.testing.assert_allclose(oracle.f32_from_bf16(got), oracle.f32_from_bf16(want),
                                       atol=1e-2, rtol=1e-2)
        off += n
    assert np.concatenate(same).mean() > 0.99


@pytest.mark.parametrize("tier", ["evict", "spill"])
def test_project_append_positions_after_evict_and_spill(gpu, tier):
    """RoPE positions of the fused step once pages have left the cache
    (rope.go:130-180 positions a token by its place in the whole sequence):
    after Evict + Compact, and after Spill (the same device state), the new
    tokens are rotated at pos_offset + live_len + j -- the count of every
    token the sequence ever held, not the live length -- and after Restore
    the positions continue from the restored length.  Checked against
    oracle.rope_apply at those absolute positions; a position taken from the
    live length alone (the slip this guards against) misses it by the
    evicted page count x page_tokens."""
    from relux_amd import KVCache, pack_qkv, rope_tables
    rng = np.random.default_rng(31 if tier == "evict" else 37)
    H, KVH, D, d_model, P, max_seq = 8, 2, 64, 256, 16, 256
    lens = [40, 70, 33, 16]
    drop = [1, 3, 2, 1]
    S = len(lens)
    c = KVCache(num_layers=1, max_len=max_seq, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=S, device=gpu.index)
    wq, wk, wv = [oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, n * D)).astype(np.float32))
                  for n in (H, KVH, KVH)]
    wp = pack_qkv(_bf16_tensor(wq, gpu), _bf16_tensor(wk, gpu), _bf16_tensor(wv, gpu), H, KVH, D)
    rope = rope_tables(D, 10000.0, max_seq, gpu)
    tables = oracle.rope_tables(D, 10000.0, max_seq)
    for i, L in enumerate(lens):  # interleaved one-page fills scatter the pages
        for t0 in range(0, L, P):
            n = min(P, L - t0)
            kv = torch.from_numpy(rng.standard_normal((n, KVH, D), dtype=np.float32)).to(gpu)
            c.Append(0, kv, kv, seq_ids=[i], n_tok=[n], layout="SHD")
    before = [c.View(0, i) for i in range(S)]
    if tier == "evict":
        c.Evict(list(range(S)), drop)
        c.Compact()
    else:
        c.AttachSpill(sum(drop))
        c.Spill(list(range(S)), drop)
    for i in range(S):
        st = c.SeqState(0, i)
        assert st["pos_offset"] == drop[i] * P and st["len"] == lens[i] - drop[i] * P
    held = list(lens)  # tokens each sequence ever held (positions of the next ones)
    live = [L - d * P for L, d in zip(lens, drop)]
    for ntok in ([1, 2, 1, 3], [2, 1, 1, 1]):
        x = rng.standard_normal((sum(ntok), d_model), dtype=np.float32)
        q = c.ProjectAppend(0, torch.from_numpy(x).to(gpu), wp, H, rope=rope, seq_ids=list(range(S)),
                            n_tok=ntok, rope_mode="offset").cpu().numpy()
        pos = [h + j for h, n in zip(held, ntok) for j in range(n)]
        _check_gqa_step(c, q, x, wq, wk, wv, H, KVH, D, tables, max_seq, range(S), ntok, live, pos)
        held = [h + n for h, n in zip(held, ntok)]
        live = [L + n for L, n in zip(live, ntok)]
    if tier == "spill":
        c.Restore(list(range(S)), drop)
        live = [L + d * P for L, d in zip(live, drop)]
        for i in range(S):
            st = c.SeqState(0, i)
            assert st["pos_offset"] == 0 and st["len"] == held[i] == live[i]
            k, v = c.View(0, i)
            assert torch.equal(k[:, :, :lens[i]].view(torch.int16), before[i][0].view(torch.int16))
            assert torch.equal(v[:, :, :lens[i]].view(torch.int16), before[i][1].view(torch.int16))
        ntok = [1, 1, 2, 1]
        x = rng.standard_normal((sum(ntok), d_model), dtype=np.float32)
        q = c.ProjectAppend(0, torch.from_numpy(x).to(gpu), wp, H, rope=rope, seq_ids=list(range(S)),
                            n_tok=ntok, rope_mode="offset").cpu().numpy()
        pos = [h + j for h, n in zip(held, ntok) for j in range(n)]
        _check_gqa_step(c, q, x, wq, wk, wv, H, KVH, D, tables, max_seq, range(S), ntok, live, pos)


@pytest.mark.parametrize("tier", ["evict", "spill"])
def test_mla_project_append_positions_after_evict_and_spill(gpu, tier):
    """The MLA fused step (mla.go:279-314) after Evict + Compact / Spill /
    Restore: q_r and the appended k^R rows rotated at the absolute position
    pos_offset + live_len + j, against oracle.rope_apply there."""
    from relux_amd import MLACache, pack_mla_proj, rope_tables
    rng = np.random.default_rng(41 if tier == "evict" else 43)
    H, D, dC, dR, d_model, P, max_seq = 4, 64, 512, 64, 256, 16, 256
    lens = [50, 20, 35]
    drop = [2, 1, 1]
    S = len(lens)
    c = MLACache(num_layers=1, max_len=max_seq, d_c=dC, d_r=dR, page_tokens=P, max_seqs=S,
                 device=gpu.index)
    mats = [oracle.bf16_from_f32(rng.normal(0, 0.02, (d_model, w)).astype(np.float32))
            for w in (H * D, H * dR, dC, dR)]
    wp = pack_mla_proj(*[_bf16_tensor(m, gpu) for m in mats], H, D)
    rope = rope_tables(dR, 10000.0, max_seq, gpu)
    tables = oracle.rope_tables(dR, 10000.0, max_seq)
    for i, L in enumerate(lens):
        for t0 in range(0, L, P):
            n = min(P, L - t0)
            cc = torch.from_numpy(rng.standard_normal((n, dC), dtype=np.float32)).to(gpu)
            kr = torch.from_numpy(rng.standard_normal((n, dR), dtype=np.float32)).to(gpu)
            c.Append(0, cc, kr, seq_ids=[i], n_tok=[n])
    if tier == "evict":
        c.Evict(list(range(S)), drop)
        c.Compact()
    else:
        c.AttachSpill(sum(drop))
        c.Spill(list(range(S)), drop)
    held = list(lens)
    live = [L - d * P for L, d in zip(lens, drop)]
    steps = [[1, 2, 1], [1, 1, 3]]
    for k, ntok in enumerate(steps):
        if tier == "spill" and k == 1:
            c.Restore(list(range(S)), drop)
            live = [L + d * P for L, d in zip(live, drop)]
            assert [c.SeqState(0, i)["pos_offset"] for i in range(S)] == [0] * S
        x = rng.standard_normal((sum(ntok), d_model), dtype=np.float32)
        qn, qr = c.ProjectAppend(0, torch.from_numpy(x).to(gpu), wp, H, D, rope=rope,
                                 seq_ids=list(range(S)), n_tok=ntok, rope_mode="offset")
        pos = [h + j for h, n in zip(held, ntok) for j in range(n)]
        R = sum(ntok)
        qc_o = oracle.matmul_bf16w(x, mats[0]).reshape(R, H, D)
        qr_o = oracle.matmul_bf16w(x, mats[1]).reshape(R, H, dR)
        c_o = oracle.matmul_bf16w(x, mats[2])
        kr_o = oracle.matmul_bf16w(x, mats[3])
        for r in range(R):
            qr_o[r] = oracle.rope_apply(qr_o[r][:, None, :], pos[r], tables, max_seq)[:, 0, :]
            kr_o[r] = oracle.rope_apply(kr_o[r][None, None, :], pos[r], tables, max_seq)[0, 0, :]
        np.testing.assert_allclose(qn.cpu().numpy(), qc_o, atol=2e-4, rtol=1e-4)
        np.testing.assert_allclose(qr.cpu().numpy(), qr_o, atol=2e-4, rtol=1e-4)
        off = 0
        same = []
        for i, n in enumerate(ntok):
            cg, krg = c.View(0, i)
            assert cg.shape[1] == live[i] + n
            cg = cg[0].view(torch.int16).cpu().numpy().view(np.uint16)[live[i]:]
            krg = krg[0].view(torch.int16).cpu().numpy().view(np.uint16)[live[i]:]
            for got, want in ((cg, oracle.bf16_from_f32(c_o[off:off + n])),
                              (krg, oracle.bf16_from_f32(kr_o[off:off + n]))):
                same.append((got == want).ravel())
                np.testing.assert_allclose(oracle.f32_from_bf16(got), oracle.f32_from_bf16(want),
                                           atol=1e-2, rtol=1e-2)
            off += n
        assert np.concatenate(same).mean() > 0.99
        held = [h + n for h, n in zip(held, ntok)]
        live = [L + n for L, n in zip(live, ntok)]
