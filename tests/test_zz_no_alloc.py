"""rlx_gqa_attend_noalloc (the decode / verify attention that allocates
nothing) against rlx_gqa_attend, through the C ABI.  Both run the same
kernels on the same plans, so the outputs must be identical bit for bit;
a torch f32 attention over the generated K/V bounds both.  Two calls in a
row share the device scratch, the second smaller than the first and made
with page-table writes still pending (a rollback that emptied pages)."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _fill(c, gpu, lens, KVH, D, gen):
    """Append lens[i] bf16 tokens to sequence i; returns the logical K/V."""
    ks, vs = [], []
    k = torch.randn(sum(lens), KVH, D, device=gpu, generator=gen).bfloat16()
    v = torch.randn(sum(lens), KVH, D, device=gpu, generator=gen).bfloat16()
    c.Append(0, k, v, seq_ids=list(range(len(lens))), n_tok=list(lens), layout="SHD")
    off = 0
    for L in lens:
        ks.append(k[off:off + L])
        vs.append(v[off:off + L])
        off += L
    return ks, vs


def _torch_ref(ks, vs, q, nqs, H, KVH):
    g = H // KVH
    outs, off = [], 0
    for k, v, nq in zip(ks, vs, nqs):
        T = k.shape[0]
        kf = k.float().permute(1, 0, 2).repeat_interleave(g, 0)      # [H, T, D]
        vf = v.float().permute(1, 0, 2).repeat_interleave(g, 0)
        qs = q[off:off + nq].float().permute(1, 0, 2)                # [H, nq, D]
        s = torch.bmm(qs, kf.transpose(1, 2).contiguous()) / math.sqrt(k.shape[-1])
        lim = T - nq + torch.arange(nq, device=q.device)
        s = s.masked_fill(torch.arange(T, device=q.device)[None, None, :] > lim[None, :, None],
                          float("-inf"))
        outs.append(torch.bmm(torch.softmax(s, dim=-1), vf).permute(1, 0, 2))
        off += nq
    return torch.cat(outs)


def _close(got, want, tol=(1e-2, 1e-3)):
    err = (got.double() - want.double()).abs()
    assert err.max().item() <= tol[0] and err.mean().item() <= tol[1], (err.max().item(), err.mean().item())


def test_noalloc_equals_attend_two_calls(gpu):
    from relux_amd import KVCache
    gen = torch.Generator(device=gpu).manual_seed(7)
    rng = np.random.default_rng(7)
    H, KVH, D, P = 32, 8, 128, 16
    lens = [int(x) for x in rng.integers(200, 5000, size=48)]
    c = KVCache(num_layers=1, max_len=5200, num_kv_heads=KVH, head_dim=D, page_tokens=P,
                max_seqs=48, device=gpu.index)
    ks, vs = _fill(c, gpu, lens, KVH, D, gen)
    seqs = list(range(48))
    # call 1: 48 sequences, one bf16 query each, bf16 output
    q = torch.randn(48, H, D, device=gpu, generator=gen).bfloat16()
    out_n = torch.empty(48, H, D, device=gpu, dtype=torch.bfloat16)
    c.AttendNoAlloc(0, q, H, out_n, seq_ids=seqs)
    out_a = c.Attend(0, q, H, seq_ids=seqs, out_dtype=torch.bfloat16)
    assert torch.equal(out_n, out_a)
    _close(out_n.float(), _torch_ref(ks, vs, q, [1] * 48, H, KVH))
    # call 2, smaller: 5 sequences with 4 f32 draft queries each (32 rows per
    # kv head, two query tiles), after a rollback that empties pages so that
    # table writes are pending when the no-alloc call starts
    sub = [3, 11, 20, 31, 47]
    drop = [P + 1, 0, 2 * P, 5, P]
    c.Rollback(sub, drop)
    ks2 = [ks[s][:lens[s] - d] for s, d in zip(sub, drop)]
    vs2 = [vs[s][:lens[s] - d] for s, d in zip(sub, drop)]
    q2 = torch.randn(5 * 4, H, D, device=gpu, generator=gen)
    out2_n = torch.empty(5 * 4, H, D, device=gpu)
    c.AttendNoAlloc(0, q2, H, out2_n, seq_ids=sub, n_q=[4] * 5)
    out2_a = c.Attend(0, q2, H, seq_ids=sub, n_q=[4] * 5)
    assert torch.equal(out2_n, out2_a)
    _close(out2_n, _torch_ref(ks2, vs2, q2, [4] * 5, H, KVH))
    # the device table the no-alloc call patched equals the host's
    for s in sub:
        st = c.SeqState(0, s)
        row = c.PageTable(0, s)
        assert all(x >= 0 for x in row[st["first"]:st["first"] + st["pages"]])
        assert all(x == -1 for x in row[st["first"] + st["pages"]:])
    c.close()


def test_noalloc_query_tiles_and_limits(gpu):
    from relux_amd import KVCache, _lib
    gen = torch.Generator(device=gpu).manual_seed(8)
    # head_dim 16, 40 queries x 2 heads per kv head: query tiles through the
    # decode kernel (rows = tiles), as rlx_gqa_attend runs them
    H, KVH, D = 4, 2, 16
    c = KVCache(num_layers=1, max_len=128, num_kv_heads=KVH, head_dim=D, max_seqs=2,
                device=gpu.index)
    _fill(c, gpu, [100, 60], KVH, D, gen)
    q = torch.randn(80, H, D, device=gpu, generator=gen)
    out_n = torch.empty_like(q)
    c.AttendNoAlloc(0, q, H, out_n, seq_ids=[0, 1], n_q=[40, 40])
    assert torch.equal(out_n, c.Attend(0, q, H, seq_ids=[0, 1], n_q=[40, 40]))
    c.close()
    # limits: more than 64 rows, and prefill-sized calls, are refused
    c = KVCache(num_layers=1, max_len=256, num_kv_heads=8, head_dim=128, max_seqs=65,
                device=gpu.index)
    _fill(c, gpu, [70] * 65, 8, 128, gen)
    q = torch.randn(65, 32, 128, device=gpu, generator=gen)
    out = torch.zeros_like(q)
    with pytest.raises(_lib.ReluxError) as e:
        c.AttendNoAlloc(0, q, 32, out, seq_ids=list(range(65)))
    assert e.value.code == _lib.RLX_ERR_UNSUPPORTED
    q = torch.randn(64, 32, 128, device=gpu, generator=gen)
    with pytest.raises(_lib.ReluxError) as e:
        c.AttendNoAlloc(0, q, 32, torch.zeros_like(q), seq_ids=[0], n_q=[64])
    assert e.value.code == _lib.RLX_ERR_UNSUPPORTED
    assert torch.count_nonzero(out).item() == 0   # nothing ran
    c.close()
