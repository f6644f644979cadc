"""Write the golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_fixtures.py

cfg1_tiny_decoder.npz  config-1 tiny GQA decoder (oracle/tiny_decoder.py):
                       prompt, greedy tokens and per-step logits in the
                       reference (compat) cache semantics and in the corrected
                       semantics, per-layer K/V cache bytes in both layouts,
                       a digest of the seeded weights.
paged_script.npz       a scripted append / rollback / evict / compact /
                       release sequence on the page-table model
                       (oracle/paged.py) with the expected page table, length,
                       first-entry and free list after every operation.
bf16_fastexp.npz       BF16FromF32 over edge-case bit patterns and fastexp32
                       over a grid of arguments.

The tests regenerate each fixture and require identical bytes, and the GPU
tests replay the paged script and the decoder against them.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from oracle import paged, tiny_decoder as td  # noqa: E402


def weights_digest(W):
    h = hashlib.sha256()
    h.update(W["embed"].tobytes())
    for Wl in W["layers"]:
        for key in sorted(Wl):
            h.update(Wl[key].tobytes())
    for key in ("norm_f", "lm_w", "lm_b"):
        h.update(W[key].tobytes())
    return h.hexdigest()


def cfg1_fixture():
    m = td.TinyDecoder(td.CFG1, seed=0)
    prompt = td.prompt_ids(td.CFG1)
    ref = td.RefCache(m.cfg)
    tok_ref, log_ref, _ = m.generate(prompt, 16, ref)
    logical = td.LogicalCache(m.cfg)
    tok_log, log_log, gap = m.generate(prompt, 16, logical)
    T = ref.len[0]
    L = m.cfg["layers"]
    kv_ref = np.stack([np.stack([ref.k[l][:T * 32], ref.v[l][:T * 32]]) for l in range(L)])
    kv_log = np.stack([np.stack([oracle.bf16_from_f32(logical.k[l]), oracle.bf16_from_f32(logical.v[l])])
                       for l in range(L)])
    return dict(prompt=np.array(prompt, np.int32), tokens_ref=np.array(tok_ref, np.int32),
                logits_ref=log_ref.astype(np.float32), tokens=np.array(tok_log, np.int32),
                logits=log_log.astype(np.float32), kv_ref_bytes=kv_ref, kv_bytes=kv_log,
                min_top2_gap=np.float32(gap),
                weights_sha256=np.array(weights_digest(m.W)))


# (op, seq, arg): append n tokens, rollback n, evict n pages, compact, release.
PAGED_SCRIPT = [
    ("append", 0, 40), ("append", 1, 17), ("append", 2, 5), ("rollback", 0, 9),
    ("append", 1, 16), ("evict", 0, 1), ("append", 2, 30), ("compact", -1, 0),
    ("rollback", 1, 33), ("append", 0, 3), ("release", 2, 0), ("append", 1, 20),
    ("evict", 1, 1), ("compact", -1, 0), ("append", 2, 1), ("rollback", 0, 1),
]
PAGED_CFG = dict(P=16, pool_pages=16, max_seqs=3, max_pages=6)


def run_paged_script(M):
    """Replay PAGED_SCRIPT on layer 0 of a PagedModel; state after each op.
    Free stacks are listed bottom..top, padded with -1."""
    tables, lens, firsts, offs, frees = [], [], [], [], []
    for op, seq, n in PAGED_SCRIPT:
        if op == "append":
            M.append(0, [seq], [n])
        elif op == "rollback":
            M.rollback(0, seq, n)
        elif op == "evict":
            M.evict(0, seq, n)
        elif op == "compact":
            M.compact(0)
        elif op == "release":
            M.release(0, seq)
        tables.append(M.table[0].astype(np.int32).copy())
        lens.append(M.len[0].astype(np.int32).copy())
        firsts.append(M.first[0].astype(np.int32).copy())
        offs.append(M.pos_offset[0].astype(np.int32).copy())
        free = list(M.free[0])
        frees.append(np.array(free + [-1] * (PAGED_CFG["pool_pages"] - len(free)), np.int32))
    return dict(tables=np.stack(tables), lens=np.stack(lens), firsts=np.stack(firsts),
                pos_offsets=np.stack(offs), free=np.stack(frees))


def paged_fixture():
    c = PAGED_CFG
    M = paged.PagedModel(1, c["P"], c["pool_pages"], c["max_seqs"], c["max_pages"])
    return run_paged_script(M)


BF16_EDGE_BITS = np.array([
    0x00000000, 0x80000000, 0x3F800000, 0xBF800000, 0x7F800000, 0xFF800000,  # 0, 1, inf
    0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001,  # ties to even, around ties
    0x00000001, 0x007FFFFF, 0x00800000, 0x80000001,  # denormals, smallest normal
    0x7F7FFFFF, 0x7F7F8000, 0xFF7FFFFF,  # largest finite: rounds up to inf
    0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FFFFFFF, 0x7F80FFFF, 0xFF81FFFF,  # NaNs
    0x42C90000, 0x447A0000, 0xC2F7E000,  # 100.5, 1000, -123.9375
], dtype=np.uint32)


def bf16_fastexp_fixture():
    x = BF16_EDGE_BITS.view(np.float32)
    grid = np.linspace(-90.0, 90.0, 3601, dtype=np.float32)
    return dict(bf16_in_bits=BF16_EDGE_BITS, bf16_out=oracle.bf16_from_f32(x),
                fastexp_x=grid, fastexp_y=oracle.fastexp32(grid))


FIXTURES = {
    "cfg1_tiny_decoder.npz": cfg1_fixture,
    "paged_script.npz": paged_fixture,
    "bf16_fastexp.npz": bf16_fastexp_fixture,
}


def main():
    for name, fn in FIXTURES.items():
        np.savez_compressed(os.path.join(HERE, name), **fn())
        print("wrote", name)


if __name__ == "__main__":
    main()
