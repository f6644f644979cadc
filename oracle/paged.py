"""Page-table state model -- TEST INFRASTRUCTURE ONLY.

relux has no paging (its caches are contiguous per-layer buffers with a
cursor, kvcache.go:34-49, mla_cache.go:21-35).  This module states the
paged semantics the HIP library must reproduce bit for bit, in plain
Python, and keeps the logical token rows so that the contiguous view the
reference would hold (KVCache.View after the same appends) can be compared
byte for byte with the library's paged gather.

Specification:
  * per layer, a pool of `pool_pages` pages and a LIFO free stack that
    initially hands out pages 0, 1, 2, ...;
  * per (layer, sequence): live length, first live table entry, position
    offset, pages in use, and a table row of `max_pages` entries (-1 empty);
  * append: sequences in call order, tokens ascending; a page is popped
    when a token lands on slot 0; the call fails without any change on
    overflow (first + ceil(len/P) > max_pages) or pool exhaustion;
  * rollback(n): len -= n; pages beyond ceil(len/P) are pushed back last
    page first, so append(a||b); rollback(|b|) == append(a);
  * evict(k): the oldest k FULL pages are pushed oldest first; first += k,
    len -= k*P, pos_offset += k*P;
  * compact: live entries move to the front of the row, the rest become -1;
  * release: every page pushed back last page first, state cleared, the
    sequence's spilled slots returned newest first;
  * host spill tier of `host_slots` slots (LIFO free list handing out 0, 1,
    2, ...): spill(k) is evict(k) whose pages' rows move to tier slots
    (taken oldest page first, appended to the sequence's spilled list);
    restore(k) pops the k newest spilled pages, newest first, each into a
    page popped from the free stack at table entry first - k + j (live
    entries move right to [k, k + pages) when first < k), first -= k,
    len += k*P, pos_offset -= k*P, and returns each slot to the tier as it
    goes; evict of a sequence with spilled pages also returns those slots
    (newest first), since they would no longer adjoin its resident tokens.
The invariants that pin this model are asserted in tests/test_paged_model.py.
"""
import numpy as np


class PagedOverflow(Exception):
    pass


class PagedPoolExhausted(Exception):
    pass


class PagedStateError(Exception):
    pass


class PagedModel:
    def __init__(self, layers, page_tokens, pool_pages, max_seqs, max_pages, host_slots=0):
        self.layers = layers
        self.P = page_tokens
        self.pool_pages = pool_pages
        self.max_seqs = max_seqs
        self.max_pages = max_pages
        self.host_slots = host_slots
        self.reset()

    def reset(self):
        L, S = self.layers, self.max_seqs
        self.free = [list(range(self.pool_pages - 1, -1, -1)) for _ in range(L)]
        self.table = [np.full((S, self.max_pages), -1, np.int32) for _ in range(L)]
        self.len = np.zeros((L, S), np.int64)
        self.first = np.zeros((L, S), np.int64)
        self.pos_offset = np.zeros((L, S), np.int64)
        self.pages = np.zeros((L, S), np.int64)
        self.rows = [[[] for _ in range(S)] for _ in range(L)]  # live token payloads
        self.host_free = list(range(self.host_slots - 1, -1, -1))
        # spilled[l][s]: (slot, rows of the page) per spilled page, oldest first
        self.spilled = [[[] for _ in range(S)] for _ in range(L)]

    def _layers(self, layer):
        return range(self.layers) if layer == -1 else [layer]

    def append(self, layer, seq_ids, n_tok, payloads=None):
        """payloads[i] is a list of n_tok[i] per-token objects (stored for
        gather comparisons)."""
        need = 0
        for s, n in zip(seq_ids, n_tok):
            new_len = self.len[layer, s] + n
            pages_after = -(-new_len // self.P)
            if self.first[layer, s] + pages_after > self.max_pages:
                raise PagedOverflow(f"layer {layer} seq {s}")
            need += pages_after - self.pages[layer, s]
        if need > len(self.free[layer]):
            raise PagedPoolExhausted(f"layer {layer} needs {need}")
        for i, (s, n) in enumerate(zip(seq_ids, n_tok)):
            for j in range(n):
                pos = int(self.len[layer, s]) + j
                if pos % self.P == 0:
                    page = self.free[layer].pop()
                    self.table[layer][s, self.first[layer, s] + pos // self.P] = page
                    self.pages[layer, s] += 1
            self.len[layer, s] += n
            if payloads is not None:
                self.rows[layer][s].extend(payloads[i])

    def token_location(self, layer, seq, t):
        """(page, slot) of live token t."""
        k = self.first[layer, seq] + t // self.P
        return int(self.table[layer][seq, k]), t % self.P

    def rollback(self, layer, seq, n):
        for l in self._layers(layer):
            if n > self.len[l, seq]:
                raise PagedStateError("rollback beyond stored tokens")
        for l in self._layers(layer):
            self.len[l, seq] -= n
            keep = -(-int(self.len[l, seq]) // self.P)
            for k in range(int(self.pages[l, seq]) - 1, keep - 1, -1):
                idx = self.first[l, seq] + k
                self.free[l].append(int(self.table[l][seq, idx]))
                self.table[l][seq, idx] = -1
            self.pages[l, seq] = keep
            if n:
                del self.rows[l][seq][len(self.rows[l][seq]) - n:]

    def _release_spilled(self, l, seq):
        for slot, _ in reversed(self.spilled[l][seq]):
            self.host_free.append(slot)
        self.spilled[l][seq] = []

    def evict(self, layer, seq, n_pages):
        for l in self._layers(layer):
            if n_pages > self.len[l, seq] // self.P:
                raise PagedStateError("evicting more than the full pages")
        for l in self._layers(layer):
            if n_pages > 0:
                self._release_spilled(l, seq)
            for k in range(n_pages):
                idx = self.first[l, seq] + k
                self.free[l].append(int(self.table[l][seq, idx]))
                self.table[l][seq, idx] = -1
            self.first[l, seq] += n_pages
            self.pages[l, seq] -= n_pages
            self.len[l, seq] -= n_pages * self.P
            self.pos_offset[l, seq] += n_pages * self.P
            del self.rows[l][seq][: n_pages * self.P]

    def compact(self, layer):
        for l in self._layers(layer):
            for s in range(self.max_seqs):
                f = int(self.first[l, s])
                if f == 0:
                    continue
                n = int(self.pages[l, s])
                row = self.table[l][s]
                live = row[f:f + n].copy()
                row[:] = -1
                row[:n] = live
                self.first[l, s] = 0

    def release(self, layer, seq):
        for l in self._layers(layer):
            for k in range(int(self.pages[l, seq]) - 1, -1, -1):
                idx = self.first[l, seq] + k
                self.free[l].append(int(self.table[l][seq, idx]))
                self.table[l][seq, idx] = -1
            self._release_spilled(l, seq)
            self.len[l, seq] = self.first[l, seq] = self.pos_offset[l, seq] = self.pages[l, seq] = 0
            self.rows[l][seq] = []

    def spill(self, layer, seq_ids, n_pages):
        """Move the oldest n_pages[i] full pages of seq_ids[i] to the host
        tier (device state == evict)."""
        ls = list(self._layers(layer))
        need = 0
        for s, n in zip(seq_ids, n_pages):
            for l in ls:
                if n > self.len[l, s] // self.P:
                    raise PagedStateError("spilling more than the full pages")
            need += n * len(ls)
        if need > len(self.host_free):
            raise PagedPoolExhausted("spill tier full")
        for s, n in zip(seq_ids, n_pages):
            for l in ls:
                for k in range(n):
                    idx = self.first[l, s] + k
                    slot = self.host_free.pop()
                    self.spilled[l][s].append((slot, self.rows[l][s][k * self.P:(k + 1) * self.P]))
                    self.free[l].append(int(self.table[l][s, idx]))
                    self.table[l][s, idx] = -1
                self.first[l, s] += n
                self.pages[l, s] -= n
                self.len[l, s] -= n * self.P
                self.pos_offset[l, s] += n * self.P
                del self.rows[l][s][: n * self.P]

    def restore(self, layer, seq_ids, n_pages):
        ls = list(self._layers(layer))
        if len(set(seq_ids)) != len(seq_ids):
            raise PagedStateError("sequence listed twice")
        for l in ls:
            need = 0
            for s, n in zip(seq_ids, n_pages):
                if n > len(self.spilled[l][s]):
                    raise PagedStateError("restoring more than spilled")
                if max(int(self.first[l, s]), n) + int(self.pages[l, s]) > self.max_pages:
                    raise PagedOverflow("restore exceeds the table row")
                need += n
            if need > len(self.free[l]):
                raise PagedPoolExhausted("restore needs pages")
        for s, n in zip(seq_ids, n_pages):
            if n == 0:
                continue
            for l in ls:
                row = self.table[l][s]
                f, pg = int(self.first[l, s]), int(self.pages[l, s])
                if f < n:
                    live = row[f:f + pg].copy()
                    row[f:f + pg] = -1
                    row[n:n + pg] = live
                    self.first[l, s] = f = n
                back = []
                for k in range(n - 1, -1, -1):
                    slot, prow = self.spilled[l][s].pop()
                    row[f - n + k] = self.free[l].pop()
                    self.host_free.append(slot)
                    back.append(prow)
                for prow in back:  # newest first -> prepend in that order
                    self.rows[l][s][:0] = prow
                self.first[l, s] -= n
                self.pages[l, s] += n
                self.len[l, s] += n * self.P
                self.pos_offset[l, s] -= n * self.P

    def state(self, layer, seq):
        return {"len": int(self.len[layer, seq]), "first": int(self.first[layer, seq]),
                "pos_offset": int(self.pos_offset[layer, seq]), "pages": int(self.pages[layer, seq])}
