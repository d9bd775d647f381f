"""DecodeBatch: device-resident block table and cache_seqlens for a graph-captured decode batch.

Prism's batched decode (engine/executor.py:320-356) keeps static graph buffers per captured batch
size and refills them every step from the host: build_block_table writes every
block_table[i, j] and cache_seqlens[i] element by element (engine/kv_cache.py:147-151), then the
executor zeroes and copies the graph's bt / sl (:345-353) and copies one cos / sin row per
sequence (:354-356).  Padded rows point at page 0, the first page a sequence gets (:348-353), and
a sequence longer than 32 pages falls back to eager execution (:72, :343).

A DecodeBatch instead keeps the table on the device for good and sends only what changed: each
step, one small packet with the rows whose length changed and the (row, column, page) entries the
device does not hold yet (a page appended at a page boundary, a page replaced by copy-on-write,
a row handed to another sequence), applied by one pkv_table_update launch.  The table is as wide
as the pool, so no sequence length forces a new capture; padded rows append into a page reserved
for them (FlashAttnKVCache.reserve_null_page).  The rotary position of each row is its
cache_seqlens entry (the length before the append), so rope_qk reads it directly and no per-row
cos / sin copy is needed.

    db = DecodeBatch(kv, max_batch=32)
    bt, sl = db.step(seq_ids, graph_batch=32)      # before every replay (host + one launch)
    ... capture once: rope_qk(qkv, sl, cos, sin, ..., block_table=bt, cache_seqlens=sl); attention(...)
    graph.replay()
    db.advance()                                    # the step's tokens are in the cache
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .attention import _require_gpu, _stream_ptr, poll_status, status_tensor


class DecodeBatch:
    """Graph-stable decode inputs over a FlashAttnKVCache, updated incrementally on the device."""

    def __init__(self, kv, max_batch: int, max_blocks: int | None = None):
        if max_batch <= 0:
            raise ValueError("max_batch must be positive")
        self.kv = kv
        self.max_batch = max_batch
        self.max_blocks = int(max_blocks if max_blocks is not None else kv.max_pages)
        if self.max_blocks <= 0:
            raise ValueError("max_blocks must be positive")
        self.null_page = kv.reserve_null_page()
        dev = kv.device
        self.block_table = torch.full((max_batch, self.max_blocks), self.null_page, dtype=torch.int32, device=dev)
        self.cache_seqlens = torch.zeros(max_batch, dtype=torch.int32, device=dev)
        # what the device holds, per row: the sequence, a prefix of its page list, its length
        self._row_seq: list[int | None] = [None] * max_batch
        self._row_pages: list[list[int] | None] = [[self.null_page] for _ in range(max_batch)]
        self._row_len = [0] * max_batch
        self._packet_dev: torch.Tensor | None = None
        self._last: tuple[list[int], int] | None = None

    # ------------------------------------------------------------------ host planning
    def plan(self, seq_ids: list[int], graph_batch: int | None = None) -> tuple[np.ndarray, int, int]:
        """The update packet that brings rows [0, graph_batch) to this step's state: row i holds
        seq_ids[i] (its pages and its current length), rows past len(seq_ids) are padding (the
        null page, length 0).  Returns (int32 packet, n_len, n_ent) and records the new state."""
        kv = self.kv
        n_seq = len(seq_ids)
        gb = n_seq if graph_batch is None else int(graph_batch)
        if not 0 <= n_seq <= gb <= self.max_batch:
            raise ValueError(f"{n_seq} sequences in a batch of {gb} rows (at most {self.max_batch})")
        if len(set(seq_ids)) != n_seq:
            raise ValueError("a sequence appears in two rows")
        if kv.null_page != self.null_page:
            # compact() moved the pool: a fresh null page, every row rewritten
            self.null_page = kv.reserve_null_page()
            self._row_seq = [None] * self.max_batch
            self._row_pages = [None] * self.max_batch
            self._row_len = [-1] * self.max_batch
        lens: list[int] = []
        ents: list[int] = []
        for i, sid in enumerate(seq_ids):
            pages = kv.seq_pages[sid]
            n = len(pages)
            if n > self.max_blocks:
                raise RuntimeError(f"sequence {sid} holds {n} pages, more than the table's {self.max_blocks} columns")
            held = self._row_pages[i] if self._row_seq[i] == sid else None
            if held is None:
                for j, pg in enumerate(pages):
                    ents += (i, j, pg)
                self._row_pages[i] = list(pages)
            elif held != pages:
                m = min(len(held), n)
                start = m if held[:m] == pages[:m] else next(j for j in range(m) if held[j] != pages[j])
                for j in range(start, n):
                    if j >= len(held) or held[j] != pages[j]:
                        ents += (i, j, pages[j])
                self._row_pages[i] = list(pages)
            self._row_seq[i] = sid
            length = kv.seq_len[sid]
            if self._row_len[i] != length:
                lens += (i, length)
                self._row_len[i] = length
        for i in range(n_seq, gb):
            if self._row_seq[i] is not None or self._row_pages[i] is None or self._row_pages[i][0] != self.null_page:
                ents += (i, 0, self.null_page)
                self._row_seq[i] = None
                self._row_pages[i] = [self.null_page]
            if self._row_len[i] != 0:
                lens += (i, 0)
                self._row_len[i] = 0
        packet = np.asarray(lens + ents, dtype=np.int32)
        return packet, len(lens) // 2, len(ents) // 3

    # ------------------------------------------------------------------ device
    def apply(self, packet: np.ndarray, n_len: int, n_ent: int, status: torch.Tensor | None = None) -> None:
        """One host-to-device copy of the packet and one pkv_table_update launch, on the current
        stream (nothing if the packet is empty)."""
        if n_len + n_ent == 0:
            return
        dev = self.block_table.device
        _require_gpu(self.block_table, "block_table")
        if self._packet_dev is None or self._packet_dev.numel() < packet.size:
            self._packet_dev = torch.empty(max(packet.size, 3 * 1024), dtype=torch.int32, device=dev)
        # fresh pinned staging from torch's caching host allocator, kept alive until the copy ran
        staged = torch.from_numpy(packet).pin_memory()
        self._packet_dev[:packet.size].copy_(staged, non_blocking=True)
        st = status if status is not None else status_tensor(dev)
        rc = _lib.load().pkv_table_update(
            self._packet_dev.data_ptr(), n_len, n_ent, self.block_table.data_ptr(), self.block_table.stride(0),
            self.cache_seqlens.data_ptr(), self.max_batch, self.max_blocks, self.kv.max_pages, st.data_ptr(),
            _stream_ptr(dev))
        _lib.check(rc, "pkv_table_update")

    def step(self, seq_ids: list[int], n_new: int = 1, graph_batch: int | None = None,
             status: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Prepare one decode step of `n_new` tokens per sequence: grow each sequence (copying
        shared pages first, FlashAttnKVCache.prepare_append), send the table changes, and return
        (block_table [graph_batch, max_blocks], cache_seqlens [graph_batch]) -- views with fixed
        addresses, so a graph captured on them stays valid.  cache_seqlens holds the lengths
        before the append, which are also the new tokens' rotary positions."""
        gb = len(seq_ids) if graph_batch is None else int(graph_batch)
        poll_status(self.block_table.device)   # raises PrismKVStatusError for bits an earlier step set
        self.kv.prepare_append(list(seq_ids), n_new)
        packet, n_len, n_ent = self.plan(seq_ids, gb)
        self.apply(packet, n_len, n_ent, status)
        self._last = (list(seq_ids), n_new)
        return self.block_table[:gb], self.cache_seqlens[:gb]

    def advance(self) -> None:
        """The last step's tokens were written: advance the host lengths (the device lengths
        follow in the next step's packet)."""
        if self._last is None:
            raise RuntimeError("advance() without a step()")
        seq_ids, n_new = self._last
        self.kv.update_seqlens(seq_ids, n_new)
        self._last = None
