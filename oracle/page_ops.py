"""ORACLE (test infrastructure): page copy / copy-on-write / compaction restated on uint16 bits.

The reference moves KV pages only in FlashAttnKVCache.transfer_sequence
(engine/kv_cache.py:189-207): for every layer and every used page i,
    target.k_caches[layer][dst_pages[i]].copy_(self.k_caches[layer][src_pages[i]])  (same for V).
The copy-on-write of a partially filled shared page and the compaction of live pages into a fresh
pool are this build's extensions of that primitive (both bit-exact copies):
  * cow:      dst[layer][new_page, :fill] = src[layer][old_page, :fill]; rows >= fill untouched;
  * compact:  live pages p_0 < ... are packed into pages 0..n-1 of a fresh pool.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

import numpy as np


def copy_pages(src_pools: list[np.ndarray], dst_pools: list[np.ndarray], src_ids, dst_ids, fill=None) -> list[np.ndarray]:
    """Return copies of dst_pools with dst[i][dst_ids[p], :fill[p]] = src[i][src_ids[p], :fill[p]]."""
    out = [d.copy() for d in dst_pools]
    for i, s in enumerate(src_pools):
        for p, (a, b) in enumerate(zip(src_ids, dst_ids)):
            f = s.shape[1] if fill is None else int(fill[p])
            out[i][int(b), :f] = s[int(a), :f]
    return out


def transfer_sequence(src_pools, dst_pools, src_pages, dst_pages, seq_len: int, page_size: int):
    """engine/kv_cache.py:183-207: copy the first ceil(seq_len / P) pages, page by page."""
    n = (seq_len + page_size - 1) // page_size
    return copy_pages(src_pools, dst_pools, src_pages[:n], dst_pages[:n])


def compact(src_pools: list[np.ndarray], live_pages, dst_num_pages: int) -> tuple[list[np.ndarray], dict[int, int]]:
    """Pack live pages (in the given order) into pages 0..n-1 of zeroed fresh pools."""
    remap = {int(p): i for i, p in enumerate(live_pages)}
    dst = [np.zeros((dst_num_pages,) + s.shape[1:], dtype=s.dtype) for s in src_pools]
    for i, s in enumerate(src_pools):
        for p, n in remap.items():
            dst[i][n] = s[p]
    return dst, remap
