"""PrefixCache drop-in: share KV pages across requests with identical token prefixes.

Same surface as engine/prefix_cache.py (PrefixCache :18, CachedPrefix :134-140):
  lookup(token_ids, model_name) -> (page_ids, num_cached_tokens)     (:30-69)
  store(token_ids, page_ids, model_name)                              (:71-95)
  ref_pages / unref_pages / is_cached_page / evict_lru / num_cached_pages  (:97-131)

Semantics kept from the reference: only full page_size blocks are cached (:41-45, :77); the key
of block i chains the keys of blocks 0..i-1 and the model name (:52, :58, :85-87); lookup stops
at the first miss and refreshes hits in LRU order (:60-67); store takes one reference per newly
cached page (:89-95); unref_pages returns the pages whose count reached zero (:102-111);
evict_lru drops the oldest entries and returns the pages whose count reached zero (:117-127).

Differences: the chained key is a 128-bit BLAKE2b digest over the token ids (the reference uses
Python's hash(), which is salted per process for the model-name string, so keys are now
reproducible across processes); and the cache cooperates with the FlashAttnKVCache it was built
on: pages an entry points at are never returned to the free list while the entry lives, and an
evicted entry's page goes back to the free list once no live sequence lists it.
"""
from __future__ import annotations

import hashlib
import time
from collections import Counter, OrderedDict

import numpy as np


def _chain_key(prev: bytes | None, model_name: str, block: tuple) -> bytes:
    h = hashlib.blake2b(digest_size=16)
    if prev is None:
        h.update(b"m:" + model_name.encode())
    else:
        h.update(b"k:" + prev)
    h.update(np.asarray(block, dtype=np.int64).tobytes())
    return h.digest()


class CachedPrefix:
    __slots__ = ["page_id", "token_hash", "created"]

    def __init__(self, page_id: int, token_hash, created: float):
        self.page_id = page_id
        self.token_hash = token_hash
        self.created = created


class PrefixCache:
    """Caches KV pages for shared token prefixes (engine/prefix_cache.py:18)."""

    def __init__(self, kv_cache, page_size: int = 256):
        self.kv = kv_cache
        self.page_size = page_size
        self._cache: OrderedDict[bytes, CachedPrefix] = OrderedDict()
        self._page_refs: dict[int, int] = {}
        self._entry_count: Counter = Counter()   # page -> number of entries pointing at it
        if kv_cache is not None and hasattr(kv_cache, "prefix_cache"):
            kv_cache.prefix_cache = self

    def _full_blocks(self, token_ids):
        P = self.page_size
        return [tuple(token_ids[i:i + P]) for i in range(0, len(token_ids) - P + 1, P)]

    def lookup(self, token_ids: list[int], model_name: str) -> tuple[list[int], int]:
        if not token_ids:
            return [], 0
        pages: list[int] = []
        n = 0
        key = None
        for block in self._full_blocks(token_ids):
            key = _chain_key(key, model_name, block)
            entry = self._cache.get(key)
            if entry is None:
                break
            pages.append(entry.page_id)
            n += self.page_size
            self._cache.move_to_end(key)
        return pages, n

    def store(self, token_ids: list[int], page_ids: list[int], model_name: str) -> None:
        key = None
        for i, block in enumerate(self._full_blocks(token_ids)):
            key = _chain_key(key, model_name, block)
            if key not in self._cache and i < len(page_ids):
                pid = page_ids[i]
                self._cache[key] = CachedPrefix(page_id=pid, token_hash=key, created=time.time())
                self._entry_count[pid] += 1
                self._page_refs[pid] = self._page_refs.get(pid, 0) + 1

    def ref_pages(self, page_ids: list[int]) -> None:
        for pid in page_ids:
            self._page_refs[pid] = self._page_refs.get(pid, 0) + 1

    def unref_pages(self, page_ids: list[int]) -> list[int]:
        freeable = []
        for pid in page_ids:
            if pid in self._page_refs:
                self._page_refs[pid] -= 1
                if self._page_refs[pid] <= 0:
                    del self._page_refs[pid]
                    freeable.append(pid)
        return freeable

    def is_cached_page(self, page_id: int) -> bool:
        return self._page_refs.get(page_id, 0) > 0

    def evict_lru(self, num_pages: int = 1) -> list[int]:
        freed = []
        while len(freed) < num_pages and self._cache:
            _, entry = self._cache.popitem(last=False)
            pid = entry.page_id
            self._entry_count[pid] -= 1
            if self._entry_count[pid] <= 0:
                del self._entry_count[pid]
            if pid in self._page_refs:
                self._page_refs[pid] -= 1
                if self._page_refs[pid] <= 0:
                    del self._page_refs[pid]
                    freed.append(pid)
            if self.kv is not None and hasattr(self.kv, "_on_entry_dropped"):
                self.kv._on_entry_dropped(pid)
        return freed

    @property
    def num_cached_pages(self) -> int:
        return len(self._cache)

    # ---- cooperation with FlashAttnKVCache (no counterpart in the reference) ----
    def has_entry_for(self, page_id: int) -> bool:
        return self._entry_count.get(page_id, 0) > 0

    def entry_pages(self) -> list[int]:
        """Page of every entry, LRU order (oldest first)."""
        return [e.page_id for e in self._cache.values()]

    def remap_pages(self, remap: dict[int, int]) -> None:
        """Rewrite page ids after the KV pages moved (FlashAttnKVCache.migrate_to / compact)."""
        for entry in self._cache.values():
            entry.page_id = remap[entry.page_id]
        self._page_refs = {remap.get(p, p): n for p, n in self._page_refs.items()}
        self._entry_count = Counter({remap[p]: n for p, n in self._entry_count.items()})

    def clear(self) -> None:
        self._cache.clear()
        self._page_refs.clear()
        self._entry_count.clear()
