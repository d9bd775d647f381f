"""ORACLE (test infrastructure): the allocator and prefix-cache state machines, without tensors.

Restates the host-side bookkeeping of engine/kv_cache.py (FlashAttnKVCache) and
engine/prefix_cache.py (PrefixCache) so randomized traces of the product drop-ins can be checked
against it, and so golden traces recorded from the reference itself (tests/golden/) pin it.

Reference behaviours restated exactly (including the ones the product deliberately fixes, which
the product tests then check separately):
  * free list starts [max_pages-1, ..., 0]; allocation is list.pop() (LIFO, page 0 first)
    (kv_cache.py:49, :79, :82, :121); free appends the sequence's pages in order (:89);
  * new_sequence with prefix pages = prefix pages + one fresh page, seq_len = prefix_len
    (:77-80); without = one fresh page, seq_len = 0 (:81-84); popping an empty free list raises
    IndexError (:79, :82); _ensure_capacity raises RuntimeError when out of pages (:120);
  * free_all resets the free list to [max_pages-1, ..., 0] (:99-103);
  * build_block_table rows hold each sequence's page list (:147-151), cache_seqlens = seq_len;
    graph_staging_elementwise restates that loop plus the executor's refill of a captured
    batch's static buffers (engine/executor.py:345-356), element by element;
  * transfer_sequence copies ceil(seq_len / P) pages after new_sequence + _ensure_capacity on the
    target (:183-207);
  * PrefixCache: only full page_size blocks are hashed (:41-45, :77); the key chains
    (model, block0) -> (key, block_i) (:52, :58, :85-87); lookup stops at the first miss and
    moves hits to the LRU tail (:60-67); store adds one ref per newly cached page (:89-95);
    unref returns pages reaching <= 0 (:102-111); evict_lru pops the oldest entries (:117-127).
    The chained key is kept as the nested tuple itself (Python's hash() of it is salted per
    process, so only hit/miss behaviour is contractual).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

from collections import OrderedDict


class KVAllocatorRef:
    def __init__(self, max_pages: int, page_size: int):
        self.max_pages = max_pages
        self.page_size = page_size
        self.free_pages = list(range(max_pages - 1, -1, -1))
        self.seq_pages: dict[int, list[int]] = {}
        self.seq_len: dict[int, int] = {}
        self.seq_owner: dict[int, str] = {}

    @property
    def pages_used(self) -> int:
        return self.max_pages - len(self.free_pages)

    @property
    def pages_free(self) -> int:
        return len(self.free_pages)

    def new_sequence(self, seq_id, owner="", prefix_pages=None, prefix_len=0):
        if prefix_pages:
            fresh = self.free_pages.pop()          # IndexError when empty, as the reference
            self.seq_pages[seq_id] = list(prefix_pages) + [fresh]
            self.seq_len[seq_id] = prefix_len
        else:
            fresh = self.free_pages.pop()
            self.seq_pages[seq_id] = [fresh]
            self.seq_len[seq_id] = 0
        self.seq_owner[seq_id] = owner

    def free_sequence(self, seq_id):
        if seq_id in self.seq_pages:
            self.free_pages += self.seq_pages.pop(seq_id)
            del self.seq_len[seq_id]
            self.seq_owner.pop(seq_id, None)

    def free_model_sequences(self, model_name):
        for sid in [s for s, o in self.seq_owner.items() if o == model_name]:
            self.free_sequence(sid)

    def free_all(self):
        self.free_pages = list(range(self.max_pages - 1, -1, -1))
        self.seq_pages.clear()
        self.seq_len.clear()
        self.seq_owner.clear()

    def sequences_for_model(self, model_name):
        return [s for s, o in self.seq_owner.items() if o == model_name]

    def memory_used_by_model(self, model_name):
        return sum(len(self.seq_pages.get(s, [])) for s in self.sequences_for_model(model_name))

    def get_seq_len(self, seq_id):
        return self.seq_len.get(seq_id, 0)

    def _ensure_capacity(self, seq_id, new_total):
        need = -(-new_total // self.page_size)
        pages = self.seq_pages[seq_id]
        while len(pages) < need:
            if not self.free_pages:
                raise RuntimeError(f"Out of KV cache pages ({self.max_pages} total)")
            pages.append(self.free_pages.pop())

    def block_table(self, seq_ids):
        """Valid columns of each row of build_block_table, and cache_seqlens."""
        return [list(self.seq_pages[s]) for s in seq_ids], [self.seq_len[s] for s in seq_ids]

    def update_seqlens(self, seq_ids, num_new_tokens):
        counts = [num_new_tokens] * len(seq_ids) if isinstance(num_new_tokens, int) else list(num_new_tokens)
        for sid, n in zip(seq_ids, counts):
            total = self.seq_len[sid] + n
            self._ensure_capacity(sid, total)
            self.seq_len[sid] = total

    def has_capacity(self, num_pages=1):
        return len(self.free_pages) >= num_pages

    def transfer_sequence(self, seq_id, target: "KVAllocatorRef", target_seq_id=None):
        """Returns (pages transferred, [(src_page, dst_page), ...])."""
        if seq_id not in self.seq_pages:
            return 0, []
        dst = seq_id if target_seq_id is None else target_seq_id
        src_len = self.seq_len[seq_id]
        n = -(-src_len // self.page_size)
        target.new_sequence(dst)
        target._ensure_capacity(dst, src_len)
        target.seq_len[dst] = src_len
        return n, list(zip(self.seq_pages[seq_id][:n], target.seq_pages[dst][:n]))


def graph_staging_elementwise(bt, sl, graph_bt, graph_sl, seq_pages, seq_len, seq_ids,
                              cos=None, sin=None, graph_cos=None, graph_sin=None):
    """The reference's per-step refill of a captured decode batch's inputs, one element at a time
    on whatever tensors are passed (device tensors on the GPU box, so each write is its own
    host-to-device copy, as in the reference):

      build_block_table (engine/kv_cache.py:147-151): bt[i, j] = page; sl[i] = seq_len[sid]
      batched_decode_step (engine/executor.py:345-356): graph_bt[:] = 0; graph_bt[:B, :nb] = bt;
          graph_sl[:] = 0; graph_sl[:B] = sl; graph_cos[i, 0] = cos[pos_i]; graph_sin[i, 0] = sin[pos_i]

    bt / sl are the persistent build buffers (at least [B, max pages] / [B]); cos / sin are
    [n_pos, hd] tables and graph_cos / graph_sin [rows, 1, hd] (optional).  Timed as the
    reference-side cost of DecodeBatch.step; tests pin the resulting rows against block_table().
    """
    B = len(seq_ids)
    nb = max(1, max(len(seq_pages[s]) for s in seq_ids)) if seq_ids else 1
    for i, sid in enumerate(seq_ids):
        for j, page in enumerate(seq_pages[sid]):
            bt[i, j] = page
        sl[i] = seq_len[sid]
    graph_bt[:] = 0
    graph_bt[:B, :nb] = bt[:B, :nb]
    graph_sl[:] = 0
    graph_sl[:B] = sl[:B]
    if cos is not None:
        for i, sid in enumerate(seq_ids):
            graph_cos[i, 0].copy_(cos[seq_len[sid]])
            graph_sin[i, 0].copy_(sin[seq_len[sid]])


class PrefixCacheRef:
    def __init__(self, page_size: int = 256):
        self.page_size = page_size
        self._cache: OrderedDict = OrderedDict()   # chained key -> page id
        self._page_refs: dict[int, int] = {}

    def _blocks(self, token_ids):
        P = self.page_size
        return [tuple(token_ids[i:i + P]) for i in range(0, len(token_ids) - P + 1, P)]

    def lookup(self, token_ids, model_name):
        if not token_ids:
            return [], 0
        pages, n = [], 0
        key = None
        for blk in self._blocks(token_ids):
            key = (model_name, blk) if key is None else (key, blk)
            if key not in self._cache:
                break
            pages.append(self._cache[key])
            n += self.page_size
            self._cache.move_to_end(key)
        return pages, n

    def store(self, token_ids, page_ids, model_name):
        key = None
        for i, blk in enumerate(self._blocks(token_ids)):
            key = (model_name, blk) if key is None else (key, blk)
            if key not in self._cache and i < len(page_ids):
                self._cache[key] = page_ids[i]
                self._page_refs[page_ids[i]] = self._page_refs.get(page_ids[i], 0) + 1

    def ref_pages(self, page_ids):
        for p in page_ids:
            self._page_refs[p] = self._page_refs.get(p, 0) + 1

    def unref_pages(self, page_ids):
        freeable = []
        for p in page_ids:
            if p in self._page_refs:
                self._page_refs[p] -= 1
                if self._page_refs[p] <= 0:
                    del self._page_refs[p]
                    freeable.append(p)
        return freeable

    def is_cached_page(self, page_id):
        return self._page_refs.get(page_id, 0) > 0

    def evict_lru(self, num_pages=1):
        freed = []
        while len(freed) < num_pages and self._cache:
            _, page = self._cache.popitem(last=False)
            if page in self._page_refs:
                self._page_refs[page] -= 1
                if self._page_refs[page] <= 0:
                    del self._page_refs[page]
                    freed.append(page)
        return freed

    @property
    def num_cached_pages(self):
        return len(self._cache)

    def lru_pages(self):
        return list(self._cache.values())
