"""FlashAttnKVCache drop-in: Prism's paged KV-cache allocator over the MI355X HIP kernels.

Keeps the attribute and method surface of engine/kv_cache.py (FlashAttnKVCache, :15-209) so
Prism's executor and scheduler can use it unchanged:

  k_caches / v_caches    per-layer [max_pages, page_size, n_kv, head_dim] bf16 tensors (:37-46),
                         here views into one [L, max_pages, ...] pool per K and V so a single
                         kernel launch can move pages of every layer
  free_pages             LIFO free list, initially [max_pages-1, ..., 0] (:49)
  seq_pages / seq_len / seq_owner                                      (:52-54)
  pages_used, pages_free, new_sequence, free_sequence, free_model_sequences, free_all,
  sequences_for_model, memory_used_by_model, get_seq_len, _ensure_capacity, build_block_table,
  update_seqlens, has_capacity, transfer_sequence                      (:63-209)

Deliberate differences (each fixes a defect of the reference or extends it):
  * running out of pages raises KVCacheOutOfPages, a subclass of both RuntimeError (what
    _ensure_capacity raises, :120) and IndexError (what new_sequence's list.pop raised, :79, :82);
  * pages a PrefixCache entry still points at are not returned to the free list by
    free_sequence (the reference frees them while cached, :87-89); they go back when the entry is
    evicted and no live sequence lists them;
  * a page is shared when more than one live sequence lists it (fork_sequence) or a prefix-cache
    entry points at it.  Before a write lands in a shared page, _ensure_capacity /
    prepare_append copy it to a fresh page (copy-on-write, only the filled slots, every layer,
    K and V, one kernel launch for the whole batch);
  * build_block_table writes the whole [B, max_blocks] slice with one host-to-device copy (the
    reference writes element by element, :147-151); columns past a sequence's pages are -1, so a
    write through a column the sequence was never given (the reference executor's decode
    capacity is one token short, engine/executor.py:206) is skipped and flagged
    (PKV_STATUS_BAD_PAGE) instead of landing in page 0, the first page the allocator hands out;
  * transfer_sequence moves all pages of all layers with one kernel launch (the reference issues
    2 * L * pages copy_ calls, :189-207); migrate_to / compact move every live page (sequences
    and prefix-cache pages) into another pool, packed, rewriting page ids everywhere.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .attention import poll_status, status_tensor


def shared_prefix_pages(bt_host: np.ndarray, sl_host: np.ndarray, page_size: int) -> int:
    """Leading block-table columns that every row of a batch of two or more lists the same page
    in, counting only pages that every sequence fills (sl >= (c + 1) * page_size): the prefix
    cascade attention may read once for the batch (branches of one prompt, prefix-cache hits)."""
    if bt_host.shape[0] < 2 or bt_host.shape[1] == 0:
        return 0
    same = (bt_host == bt_host[0:1]).all(axis=0) & (bt_host[0] >= 0)
    k = int(same.argmin()) if not same.all() else int(same.size)
    return min(k, int(sl_host.min()) // page_size)


class KVCacheOutOfPages(RuntimeError, IndexError):
    """No free KV page left (is-a RuntimeError and an IndexError, matching both reference paths)."""


class FlashAttnKVCache:
    """Paged KV cache backed by flash_attn's block-table format (engine/kv_cache.py:15)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_pages: int, page_size: int,
                 device: str, dtype: torch.dtype = torch.bfloat16):
        if max_pages <= 0 or page_size <= 0 or num_layers <= 0:
            raise ValueError("num_layers, max_pages and page_size must be positive")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_pages = max_pages
        self.page_size = page_size
        self.device = device
        self.dtype = dtype

        shape = (num_layers, max_pages, page_size, num_kv_heads, head_dim)
        self.k_pool = torch.zeros(shape, dtype=dtype, device=device)
        self.v_pool = torch.zeros(shape, dtype=dtype, device=device)
        self.k_caches = list(self.k_pool.unbind(0))
        self.v_caches = list(self.v_pool.unbind(0))

        self.free_pages = list(range(max_pages - 1, -1, -1))
        self.seq_pages: dict[int, list[int]] = {}
        self.seq_len: dict[int, int] = {}
        self.seq_owner: dict[int, str] = {}
        self._holders: dict[int, int] = {}     # page -> number of live sequences listing it
        self.prefix_cache = None               # set by PrefixCache(kv)
        self._bases: torch.Tensor | None = None
        self.null_page: int | None = None      # reserve_null_page()

        self._max_blocks_per_seq = 32
        self._block_table_buf = torch.zeros(1, self._max_blocks_per_seq, dtype=torch.int32, device=device)
        self._seqlens_buf = torch.zeros(1, dtype=torch.int32, device=device)

    # ------------------------------------------------------------------ accounting
    @property
    def pages_used(self) -> int:
        return self.max_pages - len(self.free_pages)

    @property
    def pages_free(self) -> int:
        return len(self.free_pages)

    @property
    def bytes_per_page(self) -> int:
        """Bytes of one page of one layer of K (or V)."""
        return self.page_size * self.num_kv_heads * self.head_dim * self.k_pool.element_size()

    def _pop_page(self) -> int:
        if not self.free_pages:
            raise KVCacheOutOfPages(f"Out of KV cache pages ({self.max_pages} total)")
        return self.free_pages.pop()

    def _all_pages_free(self) -> list[int]:
        return [p for p in range(self.max_pages - 1, -1, -1) if p != self.null_page]

    def reserve_null_page(self) -> int:
        """Take one page off the free list for good and return its id (the same id on every call).

        Padded rows of a graph-captured batch point their block table at it, so the dummy K/V
        their append writes never lands in a page a sequence owns.  The reference points padded
        rows at page 0 (engine/executor.py:348-353), the first page it hands out (:49).  The
        page stays reserved through free_all; compact() reserves a fresh one in the packed pool.
        """
        if self.null_page is None:
            self.null_page = self._pop_page()
        return self.null_page

    def _hold(self, page: int) -> None:
        self._holders[page] = self._holders.get(page, 0) + 1

    def _cached(self, page: int) -> bool:
        pc = self.prefix_cache
        return pc is not None and pc.has_entry_for(page)

    def _release(self, page: int) -> None:
        n = self._holders.get(page, 0) - 1
        if n > 0:
            self._holders[page] = n
            return
        self._holders.pop(page, None)
        if not self._cached(page):
            self.free_pages.append(page)

    def _on_entry_dropped(self, page: int) -> None:
        """A prefix-cache entry stopped pointing at `page` (eviction)."""
        if self._holders.get(page, 0) == 0 and not self._cached(page) and page not in self.free_pages:
            self.free_pages.append(page)

    def is_shared(self, page: int) -> bool:
        return self._holders.get(page, 0) > 1 or self._cached(page)

    # ------------------------------------------------------------------ sequences
    def new_sequence(self, seq_id: int, owner: str = "", prefix_pages: list[int] | None = None,
                     prefix_len: int = 0) -> None:
        """Start a sequence, optionally on cached prefix pages (engine/kv_cache.py:71-85)."""
        if seq_id in self.seq_pages:
            self.free_sequence(seq_id)
        fresh = self._pop_page()
        pages = (list(prefix_pages) if prefix_pages else []) + [fresh]
        for p in pages:
            self._hold(p)
        self.seq_pages[seq_id] = pages
        self.seq_len[seq_id] = prefix_len if prefix_pages else 0
        self.seq_owner[seq_id] = owner

    def fork_sequence(self, src_seq_id: int, dst_seq_id: int, owner: str | None = None) -> None:
        """dst shares every page of src (no copy); the first write into a shared page copies it.
        Forking a sequence into itself changes nothing."""
        pages = list(self.seq_pages[src_seq_id])
        if dst_seq_id == src_seq_id:
            return
        if dst_seq_id in self.seq_pages:
            self.free_sequence(dst_seq_id)
        for p in pages:
            self._hold(p)
        self.seq_pages[dst_seq_id] = pages
        self.seq_len[dst_seq_id] = self.seq_len[src_seq_id]
        self.seq_owner[dst_seq_id] = self.seq_owner.get(src_seq_id, "") if owner is None else owner

    def free_sequence(self, seq_id: int) -> None:
        if seq_id in self.seq_pages:
            for p in self.seq_pages.pop(seq_id):
                self._release(p)
            del self.seq_len[seq_id]
            self.seq_owner.pop(seq_id, None)

    def free_model_sequences(self, model_name: str) -> None:
        for sid in [s for s, o in self.seq_owner.items() if o == model_name]:
            self.free_sequence(sid)

    def free_all(self) -> None:
        self.free_pages = self._all_pages_free()
        self.seq_pages.clear()
        self.seq_len.clear()
        self.seq_owner.clear()
        self._holders.clear()
        if self.prefix_cache is not None:
            self.prefix_cache.clear()

    def sequences_for_model(self, model_name: str) -> list[int]:
        return [s for s, o in self.seq_owner.items() if o == model_name]

    def memory_used_by_model(self, model_name: str) -> int:
        return sum(len(self.seq_pages.get(s, [])) for s in self.sequences_for_model(model_name))

    def get_seq_len(self, seq_id: int) -> int:
        return self.seq_len.get(seq_id, 0)

    def has_capacity(self, num_pages: int = 1) -> bool:
        return len(self.free_pages) >= num_pages

    # ------------------------------------------------------------------ growth + copy-on-write
    def _plan_growth(self, seq_id: int, new_total: int, cow: list) -> None:
        pages = self.seq_pages[seq_id]
        P = self.page_size
        start = self.seq_len[seq_id]
        if new_total > start:
            # pages the write [start, new_total) lands in that already exist and are shared
            for idx in range(start // P, min(len(pages), -(-new_total // P))):
                old = pages[idx]
                if self.is_shared(old):
                    fill = start - idx * P if idx == start // P else 0
                    new = self._pop_page()
                    self._hold(new)
                    pages[idx] = new
                    self._release(old)
                    if fill > 0:
                        cow.append((old, new, fill))
        need = -(-new_total // P)
        while len(pages) < need:
            p = self._pop_page()
            self._hold(p)
            pages.append(p)

    def _ensure_capacity(self, seq_id: int, new_total: int) -> None:
        """Grow to ceil(new_total / P) pages (engine/kv_cache.py:116-121), copying shared pages first."""
        cow: list = []
        self._plan_growth(seq_id, new_total, cow)
        self._copy_on_write(cow)

    def prepare_append(self, seq_ids: list[int], num_new_tokens: int | list[int]) -> int:
        """_ensure_capacity for a batch of sequences with one copy-on-write launch; returns #copies."""
        counts = [num_new_tokens] * len(seq_ids) if isinstance(num_new_tokens, int) else list(num_new_tokens)
        cow: list = []
        for sid, n in zip(seq_ids, counts):
            self._plan_growth(sid, self.seq_len[sid] + n, cow)
        self._copy_on_write(cow)
        return len(cow)

    def update_seqlens(self, seq_ids: list[int], num_new_tokens: int | list[int]) -> None:
        """engine/kv_cache.py:155-169: grow and advance seq_len after the kernel wrote the KV."""
        counts = [num_new_tokens] * len(seq_ids) if isinstance(num_new_tokens, int) else list(num_new_tokens)
        for sid, n in zip(seq_ids, counts):
            total = self.seq_len[sid] + n
            self._ensure_capacity(sid, total)
            self.seq_len[sid] = total
        if torch.device(self.device).type == "cuda":
            poll_status(self.device)

    def _copy_on_write(self, cow: list) -> None:
        if not cow:
            return
        src = [c[0] for c in cow]
        dst = [c[1] for c in cow]
        fill = [c[2] for c in cow]
        copy_pages(self, self, src, dst, fill)

    # ------------------------------------------------------------------ block tables
    def block_table_host(self, seq_ids: list[int]) -> tuple[np.ndarray, np.ndarray]:
        """[B, max_blocks] int32 table (unused columns -1) and [B] int32 seq lengths, on the host."""
        max_blocks = max(1, max(len(self.seq_pages.get(s, [1])) for s in seq_ids))
        bt = np.full((len(seq_ids), max_blocks), -1, dtype=np.int32)
        sl = np.empty(len(seq_ids), dtype=np.int32)
        for i, sid in enumerate(seq_ids):
            pages = self.seq_pages[sid]
            bt[i, :len(pages)] = pages
            sl[i] = self.seq_len[sid]
        return bt, sl

    def build_block_table(self, seq_ids: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
        """engine/kv_cache.py:123-153: views of persistent device buffers, filled in one copy."""
        batch = len(seq_ids)
        bt_host, sl_host = self.block_table_host(seq_ids)
        max_blocks = bt_host.shape[1]
        if batch > self._block_table_buf.shape[0] or max_blocks > self._block_table_buf.shape[1]:
            self._block_table_buf = torch.zeros(
                max(batch, self._block_table_buf.shape[0]), max(max_blocks, self._block_table_buf.shape[1]),
                dtype=torch.int32, device=self.device)
        if batch > self._seqlens_buf.shape[0]:
            self._seqlens_buf = torch.zeros(batch, dtype=torch.int32, device=self.device)
        bt = self._block_table_buf[:batch, :max_blocks]
        sl = self._seqlens_buf[:batch]
        pin = torch.device(self.device).type == "cuda"
        # fresh pinned staging from torch's caching host allocator, which keeps it alive until
        # the asynchronous copies have run
        staged_bt = torch.empty((batch, max_blocks), dtype=torch.int32, pin_memory=pin)
        staged_sl = torch.empty((batch,), dtype=torch.int32, pin_memory=pin)
        staged_bt.numpy()[:] = bt_host
        staged_sl.numpy()[:] = sl_host
        bt.copy_(staged_bt, non_blocking=pin)
        sl.copy_(staged_sl, non_blocking=pin)
        # the keys every sequence of the batch shares (identical leading pages, filled by all):
        # recorded with both tensors' version counters, so that flash_attn_with_kvcache can take
        # cascade attention for this table as long as neither has been written since
        shared = shared_prefix_pages(bt_host, sl_host, self.page_size) * self.page_size
        bt._pkv_shared_prefix = (shared, bt._version, sl.data_ptr(), sl._version,
                                 int(sl_host.min()) if batch else 0)
        if pin:
            poll_status(self.device)   # raises PrismKVStatusError for bits an earlier call set
        return bt, sl

    # ------------------------------------------------------------------ page movement
    def layer_bases(self) -> torch.Tensor:
        """Device uint64-as-int64 [2L]: base address of each layer's K cache, then each V cache."""
        if self._bases is None or self._bases.device != self.k_pool.device:
            ptrs = [t.data_ptr() for t in self.k_caches] + [t.data_ptr() for t in self.v_caches]
            self._bases = torch.tensor(ptrs, dtype=torch.int64, device=self.k_pool.device)
        return self._bases

    def transfer_sequence(self, seq_id: int, target_kv: "FlashAttnKVCache",
                          target_seq_id: int | None = None, staged: bool | None = None) -> int:
        """Copy a sequence's KV into another cache (engine/kv_cache.py:174-209); returns #pages.
        staged: see copy_pages (the default stages only between devices)."""
        if seq_id not in self.seq_pages:
            return 0
        dst_seq_id = target_seq_id if target_seq_id is not None else seq_id
        src_pages = self.seq_pages[seq_id]
        src_len = self.seq_len[seq_id]
        n = (src_len + self.page_size - 1) // self.page_size
        target_kv.new_sequence(dst_seq_id)
        target_kv._ensure_capacity(dst_seq_id, src_len)
        target_kv.seq_len[dst_seq_id] = src_len
        if n:
            copy_pages(self, target_kv, src_pages[:n], target_kv.seq_pages[dst_seq_id][:n], None, staged)
        return n

    def live_pages(self) -> list[int]:
        """Every page a live sequence or prefix-cache entry uses, first-use order, no repeats."""
        seen: dict[int, None] = {}
        for pages in self.seq_pages.values():
            for p in pages:
                seen.setdefault(p, None)
        if self.prefix_cache is not None:
            for p in self.prefix_cache.entry_pages():
                seen.setdefault(p, None)
        return list(seen)

    def migrate_to(self, target: "FlashAttnKVCache") -> dict[int, int]:
        """Move every live page into `target` (one launch), packed in live_pages() order.

        Sequences, owners, lengths, sharing and the attached prefix cache (ids and refcounts)
        move with the pages; this cache is left empty.  Returns {old page: new page}.
        """
        if (target.num_layers, target.num_kv_heads, target.head_dim, target.page_size, target.dtype) != \
                (self.num_layers, self.num_kv_heads, self.head_dim, self.page_size, self.dtype):
            raise RuntimeError("migrate_to needs a target cache of the same geometry")
        if target.seq_pages or target.pages_used > (target.null_page is not None):
            raise RuntimeError("migrate_to needs an empty target cache")
        live = self.live_pages()
        if len(live) > target.pages_free:
            raise KVCacheOutOfPages(f"{len(live)} live pages do not fit {target.pages_free}")
        remap = {p: target._pop_page() for p in live}
        if live:
            copy_pages(self, target, live, [remap[p] for p in live], None)
        for sid, pages in self.seq_pages.items():
            new_pages = [remap[p] for p in pages]
            for p in new_pages:
                target._hold(p)
            target.seq_pages[sid] = new_pages
            target.seq_len[sid] = self.seq_len[sid]
            target.seq_owner[sid] = self.seq_owner.get(sid, "")
        pc = self.prefix_cache
        if pc is not None:
            pc.remap_pages(remap)
            pc.kv = target
            target.prefix_cache = pc
            self.prefix_cache = None
        self.free_pages = self._all_pages_free()
        self.seq_pages.clear()
        self.seq_len.clear()
        self.seq_owner.clear()
        self._holders.clear()
        return remap

    def compact(self) -> dict[int, int]:
        """Pack every live page into pages 0..n-1 of a fresh pool of the same size, in place.

        The pool tensors are replaced (k_caches / v_caches keep their list objects but hold new
        views): HIP graphs that captured the old cache addresses must be captured again.
        """
        fresh = FlashAttnKVCache(self.num_layers, self.num_kv_heads, self.head_dim, self.max_pages,
                                 self.page_size, self.device, self.dtype)
        remap = self.migrate_to(fresh)
        self.k_pool, self.v_pool = fresh.k_pool, fresh.v_pool
        self.k_caches[:] = fresh.k_caches
        self.v_caches[:] = fresh.v_caches
        self._bases = None
        self.free_pages = fresh.free_pages
        self.seq_pages, self.seq_len, self.seq_owner = fresh.seq_pages, fresh.seq_len, fresh.seq_owner
        self._holders = fresh._holders
        if fresh.prefix_cache is not None:
            fresh.prefix_cache.kv = self
            self.prefix_cache = fresh.prefix_cache
        if self.null_page is not None:
            self.null_page = None
            self.reserve_null_page()
        return remap


def _upload(rows, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A small host table on the device without stalling the host: staged in pinned memory (torch's
    caching host allocator keeps the block until the copy has run) and copied asynchronously on
    the current stream, so copy-on-write inside a decode step does not wait for the GPU."""
    return torch.tensor(rows, dtype=dtype).pin_memory().to(device, non_blocking=True)


def copy_pages(src: FlashAttnKVCache, dst: FlashAttnKVCache, src_ids: list[int], dst_ids: list[int],
               fill: list[int] | None, staged: bool | None = None) -> None:
    """One pkv_copy_pages launch over every layer's K and V: dst[dst_ids[i]] <- src[src_ids[i]]
    (first fill[i] slots, or whole pages), asynchronous on the current stream.

    Between caches on different devices (or with staged=True on one device) the pages move by
    the staged path instead: one gather of every layer's pages into a contiguous buffer on the
    source device, one device-to-device copy of that buffer (xGMI between GPUs), one scatter
    into the target pool."""
    if not src_ids:
        return
    if src.k_pool.device.type != "cuda" or dst.k_pool.device.type != "cuda":
        raise RuntimeError("KV page copies run on the ROCm device; this cache lives on "
                           f"{src.k_pool.device}/{dst.k_pool.device} (prism_amd has no CPU path)")
    if src.bytes_per_page != dst.bytes_per_page or src.num_layers != dst.num_layers:
        raise RuntimeError("page copy between caches of different geometry")
    if staged or (staged is None and src.k_pool.device != dst.k_pool.device):
        _copy_pages_staged(src, dst, src_ids, dst_ids, fill)
        return
    dev = src.k_pool.device
    ids = _upload([list(src_ids), list(dst_ids)] + ([list(fill)] if fill is not None else []), torch.int32, dev)
    lib = _lib.load()
    slot_bytes = src.num_kv_heads * src.head_dim * src.k_pool.element_size()
    page_stride = src.k_caches[0].stride(0) * src.k_pool.element_size()
    rc = lib.pkv_copy_pages(
        src.layer_bases().data_ptr(), dst.layer_bases().data_ptr(), 2 * src.num_layers,
        ids[0].data_ptr(), ids[1].data_ptr(), ids[2].data_ptr() if fill is not None else 0, len(src_ids),
        page_stride, dst.k_caches[0].stride(0) * dst.k_pool.element_size(), slot_bytes, src.page_size,
        src.max_pages, dst.max_pages, status_tensor(dev).data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "pkv_copy_pages")


def _copy_pages_staged(src: FlashAttnKVCache, dst: FlashAttnKVCache, src_ids, dst_ids, fill) -> None:
    """Disaggregated move (engine/kv_cache.py:174-209 transfer_sequence, engine/disaggregated.py:144):
    gather on the source device into [2L, n, page] staging, one copy of the staging buffer to the
    target device (a peer copy over xGMI between GPUs; the same code on one device), scatter into
    the target pool.  Three launches for any number of layers and pages."""
    n = len(src_ids)
    L2 = 2 * src.num_layers
    page_elems = src.page_size * src.num_kv_heads * src.head_dim
    staging = torch.empty((L2, n, page_elems), dtype=src.dtype, device=src.k_pool.device)
    sbases = _upload([staging[i].data_ptr() for i in range(L2)], torch.int64, src.k_pool.device)
    ids = _upload(list(src_ids), torch.int32, src.k_pool.device)
    esz = src.k_pool.element_size()
    lib = _lib.load()
    rc = lib.pkv_gather_pages(src.layer_bases().data_ptr(), sbases.data_ptr(), L2, ids.data_ptr(), n, 0,
                              src.k_caches[0].stride(0) * esz, page_elems * esz, page_elems * esz,
                              src.max_pages, n, status_tensor(src.k_pool.device).data_ptr(),
                              torch.cuda.current_stream(src.k_pool.device).cuda_stream)
    _lib.check(rc, "pkv_gather_pages")
    remote = staging.to(dst.k_pool.device)
    rbases = _upload([remote[i].data_ptr() for i in range(L2)], torch.int64, dst.k_pool.device)
    t = _upload([list(range(n)), list(dst_ids)] + ([list(fill)] if fill is not None else []), torch.int32,
                dst.k_pool.device)
    rc = lib.pkv_copy_pages(rbases.data_ptr(), dst.layer_bases().data_ptr(), L2, t[0].data_ptr(), t[1].data_ptr(),
                            t[2].data_ptr() if fill is not None else 0, n, page_elems * esz,
                            dst.k_caches[0].stride(0) * esz, src.num_kv_heads * src.head_dim * esz, src.page_size,
                            n, dst.max_pages, status_tensor(dst.k_pool.device).data_ptr(),
                            torch.cuda.current_stream(dst.k_pool.device).cuda_stream)
    _lib.check(rc, "pkv_copy_pages")
