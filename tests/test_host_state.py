"""Host-side state of the drop-ins where they deliberately differ from the reference (CPU only).

The reference returns every page of a freed sequence to the free list even while a prefix-cache
entry still points at it (engine/kv_cache.py:87-89), and never shares a page it will write.  The
product keeps such pages off the free list, shares pages between forked sequences, and copies a
shared page before the first write into it (copy-on-write).  Page copies are recorded here by a
CPU stand-in for the kernel launcher; the kernels themselves are checked in test_gpu_pages.py.
"""
import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

import prism_amd.kv_cache as kvm
from oracle import page_ops
from oracle.paged_attention import bf16_bits
from prism_amd import FlashAttnKVCache, KVCacheOutOfPages, PrefixCache


@pytest.fixture
def copies(monkeypatch):
    """Replace the page-copy launcher with a CPU copy that records each call."""
    log = []

    def cpu_copy(src, dst, src_ids, dst_ids, fill):
        log.append((list(src_ids), list(dst_ids), None if fill is None else list(fill)))
        for i, (s, d) in enumerate(zip(src_ids, dst_ids)):
            n = src.page_size if fill is None else fill[i]
            dst.k_pool[:, d, :n] = src.k_pool[:, s, :n]
            dst.v_pool[:, d, :n] = src.v_pool[:, s, :n]

    monkeypatch.setattr(kvm, "copy_pages", cpu_copy)
    return log


def _kv(pages=16, P=16, layers=2, seed=0):
    kv = FlashAttnKVCache(layers, 1, 8, pages, P, "cpu")
    g = torch.Generator().manual_seed(seed)
    kv.k_pool.copy_(torch.randn(kv.k_pool.shape, generator=g).to(torch.bfloat16))
    kv.v_pool.copy_(torch.randn(kv.v_pool.shape, generator=g).to(torch.bfloat16))
    return kv


def _check_invariants(kv):
    free = kv.free_pages
    assert len(set(free)) == len(free), "page twice in the free list"
    held = {p for pages in kv.seq_pages.values() for p in pages}
    cached = set(kv.prefix_cache.entry_pages()) if kv.prefix_cache is not None else set()
    assert not (set(free) & held), "live page on the free list"
    assert not (set(free) & cached), "cached page on the free list"
    assert set(free) | held | cached == set(range(kv.max_pages)), "page leaked"
    for p in held:
        n = sum(pages.count(p) for pages in kv.seq_pages.values())
        assert kv._holders[p] == n
    for sid, pages in kv.seq_pages.items():
        assert len(pages) >= 1 and kv.seq_len[sid] <= len(pages) * kv.page_size


def test_out_of_pages_is_both_reference_exception_types():
    kv = _kv(pages=2)
    kv.new_sequence(0)
    kv.new_sequence(1)
    with pytest.raises(RuntimeError):
        kv.new_sequence(2)
    with pytest.raises(IndexError):
        kv._ensure_capacity(0, 100)
    assert issubclass(KVCacheOutOfPages, RuntimeError) and issubclass(KVCacheOutOfPages, IndexError)


def test_new_sequence_on_a_live_id_frees_its_pages_first():
    kv = _kv(pages=4)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 40)
    assert kv.pages_used == 3
    kv.new_sequence(0)
    assert kv.pages_used == 1 and len(kv.seq_pages[0]) == 1
    _check_invariants(kv)


def test_cached_pages_survive_free_and_return_on_eviction(copies):
    kv = _kv(pages=8, P=4)
    pc = PrefixCache(kv, page_size=4)
    kv.new_sequence(0, "m")
    kv._ensure_capacity(0, 10)
    kv.seq_len[0] = 10
    tokens = list(range(10))
    pc.store(tokens, kv.seq_pages[0], "m")     # two full blocks cached
    cached = kv.seq_pages[0][:2]
    kv.free_sequence(0)
    assert not set(cached) & set(kv.free_pages)   # the reference would have freed them
    _check_invariants(kv)
    # a new request reuses the prefix
    pages, n = pc.lookup(tokens, "m")
    assert pages == cached and n == 8
    kv.new_sequence(1, "m", prefix_pages=pages, prefix_len=n)
    assert kv.seq_pages[1][:2] == cached and kv.seq_len[1] == 8
    # evicting while sequence 1 still lists the pages does not free them
    pc.evict_lru(2)
    assert not set(cached) & set(kv.free_pages)
    kv.free_sequence(1)
    assert set(cached) <= set(kv.free_pages)
    _check_invariants(kv)
    assert copies == []


def test_fork_and_copy_on_write(copies):
    kv = _kv(pages=16, P=16)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 21)
    kv.seq_len[0] = 21
    for sid in (1, 2):
        kv.fork_sequence(0, sid)
    shared = list(kv.seq_pages[0])
    assert kv._holders[shared[1]] == 3 and kv.is_shared(shared[1])
    before = [bf16_bits(kv.k_pool[l]) for l in range(2)]
    n = kv.prepare_append([1, 2], 4)
    assert n == 2 and len(copies) == 1            # one launch for the whole batch
    src, dst, fill = copies[0]
    assert src == [shared[1], shared[1]] and fill == [5, 5]
    assert dst == [kv.seq_pages[1][1], kv.seq_pages[2][1]]
    assert kv.seq_pages[1][0] == shared[0]        # the full page is not written, stays shared
    for l in range(2):
        exp = page_ops.copy_pages([before[l]], [before[l]], src, dst, fill)[0]
        assert np.array_equal(bf16_bits(kv.k_pool[l]), exp)
    # parent is now the only holder of page 1: it writes in place
    assert kv.prepare_append([0], 3) == 0 and kv.seq_pages[0] == shared
    _check_invariants(kv)


def test_write_that_starts_on_a_page_boundary_copies_nothing(copies):
    kv = _kv(pages=8, P=16)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 32)
    kv.seq_len[0] = 32
    kv.fork_sequence(0, 1)
    kv._ensure_capacity(1, 33)                     # new page, no shared page written
    assert copies == [] and kv.seq_pages[1][:2] == kv.seq_pages[0][:2]
    _check_invariants(kv)


def test_fork_into_itself_changes_nothing(copies):
    kv = _kv(pages=8, P=4)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 6)
    kv.seq_len[0] = 6
    pages, holders = list(kv.seq_pages[0]), dict(kv._holders)
    kv.fork_sequence(0, 0)
    assert kv.seq_pages[0] == pages and kv._holders == holders and kv.seq_len[0] == 6
    assert copies == []
    _check_invariants(kv)


def test_migrate_and_compact_bookkeeping(copies):
    kv = _kv(pages=12, P=4)
    pc = PrefixCache(kv, page_size=4)
    for sid in range(4):
        kv.new_sequence(sid, owner=f"m{sid % 2}")
        kv._ensure_capacity(sid, 3 + 4 * sid)
        kv.seq_len[sid] = 3 + 4 * sid
    pc.store(list(range(8)), kv.seq_pages[3][:2], "m1")
    kv.fork_sequence(2, 9)
    kv.free_sequence(1)
    live = kv.live_pages()
    owners = {s: list(p) for s, p in kv.seq_pages.items()}
    holders = dict(kv._holders)
    data = {p: kv.k_pool[:, p].clone() for p in live}
    remap = kv.compact()
    assert sorted(remap.values()) == list(range(len(live)))
    assert copies[-1][0] == live and copies[-1][1] == [remap[p] for p in live]
    for sid, pages in owners.items():
        assert kv.seq_pages[sid] == [remap[p] for p in pages]
    assert kv._holders == {remap[p]: n for p, n in holders.items()}
    for p in live:
        assert torch.equal(kv.k_pool[:, remap[p]], data[p])
    assert pc.lookup(list(range(8)), "m1") == ([remap[p] for p in owners[3][:2]], 8)
    assert kv.pages_used == len(live)
    _check_invariants(kv)


_ops = st.lists(st.tuples(st.sampled_from(["new", "fork", "grow", "free", "store", "evict", "lookup_new"]),
                          st.integers(0, 7), st.integers(0, 40)), max_size=60)


@settings(max_examples=60, deadline=None)
@given(_ops)
def test_random_operations_keep_pages_accounted(ops):
    import prism_amd.kv_cache as m

    saved = m.copy_pages
    m.copy_pages = lambda src, dst, s, d, f: None     # bookkeeping only
    try:
        kv = FlashAttnKVCache(1, 1, 8, 24, 4, "cpu")
        pc = PrefixCache(kv, page_size=4)
        for op, a, n in ops:
            live = sorted(kv.seq_pages)
            try:
                if op == "new":
                    kv.new_sequence(a, "m")
                elif op == "fork" and live:
                    kv.fork_sequence(live[a % len(live)], a + 100)
                elif op == "grow" and live:
                    sid = live[a % len(live)]
                    kv.prepare_append([sid], n % 9)
                    kv.seq_len[sid] += n % 9
                elif op == "free" and live:
                    kv.free_sequence(live[a % len(live)])
                elif op == "store" and live:
                    sid = live[a % len(live)]
                    toks = [sid] * kv.seq_len[sid]
                    pc.store(toks, kv.seq_pages[sid], "m")
                elif op == "evict":
                    pc.evict_lru(a % 3)
                elif op == "lookup_new" and live:
                    sid = live[a % len(live)]
                    pages, got = pc.lookup([sid] * kv.seq_len[sid], "m")
                    if pages:
                        kv.new_sequence(a + 200, "m", prefix_pages=pages, prefix_len=got)
            except KVCacheOutOfPages:
                pass
            _check_invariants(kv)
    finally:
        m.copy_pages = saved


def test_unassigned_block_table_columns_never_name_a_live_page():
    # A mixed batch where one sequence sits exactly on a page boundary.  The reference executor
    # advances seq_len before building the table and grows capacity one token short
    # (engine/executor.py:205-208, kv_cache.py:116-121), so its next append lands in the column
    # after the sequence's last page.  That column must not hold a page anyone owns (the
    # reference's zero would be page 0, the first page its allocator hands out, kv_cache.py:49).
    from oracle.paged_attention import slot_mapping

    kv = _kv(pages=16, P=16)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 50)
    kv.seq_len[0] = 49
    kv.new_sequence(1)
    kv.seq_len[1] = 16                        # exactly one full page, no room for token 16
    bt, sl = kv.build_block_table([0, 1])
    bt = bt.numpy()
    assert bt[1].tolist() == [kv.seq_pages[1][0], -1, -1, -1]
    assert bt[0, :4].tolist() == kv.seq_pages[0]
    live = {p for pages in kv.seq_pages.values() for p in pages}
    slots = slot_mapping(bt, sl.numpy(), 1, 16)
    page_of = slots // 16
    assert page_of[0, 0] in kv.seq_pages[0]
    assert page_of[1, 0] < 0 and page_of[1, 0] not in live   # the kernels flag it and skip the write


def test_build_block_table_records_the_shared_prefix(copies):
    # branches of one prompt (forks of a 40-token sequence on 16-token pages): two full pages are
    # shared and filled by every branch; the third column is shared too but not full, and after
    # copy-on-write each branch holds its own copy of it
    from prism_amd import shared_prefix_of
    from prism_amd.kv_cache import shared_prefix_pages
    kv = _kv(pages=24, P=16)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 40)
    kv.seq_len[0] = 40
    for sid in (1, 2, 3):
        kv.fork_sequence(0, sid)
    bt, sl = kv.build_block_table([0, 1, 2, 3])
    assert shared_prefix_of(bt, sl) == 32
    # without an append, causal query row 0 sees keys t <= 40 - s_q: the prefix is cut to the
    # whole pages below that (39 keys -> 2 pages, 31 -> 1, 11 -> none); an append or a
    # non-causal call keeps it
    assert shared_prefix_of(bt, sl, s_q=2, causal=True, appends=False, page_size=16) == 32
    assert shared_prefix_of(bt, sl, s_q=10, causal=True, appends=False, page_size=16) == 16
    assert shared_prefix_of(bt, sl, s_q=30, causal=True, appends=False, page_size=16) == 0
    assert shared_prefix_of(bt, sl, s_q=30, causal=False, appends=False, page_size=16) == 32
    assert shared_prefix_of(bt, sl, s_q=30, causal=True, appends=True, page_size=16) == 32
    kv.prepare_append([0, 1, 2, 3], 5)
    bt, sl = kv.build_block_table([0, 1, 2, 3])
    assert len(set(bt[:, 2].tolist())) == 4 and shared_prefix_of(bt, sl) == 32
    # stale or foreign tensors record nothing
    assert shared_prefix_of(bt.clone(), sl) == 0
    assert shared_prefix_of(bt, sl.clone()) == 0
    bt2, sl2 = kv.build_block_table([0, 1, 2, 3])   # rebuilt into the same buffers: bt is stale
    assert shared_prefix_of(bt, sl) == 0 and shared_prefix_of(bt2, sl2) == 32
    bt2[1, 0] = bt2[1, 0]                              # any in-place write drops it
    assert shared_prefix_of(bt2, sl2) == 0
    # one sequence, or a batch that shares nothing, has no shared prefix
    bt, sl = kv.build_block_table([0])
    assert shared_prefix_of(bt, sl) == 0
    kv.new_sequence(9)
    kv._ensure_capacity(9, 40)
    kv.seq_len[9] = 40
    bt, sl = kv.build_block_table([0, 9])
    assert shared_prefix_of(bt, sl) == 0
    # the count itself: identical leading columns, capped by the shortest sequence's full pages
    t = np.array([[3, 4, 5, 6], [3, 4, 5, 7], [3, 4, 5, -1]], dtype=np.int32)
    assert shared_prefix_pages(t, np.array([64, 64, 48]), 16) == 3
    assert shared_prefix_pages(t, np.array([64, 64, 47]), 16) == 2
    assert shared_prefix_pages(t[:1], np.array([64]), 16) == 0
    assert shared_prefix_pages(np.full((2, 3), -1, dtype=np.int32), np.array([0, 0]), 16) == 0
    _check_invariants(kv)


def test_status_error_names_every_bit():
    # the exception a status poll raises carries the bits and the device, and names each flag
    from prism_amd import PrismKVStatusError
    from prism_amd import _lib
    bits = _lib.PKV_STATUS_BAD_PAGE | _lib.PKV_STATUS_MERGE_TIMEOUT
    e = PrismKVStatusError(bits, 3)
    assert e.bits == bits and e.device == 3 and isinstance(e, RuntimeError)
    assert "BAD_PAGE" in str(e) and "MERGE_TIMEOUT" in str(e) and "cuda:3" in str(e)
    assert "PARTIAL_RANGE" not in str(e)
