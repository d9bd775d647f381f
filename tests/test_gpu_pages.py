"""GPU parity of page movement: batched copy, copy-on-write, transfer_sequence, compaction.

All bit-exact against the oracle's page-op restatements (oracle/page_ops.py), comparing whole
pools so that untouched pages are checked too.
"""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import page_ops
from oracle import paged_attention as pa
from prism_amd import FlashAttnKVCache, PrefixCache

pytestmark = pytest.mark.gpu


def _pools(kv):
    return [pa.bf16_bits(t) for t in kv.k_caches] + [pa.bf16_bits(t) for t in kv.v_caches]


def _random_kv(gpu, layers=3, pages=20, P=16, n_kv=2, hd=64, seed=0):
    kv = FlashAttnKVCache(layers, n_kv, hd, pages, P, str(gpu), torch.bfloat16)
    g = torch.Generator(device=gpu).manual_seed(seed)
    kv.k_pool.normal_(generator=g)
    kv.v_pool.normal_(generator=g)
    return kv


def test_copy_pages_full_and_partial(gpu):
    kv = _random_kv(gpu)
    before = _pools(kv)
    src, dst, fill = [3, 7, 11], [0, 19, 5], [16, 5, 1]
    prism_amd.copy_pages(kv, kv, src, dst, fill)
    torch.cuda.synchronize()
    expect = page_ops.copy_pages(before, before, src, dst, fill)
    for got, exp in zip(_pools(kv), expect):
        assert np.array_equal(got, exp)


def test_transfer_sequence_matches_reference_semantics(gpu):
    a = _random_kv(gpu, seed=1)
    b = _random_kv(gpu, seed=2)
    a.new_sequence(7)
    a._ensure_capacity(7, 40)
    a.seq_len[7] = 40
    src_pages = list(a.seq_pages[7])
    before_a, before_b = _pools(a), _pools(b)
    n = a.transfer_sequence(7, b, 9)
    torch.cuda.synchronize()
    assert n == 3 and b.seq_len[9] == 40
    expect = page_ops.transfer_sequence(before_a, before_b, src_pages, b.seq_pages[9], 40, 16)
    for got, exp in zip(_pools(b), expect):
        assert np.array_equal(got, exp)


def test_copy_on_write_of_shared_partial_page(gpu):
    kv = _random_kv(gpu, layers=2, pages=16, P=16)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 21)
    kv.seq_len[0] = 21                      # page 1 of seq 0 holds 5 rows
    for sid in (1, 2, 3):
        kv.fork_sequence(0, sid)
    shared = list(kv.seq_pages[0])
    before = _pools(kv)
    n = kv.prepare_append([1, 2, 3], 4)     # each child writes rows 21..24 into the shared page
    torch.cuda.synchronize()
    assert n == 3                            # parent still holds the page, so every child copies
    for sid in (1, 2, 3):
        assert kv.seq_pages[sid][0] == shared[0]          # full page 0 still shared (not written)
        assert kv.seq_pages[sid][1] != shared[1]
    new_pages = [kv.seq_pages[s][1] for s in (1, 2, 3)]
    expect = page_ops.copy_pages(before, before, [shared[1]] * 3, new_pages, [5, 5, 5])
    for got, exp in zip(_pools(kv), expect):
        assert np.array_equal(got, exp)
    # the parent is now the sole holder: its own append writes in place
    assert kv.prepare_append([0], 3) == 0 and kv.seq_pages[0] == shared


def test_compaction_preserves_every_live_page(gpu):
    kv = _random_kv(gpu, layers=2, pages=24, P=16)
    pc = PrefixCache(kv, page_size=16)
    rng = np.random.default_rng(0)
    for sid in range(6):
        kv.new_sequence(sid, owner="m")
        kv._ensure_capacity(sid, int(rng.integers(1, 60)))
    tokens = list(range(40))
    kv.seq_len[0] = 40
    kv._ensure_capacity(0, 40)
    pc.store(tokens, kv.seq_pages[0], "m")
    for sid in (1, 3, 4):
        kv.free_sequence(sid)
    live = kv.live_pages()
    owners = {s: list(p) for s, p in kv.seq_pages.items()}
    before = _pools(kv)
    remap = kv.compact()
    torch.cuda.synchronize()
    assert sorted(remap.values()) == list(range(len(live)))
    expect, exp_remap = page_ops.compact(before, live, kv.max_pages)
    assert exp_remap == remap
    got = _pools(kv)
    for g_, e_ in zip(got, expect):
        assert np.array_equal(g_[: len(live)], e_[: len(live)])
    for sid, pages in owners.items():
        assert kv.seq_pages[sid] == [remap[p] for p in pages]
    assert pc.lookup(tokens, "m") == ([remap[p] for p in owners[0][:2]], 32)
    assert kv.pages_used == len(live)


@pytest.mark.parametrize("fill", [None, [16, 5, 1, 9]])
def test_staged_copy_matches_direct_copy(gpu, fill):
    # the disaggregated path (gather into staging, one device-to-device copy, scatter), forced on
    # one device, is bit-exact with the direct copy and the oracle
    a = _random_kv(gpu, seed=3)
    b = _random_kv(gpu, seed=4)
    before_a, before_b = _pools(a), _pools(b)
    src, dst = [3, 7, 11, 19], [0, 19, 5, 12]
    prism_amd.copy_pages(a, b, src, dst, fill, staged=True)
    torch.cuda.synchronize()
    expect = page_ops.copy_pages(before_a, before_b, src, dst, fill)
    for got, exp in zip(_pools(b), expect):
        assert np.array_equal(got, exp)
    for got, exp in zip(_pools(a), before_a):
        assert np.array_equal(got, exp)


def test_staged_transfer_sequence(gpu):
    a = _random_kv(gpu, seed=5)
    b = _random_kv(gpu, seed=6)
    a.new_sequence(7)
    a._ensure_capacity(7, 40)
    a.seq_len[7] = 40
    src_pages = list(a.seq_pages[7])
    before_a, before_b = _pools(a), _pools(b)
    n = a.transfer_sequence(7, b, 9, staged=True)
    torch.cuda.synchronize()
    assert n == 3 and b.seq_len[9] == 40
    expect = page_ops.transfer_sequence(before_a, before_b, src_pages, b.seq_pages[9], 40, 16)
    for got, exp in zip(_pools(b), expect):
        assert np.array_equal(got, exp)
