"""GPU parity of cascade (shared-prefix) attention, pkv_cascade_attn through the C ABI: batches
whose sequences list the same pages for a shared prefix, each with its own suffix and new rows,
against the fp64 oracle (which knows nothing of the sharing) and against the ordinary decode path,
plus the input checks (a sequence not sharing the prefix, or shorter than it, is flagged)."""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close

pytestmark = pytest.mark.gpu


def _shared_case(gpu, *, suffix, shared_pages, page_size, s_q, n_heads=28, n_kv=4, hd=128, seed=0,
                 break_row=None):
    """Pool + block tables: every sequence's first `shared_pages` columns are the same pages;
    sequence b holds shared_pages * P + suffix[b] keys before the append."""
    g = torch.Generator().manual_seed(seed)
    B = len(suffix)
    shared = shared_pages * page_size
    ctx = np.array([shared + s for s in suffix], dtype=np.int64)
    own = [int(np.ceil((c + s_q) / page_size)) - shared_pages for c in ctx]
    num_pages = shared_pages + sum(own) + 4
    perm = torch.randperm(num_pages, generator=g).to(torch.int32)
    width = shared_pages + max(own)
    bt = torch.zeros(B, width, dtype=torch.int32)
    off = shared_pages
    for b in range(B):
        bt[b, :shared_pages] = perm[:shared_pages]
        bt[b, shared_pages:shared_pages + own[b]] = perm[off:off + own[b]]
        off += own[b]
    if break_row is not None:
        bt[break_row, 0] = perm[-1]  # a page outside the shared set (still inside the pool)
    kc = torch.randn(num_pages, page_size, n_kv, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(num_pages, page_size, n_kv, hd, generator=g).to(torch.bfloat16)
    q = torch.randn(B, s_q, n_heads, hd, generator=g).to(torch.bfloat16)
    k = torch.randn(B, s_q, n_kv, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(B, s_q, n_kv, hd, generator=g).to(torch.bfloat16)
    sl = torch.tensor(ctx, dtype=torch.int32)
    cpu = dict(q=q, k=k, v=v, k_cache=kc, v_cache=vc, block_table=bt, cache_seqlens=sl)
    return cpu, {n: t.to(gpu) for n, t in cpu.items()}, shared


CASES = [
    # (suffix lengths, shared pages, page size, s_q)
    ([(i * 97) % 300 for i in range(64)], 2, 256, 5),   # config-5 shape, smaller: R = 35
    ([0, 31, 200], 3, 32, 1),                            # a suffix of zero keys; R = 7
    ([(i * 53) % 170 for i in range(40)], 2, 64, 2),     # R = 14, suffixes at tile / page edges
    ([5, 0, 700, 33, 64, 1, 250, 96], 1, 256, 8),       # R = 56: four row tiles per wave
    ([3000, 17], 4, 256, 5),                             # one long suffix: many ranges per sequence
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_cascade_matches_oracle_and_plain_decode(gpu, case):
    suffix, shared_pages, P, s_q = case
    print(f"cascade case B={len(suffix)} shared={shared_pages}x{P} s_q={s_q}", flush=True)
    cpu, dev, shared = _shared_case(gpu, suffix=suffix, shared_pages=shared_pages, page_size=P, s_q=s_q)
    kc0, vc0 = dev["k_cache"].clone(), dev["v_cache"].clone()
    out = torch.full_like(dev["q"], float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                      cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                      causal=True, shared_prefix_tokens=shared, out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                                 cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                                 causal=True)
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"cascade {case}")
    # the ordinary path on the same inputs (a fresh copy of the caches) agrees to rounding
    plain = prism_amd.flash_attn_with_kvcache(dev["q"], kc0, vc0, dev["k"], dev["v"],
                                              cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                              causal=True)
    torch.cuda.synchronize()
    diff = (plain.float() - out.float()).abs()
    assert float(diff.max()) <= 1.6e-2, f"cascade vs plain decode: max diff {float(diff.max())}"
    assert prism_amd.read_status(gpu) == 0


def test_cascade_flags_a_sequence_outside_the_prefix(gpu):
    cpu, dev, shared = _shared_case(gpu, suffix=[10, 20, 30], shared_pages=2, page_size=32, s_q=5, break_row=1)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                      cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                      causal=True, shared_prefix_tokens=shared)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_SHARED_PREFIX
    # a sequence shorter than the declared prefix
    cpu, dev, shared = _shared_case(gpu, suffix=[10, 20, 30], shared_pages=2, page_size=32, s_q=5)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                      cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                      causal=True, shared_prefix_tokens=shared + 32)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_SHARED_PREFIX


def test_cascade_falls_back_off_page_boundaries(gpu):
    # a prefix that is not a whole number of pages runs the ordinary decode path
    cpu, dev, shared = _shared_case(gpu, suffix=[10, 300, 0], shared_pages=2, page_size=256, s_q=5)
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=True, shared_prefix_tokens=shared - 16)
    torch.cuda.synchronize()
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(out, ref, "cascade fallback")


def test_cascade_without_append_checks_row_visibility(gpu):
    # k = v = None, causal, s_q = 5: row 0 of a sequence with c keys sees keys [0, c - 5], so the
    # prefix pass (which gives every row all shared keys) is right only when c >= shared + 4
    cpu, dev, shared = _shared_case(gpu, suffix=[4, 40, 300], shared_pages=2, page_size=32, s_q=5)
    out = torch.full_like(dev["q"], float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], cache_seqlens=dev["cache_seqlens"],
                                      block_table=dev["block_table"], causal=True, shared_prefix_tokens=shared,
                                      out=out)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(out, ref, "cascade without append")
    # a suffix of 3 keys: row 0 would wrongly see the last prefix key, so the call is flagged
    cpu, dev, shared = _shared_case(gpu, suffix=[3, 40, 300], shared_pages=2, page_size=32, s_q=5)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], cache_seqlens=dev["cache_seqlens"],
                                      block_table=dev["block_table"], causal=True, shared_prefix_tokens=shared)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_SHARED_PREFIX


def test_cascade_chosen_from_the_block_table_of_forked_branches(gpu):
    # a verify batch of 8 branches forked from one 2400-token prompt, each grown by its own suffix
    # (the boundary page copied on write): build_block_table records the 9 shared full pages and
    # flash_attn_with_kvcache, called exactly as the reference calls it (no shared-prefix
    # argument), takes cascade attention; results match the oracle and the ordinary path
    from prism_amd import shared_prefix_of
    P, n_kv, hd, nh, s_q = 256, 4, 128, 28, 5
    kv = prism_amd.FlashAttnKVCache(1, n_kv, hd, 64, P, str(gpu))
    g = torch.Generator().manual_seed(7)
    kv.k_pool.copy_(torch.randn(kv.k_pool.shape, generator=g).to(torch.bfloat16))
    kv.v_pool.copy_(torch.randn(kv.v_pool.shape, generator=g).to(torch.bfloat16))
    kv.new_sequence(0)
    kv._ensure_capacity(0, 2400)
    kv.seq_len[0] = 2400
    ids = list(range(8))
    for sid in ids[1:]:
        kv.fork_sequence(0, sid)
    for sid in ids:
        grow = (sid * 37) % 300
        kv.prepare_append([sid], grow)
        kv.update_seqlens([sid], grow)
    kv.prepare_append(ids, s_q)
    bt, sl = kv.build_block_table(ids)
    assert shared_prefix_of(bt, sl) == 9 * P
    assert 9 * P >= prism_amd.attention.AUTO_CASCADE_MIN_TOKENS
    q = torch.randn(len(ids), s_q, nh, hd, generator=g).to(torch.bfloat16)
    k = torch.randn(len(ids), s_q, n_kv, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(len(ids), s_q, n_kv, hd, generator=g).to(torch.bfloat16)
    kc_cpu, vc_cpu = kv.k_caches[0].cpu(), kv.v_caches[0].cpu()
    kc0, vc0 = kv.k_caches[0].clone(), kv.v_caches[0].clone()
    print(f"auto cascade B={len(ids)} shared={9 * P} s_q={s_q}", flush=True)
    out = prism_amd.flash_attn_with_kvcache(q.to(gpu), kv.k_caches[0], kv.v_caches[0], k.to(gpu), v.to(gpu),
                                            cache_seqlens=sl, block_table=bt, causal=True)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(q, kc_cpu, vc_cpu, k, v, cache_seqlens=sl.cpu(),
                                                 block_table=bt.cpu(), causal=True)
    assert np.array_equal(pa.bf16_bits(kv.k_caches[0]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(kv.v_caches[0]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, "auto cascade")
    plain = prism_amd.flash_attn_with_kvcache(q.to(gpu), kc0, vc0, k.to(gpu), v.to(gpu), cache_seqlens=sl,
                                              block_table=bt, causal=True, shared_prefix_tokens=0)
    torch.cuda.synchronize()
    assert float((plain.float() - out.float()).abs().max()) <= 1.6e-2
