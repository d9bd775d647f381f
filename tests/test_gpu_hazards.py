"""GPU tests of the hazards that used to be silent, each now turned into a status bit or a working
path (through the C ABI via the drop-ins):

* a write through a block-table column the sequence was never given (the reference executor's
  decode capacity is one token short, engine/executor.py:206 with engine/kv_cache.py:144-150):
  build_block_table marks such columns -1, so the append is skipped and PKV_STATUS_BAD_PAGE is set
  instead of the row landing in page 0, a page another sequence owns;
* a balanced-kernel split-K partial beyond fp16's range (|V| >= 65520): PKV_STATUS_PARTIAL_RANGE,
  and the per-head kernel (fp32 partials) gives the right answer;
* Prism's capture pattern: eager warm-up on the current stream, then HIP graph capture on a new
  stream (engine/executor.py:186-197, :288-303), replays equal to eager calls.
"""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close, make_paged_case

pytestmark = pytest.mark.gpu


def test_short_capacity_write_is_flagged_not_landed_in_page_zero(gpu):
    # two sequences: seq 0 long (3 pages), seq 1 at exactly one full page (256 tokens, 1 page).
    # The reference executor appends seq 1's next token at slot 256 (column 1) without growing it
    # first; column 1 of its row must not name a page anyone owns.
    kv = prism_amd.FlashAttnKVCache(1, 4, 128, 8, 256, str(gpu))
    g = torch.Generator(device=gpu).manual_seed(3)
    kv.k_pool.normal_(generator=g)
    kv.v_pool.normal_(generator=g)
    kv.new_sequence(0)
    kv._ensure_capacity(0, 600)
    kv.seq_len[0] = 599
    kv.new_sequence(1)
    kv.seq_len[1] = 256
    bt, sl = kv.build_block_table([0, 1])
    assert bt.cpu()[1, 1:].tolist() == [-1, -1]
    before_k, before_v = kv.k_pool.clone(), kv.v_pool.clone()
    q = torch.randn(2, 1, 28, 128, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(2, 1, 4, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(2, 1, 4, 128, generator=g, device=gpu).to(torch.bfloat16)
    prism_amd.flash_attn_with_kvcache(q, kv.k_caches[0], kv.v_caches[0], k=k, v=v, cache_seqlens=sl,
                                      block_table=bt, causal=True)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_BAD_PAGE
    # only seq 0's own append landed: one row of its third page
    changed = ((kv.k_pool != before_k) | (kv.v_pool != before_v)).flatten(3).any(3).nonzero().tolist()
    p0 = kv.seq_pages[0][2]
    assert changed and all(c[1] == p0 and c[2] == 599 - 512 for c in changed), changed


def test_fp16_partial_overflow_is_flagged(gpu):
    # V rows of magnitude ~1e6 (bf16 holds them; fp16 partials cannot) on the balanced kernel
    cpu, dev = make_paged_case(gpu, batch=3, ctx=[3000, 17, 4100], page_size=256, n_kv=4, n_heads=28,
                               head_dim=128, s_q=1, seed=7)
    big = (dev["v_cache"].float() * 1e6).to(torch.bfloat16)
    dev["v_cache"].copy_(big)
    cpu["v_cache"] = big.cpu()
    kw = dict(cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"], causal=True)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_PARTIAL_RANGE
    # fp32 partials: correct, within the tolerance scaled by the magnitude
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], kernel="heads", **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(out.float() / 1e6, ref / 1e6, "fp32 partials at |V| ~ 1e6")
    # ordinary magnitudes never set the bit
    small = (dev["v_cache"].float() / 1e6).to(torch.bfloat16)
    dev["v_cache"].copy_(small)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0


@pytest.mark.parametrize("s_q", [1, 5])
def test_capture_on_a_fresh_stream_after_eager_warmup(gpu, s_q):
    # engine/executor.py:186-197: warm up on the current stream, capture on a new stream, replay
    cpu, dev = make_paged_case(gpu, batch=32, ctx=[(i * 397) % 3000 + 1 for i in range(32)], page_size=256,
                               n_kv=4, n_heads=28, head_dim=128, s_q=s_q, seed=11)
    kw = dict(cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"], causal=True)
    eager = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"], **kw)
    torch.cuda.synchronize()
    out = torch.full_like(eager, float("nan"))
    cap = torch.cuda.Stream(device=gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                              out=out, **kw)
    torch.cuda.current_stream(gpu).wait_stream(cap)
    for rep in range(3):
        out.fill_(float("nan"))
        graph.replay()
        # eager work between replays on the same stream, sharing the workspace
        again = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"], **kw)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager call"
        assert torch.equal(again, eager)
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(out, ref, f"captured s_q={s_q}")


def test_status_bits_reach_the_host_at_build_block_table(gpu):
    # the short-capacity write of the test above, then the host points Prism passes every step:
    # the first build_block_table starts an asynchronous read of the status word, a later one
    # raises PrismKVStatusError with the bit (nothing on the host waited for the GPU)
    kv = prism_amd.FlashAttnKVCache(1, 4, 128, 8, 256, str(gpu))
    kv.new_sequence(0)
    kv._ensure_capacity(0, 300)
    kv.seq_len[0] = 299
    kv.new_sequence(1)
    kv.seq_len[1] = 256
    bt, sl = kv.build_block_table([0, 1])
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn(2, 1, 28, 128, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(2, 1, 4, 128, generator=g, device=gpu).to(torch.bfloat16)
    prism_amd.flash_attn_with_kvcache(q, kv.k_caches[0], kv.v_caches[0], k=k, v=k.clone(), cache_seqlens=sl,
                                      block_table=bt, causal=True)
    kv.build_block_table([0, 1])          # starts the read; nothing has landed yet
    torch.cuda.synchronize()
    with pytest.raises(prism_amd.PrismKVStatusError) as e:
        kv.build_block_table([0, 1])
    assert e.value.bits & prism_amd._lib.PKV_STATUS_BAD_PAGE and "BAD_PAGE" in str(e.value)
    # reported once: the word and the host copies are clear again
    torch.cuda.synchronize()
    kv.update_seqlens([0], 1)
    assert prism_amd.read_status(gpu) == 0


def test_stale_merge_counters_are_flagged_then_cleared(gpu):
    # a merge that timed out leaves its arrival counter armed; the next call's merge workgroups
    # must flag PKV_STATUS_MERGE_TIMEOUT instead of merging stale partials, and reading the bit
    # clears the workspace's counters so that the call after it is right again.  The leftover
    # state is planted from the host (every counter word set), so every kernel exits normally.
    from prism_amd import attention as attn
    cpu, dev = make_paged_case(gpu, batch=3, ctx=[3000, 17, 4100], page_size=256, n_kv=4, n_heads=28,
                               head_dim=128, s_q=1, seed=21)
    kw = dict(cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"], causal=True, two_pass=False,
              grid=8)
    good = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(good, ref, "in-launch merge, 8 workgroups")
    ws = attn._workspaces[(gpu.index or 0, torch.cuda.current_stream(gpu).cuda_stream)]
    ws[:65536].view(torch.int32).fill_(0x7FFF7FFF)
    out = torch.full_like(good, float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], out=out, **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_MERGE_TIMEOUT
    assert not torch.equal(out, good)      # the split sequences' rows were left unwritten
    torch.cuda.synchronize()
    assert int(ws[:65536].view(torch.int32).abs().sum()) == 0   # read_status cleared the counters
    again = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(again, good)
    assert prism_amd.read_status(gpu) == 0
    # the noalloc scratch is cleared by the flag its next call then carries
    attn._reset_counters.add(gpu.index or 0)
    na = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], noalloc=True, **kw)
    torch.cuda.synchronize()
    assert not attn._reset_counters and torch.equal(na, good)


def test_merge_timeout_marks_its_counter_until_the_counters_are_cleared(gpu):
    # every arrival counter planted at -1 from the host, so each count stops one short of its part
    # count: the merge workgroups wait out their bounded poll, flag PKV_STATUS_MERGE_TIMEOUT and
    # mark their counters (bit 30); the next call's merge workgroups find a count above the part
    # count and flag again without merging; reading the bit clears the counters, and the call
    # after that is right.  Every kernel exits normally (the wait is bounded).
    from prism_amd import attention as attn
    cpu, dev = make_paged_case(gpu, batch=3, ctx=[3000, 17, 4100], page_size=256, n_kv=4, n_heads=28,
                               head_dim=128, s_q=1, seed=22)
    kw = dict(cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"], causal=True, two_pass=False,
              grid=8)
    good = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(good, ref, "in-launch merge, 8 workgroups")
    ws = attn._workspaces[(gpu.index or 0, torch.cuda.current_stream(gpu).cuda_stream)]
    cnt = ws[:65536].view(torch.int32)
    cnt.fill_(-1)
    word = attn.status_tensor(gpu)
    out = torch.full_like(good, float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], out=out, **kw)
    torch.cuda.synchronize()
    assert int(word.item()) & prism_amd._lib.PKV_STATUS_MERGE_TIMEOUT
    marked = cnt.cpu()
    assert ((marked >= (1 << 30)) & (marked < (1 << 30) + 64)).any()   # a timed-out count, marked
    assert not torch.equal(out, good)      # the split sequences' rows were left unwritten
    word.zero_()
    out2 = torch.full_like(good, float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], out=out2, **kw)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) & prism_amd._lib.PKV_STATUS_MERGE_TIMEOUT   # the mark, seen
    assert not torch.equal(out2, good)
    torch.cuda.synchronize()
    assert int(cnt.abs().sum()) == 0      # read_status cleared the counters
    again = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(again, good)
    assert prism_amd.read_status(gpu) == 0


@pytest.mark.parametrize("prefix,s_q", [(2560, 5), (2048, 2)])
def test_no_append_causal_verify_cuts_the_automatic_cascade_prefix(gpu, prefix, s_q):
    # 8 branches of one prompt on full shared pages, called the way flash_attn allows without an
    # append: causal query row 0 sees keys t <= L - s_q only, so the automatic cascade may read
    # only the whole pages below that as a shared prefix (2560 keys, s_q 5: 2304, still a
    # cascade; 2048, s_q 2: 1792, below the automatic threshold: the ordinary path).  A prefix
    # that row 0 cannot see whole would flag PKV_STATUS_SHARED_PREFIX and give row 0 a key it
    # must not see.
    kv = prism_amd.FlashAttnKVCache(1, 4, 128, 24, 256, str(gpu))
    g = torch.Generator(device=gpu).manual_seed(prefix + s_q)
    kv.k_pool.normal_(generator=g)
    kv.v_pool.normal_(generator=g)
    kv.new_sequence(100)
    kv._ensure_capacity(100, prefix)
    kv.seq_len[100] = prefix
    ids = list(range(8))
    for sid in ids:
        kv.fork_sequence(100, sid)
    bt, sl = kv.build_block_table(ids)
    want = (prefix - s_q + 1) // 256 * 256
    assert prism_amd.shared_prefix_of(bt, sl, s_q=s_q, causal=True, appends=False, page_size=256) == want
    q = torch.randn(8, s_q, 28, 128, generator=g, device=gpu).to(torch.bfloat16)
    kc, vc = kv.k_caches[0].cpu(), kv.v_caches[0].cpu()
    out = prism_amd.flash_attn_with_kvcache(q, kv.k_caches[0], kv.v_caches[0], cache_seqlens=sl, block_table=bt,
                                            causal=True)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    ref, _, _ = pa.flash_attn_with_kvcache_ref(q.cpu(), kc, vc, cache_seqlens=sl.cpu(),
                                               block_table=bt.cpu().clamp(min=0), causal=True)
    assert_attn_close(out, ref, f"no-append causal verify, prefix {prefix}, s_q {s_q}")
