"""GPU tests of DecodeBatch, the device-resident decode block table (pkv_table_update), through
the C ABI: the device rows follow the allocator exactly (growth at page boundaries,
copy-on-write, batch churn, padding), bad packet entries are flagged and skipped, and a decode
step captured once in a HIP graph and replayed over several steps, fed only by DecodeBatch,
gives bit-identical outputs and caches to the same steps run eagerly on host-built tables."""
import random

import numpy as np
import pytest
import torch

import prism_amd
from oracle import epilogue as ep
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close

pytestmark = pytest.mark.gpu


def _check_device_rows(db, kv, seq_ids, gb):
    bt = db.block_table.cpu().numpy()
    sl = db.cache_seqlens.cpu().numpy()
    for i, sid in enumerate(seq_ids):
        pages = kv.seq_pages[sid]
        assert list(bt[i, :len(pages)]) == pages, f"row {i} (sequence {sid})"
        assert sl[i] == kv.seq_len[sid], f"row {i} length"
    for i in range(len(seq_ids), gb):
        assert bt[i, 0] == db.null_page and sl[i] == 0, f"padded row {i}"


def test_device_rows_follow_the_allocator(gpu):
    rng = random.Random(11)
    kv = prism_amd.FlashAttnKVCache(2, 2, 64, 400, 16, str(gpu))
    db = prism_amd.DecodeBatch(kv, max_batch=16)
    live: list[int] = []
    next_id = 0
    for step in range(120):
        if live and rng.random() < 0.1:
            kv.free_sequence(live.pop(rng.randrange(len(live))))
        if live and len(live) < 16 and rng.random() < 0.1 and kv.pages_free > 40:
            # a fork shares every page; the next write into the shared last page copies it
            src = rng.choice(live)
            kv.fork_sequence(src, next_id)
            live.append(next_id)
            next_id += 1
        while len(live) < rng.randint(2, 12) and kv.pages_free > 40:
            kv.new_sequence(next_id)
            kv.seq_len[next_id] = 0
            kv._ensure_capacity(next_id, rng.randint(1, 300))
            kv.seq_len[next_id] = len(kv.seq_pages[next_id]) * 16 - rng.randint(1, 16)
            live.append(next_id)
            next_id += 1
        if rng.random() < 0.05:
            rng.shuffle(live)
        gb = rng.randint(len(live), 16)
        n_new = rng.choice([1, 1, 1, 3])
        print(f"step {step}: {len(live)} sequences in {gb} rows, +{n_new}", flush=True)
        db.step(list(live), n_new, graph_batch=gb)
        torch.cuda.synchronize()
        _check_device_rows(db, kv, live, gb)
        db.advance()
    assert prism_amd.read_status(gpu) == 0


def test_table_update_flags_bad_entries(gpu):
    kv = prism_amd.FlashAttnKVCache(1, 2, 64, 20, 16, str(gpu))
    db = prism_amd.DecodeBatch(kv, max_batch=4, max_blocks=8)
    before = db.block_table.clone()
    packet = np.array([1, 7, 9, 3,                  # lengths: row 1 -> 7, row 9 (out of range)
                       0, 2, 5, 2, 8, 5, 3, 0, 20,  # entries: good, column 8 (out), page 20 (out)
                       3, 1, 19], dtype=np.int32)   # good
    db.apply(packet, 2, 4)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 1
    want = before.clone()
    want[0, 2] = 5
    want[3, 1] = 19
    assert torch.equal(db.block_table, want)
    assert db.cache_seqlens.tolist() == [0, 7, 0, 0]


def _twin_caches(gpu, num_pages, page_size, n_kv, hd, seed):
    a = prism_amd.FlashAttnKVCache(1, n_kv, hd, num_pages, page_size, str(gpu))
    b = prism_amd.FlashAttnKVCache(1, n_kv, hd, num_pages, page_size, str(gpu))
    g = torch.Generator(device="cpu").manual_seed(seed)
    init = torch.randn(a.k_pool.shape, generator=g).to(torch.bfloat16)
    a.k_pool.copy_(init)
    b.k_pool.copy_(init)
    init = torch.randn(a.v_pool.shape, generator=g).to(torch.bfloat16)
    a.v_pool.copy_(init)
    b.v_pool.copy_(init)
    return a, b


def test_captured_decode_step_matches_eager_host_tables(gpu):
    # Qwen2.5-7B attention shape (the balanced decode kernel), 32-token pages so a few steps
    # cross page boundaries; 5 sequences in an 8-row graph (3 padded rows)
    nh, nkv, hd, P, B, GB = 28, 4, 128, 32, 5, 8
    kvA, kvB = _twin_caches(gpu, 96, P, nkv, hd, seed=5)
    nullB = kvB.reserve_null_page()
    db = prism_amd.DecodeBatch(kvA, max_batch=GB)
    assert db.null_page == nullB
    lens = [29, 62, 95, 1, 200]
    for kv in (kvA, kvB):
        for s, L in enumerate(lens):
            kv.new_sequence(s)
            kv.seq_len[s] = 0
            kv._ensure_capacity(s, L)
            kv.seq_len[s] = L
        kv.fork_sequence(2, 7)  # sequence 7 shares 2's pages: its first write copies the last one
    seq_ids = [0, 1, 7, 3, 4]
    cos, sin = ep.rope_tables(hd, 512)
    cos, sin = cos.to(gpu), sin.to(gpu)
    width = (nh + 2 * nkv) * hd
    qkv = torch.zeros(GB, 1, width, dtype=torch.bfloat16, device=gpu)
    q_out = torch.empty(GB, 1, nh, hd, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(GB, 1, nh, hd, dtype=torch.bfloat16, device=gpu)
    sl_after = torch.empty(GB, dtype=torch.int32, device=gpu)

    bt, sl = db.step(seq_ids, 1, graph_batch=GB)

    def graph_step():
        prism_amd.rope_qk(qkv, sl, cos, sin, nh, nkv, return_k=False, q_out=q_out,
                          k_cache=kvA.k_caches[0], v_cache=kvA.v_caches[0], block_table=bt, cache_seqlens=sl)
        torch.add(sl, 1, out=sl_after)
        prism_amd.flash_attn_with_kvcache(q_out, kvA.k_caches[0], kvA.v_caches[0], cache_seqlens=sl_after,
                                          block_table=bt, causal=True, out=out)

    # eager warm-up on the capture stream sizes the split-K workspace, then capture; the
    # warm-up wrote the step-0 rows, which the first replay rewrites identically
    cap = torch.cuda.Stream(device=gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        graph_step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            graph_step()
    torch.cuda.current_stream(gpu).wait_stream(cap)
    torch.cuda.synchronize()

    gen = torch.Generator(device="cpu").manual_seed(9)
    for step in range(6):
        print(f"graph step {step}: lengths {[kvA.seq_len[s] for s in seq_ids]}", flush=True)
        x = torch.randn(GB, 1, width, generator=gen).to(torch.bfloat16).to(gpu)
        if step > 0:
            db.step(seq_ids, 1, graph_batch=GB)
        qkv.copy_(x)
        graph.replay()
        # the same step eagerly on host-built tables of the twin cache, padded the same way
        kvB.prepare_append(seq_ids, 1)
        bt_h, sl_h = kvB.block_table_host(seq_ids)
        btB = torch.full((GB, bt_h.shape[1]), nullB, dtype=torch.int32)
        btB[:B] = torch.from_numpy(bt_h)
        slB = torch.zeros(GB, dtype=torch.int32)
        slB[:B] = torch.from_numpy(sl_h)
        btB, slB = btB.to(gpu), slB.to(gpu)
        qB, _ = prism_amd.rope_qk(x, slB, cos, sin, nh, nkv, return_k=False, k_cache=kvB.k_caches[0],
                                  v_cache=kvB.v_caches[0], block_table=btB, cache_seqlens=slB)
        outB = prism_amd.flash_attn_with_kvcache(qB, kvB.k_caches[0], kvB.v_caches[0], cache_seqlens=slB + 1,
                                                 block_table=btB, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(out[:B], outB[:B]), f"step {step}: graph output differs from the eager one"
        db.advance()
        kvB.update_seqlens(seq_ids, 1)
    # every page but the null one is identical: padded rows never wrote into a sequence's page (the
    # null page itself holds whichever padded row's dummy K/V landed last in each launch)
    real = [p for p in range(kvA.max_pages) if p != nullB]
    assert torch.equal(kvA.k_pool[:, real], kvB.k_pool[:, real]), "K caches differ"
    assert torch.equal(kvA.v_pool[:, real], kvB.v_pool[:, real]), "V caches differ"
    assert kvA.seq_pages == kvB.seq_pages
    # the last step's output against the fp64 oracle over the cache
    ref = pa.attention_fp64(pa.bf16_bits(q_out[:B]), pa.bf16_bits(kvA.k_caches[0]), pa.bf16_bits(kvA.v_caches[0]),
                            db.block_table[:B].cpu().numpy(), db.cache_seqlens[:B].cpu().numpy() + 1, causal=True)
    assert_attn_close(out[:B], ref, "captured decode step")
