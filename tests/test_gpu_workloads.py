"""GPU parity at the five benchmark workloads themselves (prism_amd.workloads, seed 0, full size).

Every call goes through the drop-in (prism_amd.flash_attn_with_kvcache -> the C ABI) on the same
pools, block tables and lengths bench.py times, and is checked against the CPU oracle:

* attention output within the north_star bf16 tolerance of the fp64 oracle (max-abs <= 1e-2,
  mean-abs <= 1e-3, pkv_testutil);
* the appended rows bit-exact: every page a sequence references is compared with the oracle's
  append on a snapshot taken before the call, and every other page of the layer's pool (the
  2043-page, 535 MB per-layer tensors) must be unchanged, bit for bit;
* config 5's page operations bit-exact against oracle/page_ops.py: the copy-on-write of the shared
  boundary page into 63 children, the compaction of every live page into a fresh pool, and the
  staged (disaggregated) transfer of one sequence.

The oracle sees only the pages the batch references (gathered on the device, block tables remapped
onto them), so an fp64 check of a full-size layer takes about a second.  Config 4's prefill
oracle runs on two KV heads (10 query heads) at every row of one layer and on every head at a
sample of rows of another; its append check covers every head.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import prism_amd
from oracle import page_ops
from oracle import paged_attention as pa
from pkv_testutil import LayerCheck, free_cached as _free
from prism_amd import workloads

pytestmark = pytest.mark.gpu


def _call(w, l, out, **kw):
    kv = w.kv
    return prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                             cache_seqlens=w.cache_seqlens, block_table=w.block_table,
                                             causal=True, out=out, **kw)


def _decode_layers(w, layers, what, **kw):
    for l in layers:
        print(f"{what} layer {l}: B={w.batch} s_q={w.s_q} sum_ctx={int(w.ctx.sum())} max_ctx={int(w.ctx.max())}",
              flush=True)
        chk = LayerCheck(w, l)
        out = torch.full_like(w.q[l], float("nan"))
        _call(w, l, out, **kw)
        chk.check(out, f"{what} layer {l}")
        del chk
        _free()


@pytest.mark.parametrize("merge", [None, False])
def test_config3_headline_decode(gpu, merge):
    # the metric's workload: 28 layers, B = 32 lognormal contexts (seed 0: sum 55,816, max 5,882),
    # a 2043-page pool with 40% churn; the library's kernel choice, two-pass and in-launch merge
    w = workloads.config3(gpu, seed=0)
    assert w.layers == 28 and w.batch == 32 and w.kv.max_pages == 2043
    assert int(w.ctx.sum()) == 55816 and int(w.ctx.max()) == 5882
    _decode_layers(w, [0, 13, 27], f"config3 merge={merge}", two_pass=merge)
    del w
    _free()


def test_config3_graph_replay_matches_eager(gpu):
    # bench.py's timed step: the 28 calls captured once in a HIP graph; every replay's outputs are
    # bit-identical to the eager calls' and the first layer still matches the oracle
    w = workloads.config3(gpu, seed=0)
    L = w.layers
    eager = [torch.full_like(q, float("nan")) for q in w.q]
    chk = LayerCheck(w, 0)
    for l in range(L):
        _call(w, l, eager[l])
    chk.check(eager[0], "config3 eager layer 0")
    outs = [torch.full_like(q, float("nan")) for q in w.q]
    cap = torch.cuda.Stream(device=gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for l in range(L):
                _call(w, l, outs[l])
    torch.cuda.current_stream(gpu).wait_stream(cap)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for l in range(L):
            assert torch.equal(outs[l], eager[l]), f"replay {rep} layer {l} differs from eager"
    print("config3 graph: 3 replays of 28 layers bit-identical to eager", flush=True)
    del chk, graph, w
    _free()


def test_config2_decode(gpu):
    # B = 8 at context 2048 on the scattered 30 GB pool (the reference's bs = 8 decode graph)
    w = workloads.config2(gpu, seed=0)
    assert w.layers == 28 and w.batch == 8 and (w.ctx == 2048).all()
    _decode_layers(w, [0, 27], "config2")
    del w
    _free()


@pytest.mark.parametrize("shape", ["14B", "0.5B", "7B-tp4"])
def test_ragged_decode_other_shapes(gpu, shape):
    # config 3's ragged batch at the 14B (8 KV heads), 0.5B (2 KV heads, head_dim 64) and 7B
    # tensor-parallel-shard (1 KV head) shapes, first and last layer
    w = workloads.ragged_decode(shape, gpu, seed=0)
    assert int(w.ctx.sum()) == 55816
    _decode_layers(w, [0, w.layers - 1], f"decode-{shape}")
    del w
    _free()


def test_config4_chunked_prefill(gpu):
    # 14B: 8 chunks of 512 appended onto prefixes ~U{0..4096}, causal within the chunk; the fp64
    # oracle on KV heads 0 and 5 (query heads 0-4 and 25-29) of every sequence and row at layer 0,
    # and on all 40 query heads at a sample of 64 query rows (tile and chunk edges included) at
    # layer 47
    w = workloads.config4(gpu, seed=0)
    assert w.layers == 48 and w.s_q == 512 and w.batch == 8
    edges = [0, 1, 15, 16, 31, 32, 33, 127, 128, 255, 256, 257, 383, 384, 510, 511]
    draw = np.random.default_rng(4).choice(512, size=48, replace=False)
    rows47 = np.unique(np.concatenate([edges, draw]))
    for l, heads, rows in ((0, [0, 5], None), (47, None, rows47)):
        print(f"config4 layer {l}: prefixes {w.ctx.tolist()}", flush=True)
        chk = LayerCheck(w, l, kv_heads=heads)
        out = torch.full_like(w.q[l], float("nan"))
        _call(w, l, out)
        chk.check(out, f"config4 layer {l}", rows=rows)
        assert torch.isfinite(out.float()).all(), "config4: a query head outside the sample was not written"
        del chk
        _free()
    del w
    _free()


def _pool_pages(kv, layers, pages):
    """uint16 bits [2 * len(layers), n, P, n_kv, hd] of the given pages (K layers, then V layers)."""
    idx = torch.as_tensor(list(pages), dtype=torch.int64, device=kv.k_pool.device)
    return [pa.bf16_bits(kv.k_caches[l].index_select(0, idx)) for l in layers] + \
           [pa.bf16_bits(kv.v_caches[l].index_select(0, idx)) for l in layers]


def test_config5_prefix_cow_verify_compaction_transfer(gpu):
    # 64 sequences forked from one 2048 - r token prefix held in a PrefixCache; the first suffix
    # write copies the partially filled boundary page into 63 children (one launch, every layer)
    snap = {}

    def before_cow(kv):
        snap["k"] = kv.k_pool.clone()
        snap["v"] = kv.v_pool.clone()
        snap["free"] = list(kv.free_pages)

    pc = prism_amd.PrefixCache(None)
    w = workloads.config5(gpu, seed=0, prefix_cache=pc, before_cow=before_cow)
    kv = w.kv
    assert kv.prefix_cache is pc and pc.num_cached_pages == w.meta["shared_prefix"] // kv.page_size
    P = kv.page_size
    fill = w.meta["boundary_fill"]
    bidx = w.meta["shared_prefix"] // P
    root_boundary = w.meta["root_pages"][bidx]
    assert w.meta["cow_copies"] == 63 and 0 < fill < P
    torch.cuda.synchronize()

    # ---- copy-on-write: the oracle applied to the pre-COW pages of sampled layers, every layer by
    # a device comparison with the snapshot
    dst = [kv.seq_pages[s][bidx] for s in w.seq_ids if kv.seq_pages[s][bidx] != root_boundary]
    assert len(dst) == 63 and len(set(dst)) == 63
    involved = [root_boundary] + dst
    layers = [0, 27]
    before = [pa.bf16_bits(snap[t][l].index_select(0, torch.tensor(involved, device=gpu)))
              for t in ("k", "v") for l in layers]
    mini_dst = list(range(1, len(involved)))
    expect = page_ops.copy_pages(before, before, [0] * len(dst), mini_dst, [fill] * len(dst))
    got = [pa.bf16_bits(getattr(kv, f"{t}_caches")[l].index_select(0, torch.tensor(involved, device=gpu)))
           for t in ("k", "v") for l in layers]
    for g_, e_ in zip(got, expect):
        assert np.array_equal(g_, e_), "copy-on-write not bit-exact against oracle/page_ops"
    changed = set()
    for t in ("k", "v"):
        diff = (getattr(kv, f"{t}_pool") != snap[t]).flatten(2).any(2).any(0)
        changed |= set(torch.nonzero(diff).flatten().tolist())
    assert changed <= set(dst), "copy-on-write touched a page outside its destinations"
    print(f"config5 COW: 63 pages x {fill} slots x 56 tensors bit-exact; {len(changed)} pages changed", flush=True)
    snap.clear()
    _free()

    # ---- verify attention, ordinary and cascade paths, on the pages every child shares
    shared_tokens = bidx * P
    for l in (0, 27):
        for sp in (0, shared_tokens):
            chk = LayerCheck(w, l)
            out = torch.full_like(w.q[l], float("nan"))
            print(f"config5 verify layer {l} shared_prefix_tokens={sp}", flush=True)
            _call(w, l, out, shared_prefix_tokens=sp)
            chk.check(out, f"config5 verify layer {l} cascade={bool(sp)}")
            del chk
            _free()
    assert prism_amd.read_status(gpu) == 0

    # ---- staged (disaggregated) transfer of one child into another cache
    sid = w.seq_ids[-1]
    n = -(-kv.seq_len[sid] // P)
    src_pages = kv.seq_pages[sid][:n]
    target = prism_amd.FlashAttnKVCache(kv.num_layers, kv.num_kv_heads, kv.head_dim, n + 3, P, str(gpu))
    got_n = kv.transfer_sequence(sid, target, 5, staged=True)
    torch.cuda.synchronize()
    assert got_n == n and target.seq_len[5] == kv.seq_len[sid]
    src_bits = _pool_pages(kv, range(kv.num_layers), src_pages)
    dst_bits = [np.zeros((n + 3,) + b.shape[1:], dtype=np.uint16) for b in src_bits]
    expect = page_ops.transfer_sequence(src_bits, dst_bits, list(range(n)), target.seq_pages[5], kv.seq_len[sid], P)
    got = [pa.bf16_bits(t) for t in target.k_caches] + [pa.bf16_bits(t) for t in target.v_caches]
    for g_, e_ in zip(got, expect):
        assert np.array_equal(g_, e_), "staged transfer not bit-exact"
    print(f"config5 staged transfer: {n} pages x 56 tensors bit-exact", flush=True)
    del target
    _free()

    # ---- compaction of every live page (sequences + prefix-cache entries) into a fresh pool
    live = kv.live_pages()
    tables = {s: list(p) for s, p in kv.seq_pages.items()}
    lens = dict(kv.seq_len)
    k_old = kv.k_pool.index_select(1, torch.tensor(live, device=gpu))
    v_old = kv.v_pool.index_select(1, torch.tensor(live, device=gpu))
    old_bits = _pool_pages(kv, layers, live)
    remap = kv.compact()
    torch.cuda.synchronize()
    n_live = len(live)
    print(f"config5 compaction: {n_live} live pages", flush=True)
    assert sorted(remap.values()) == list(range(n_live))
    exp_pools, exp_remap = page_ops.compact(old_bits, list(range(n_live)), n_live)
    assert [exp_remap[i] for i in range(n_live)] == [remap[p] for p in live]
    new_bits = _pool_pages(kv, layers, [remap[p] for p in live])
    for g_, e_ in zip(new_bits, exp_pools):
        assert np.array_equal(g_, e_), "compaction not bit-exact against oracle/page_ops"
    assert torch.equal(kv.k_pool[:, :n_live], k_old) and torch.equal(kv.v_pool[:, :n_live], v_old)
    for s, pages in tables.items():
        assert kv.seq_pages[s] == [remap[p] for p in pages] and kv.seq_len[s] == lens[s]
    assert sorted(pc.entry_pages()) == sorted(remap[p] for p in w.meta["root_pages"][:bidx])
    del k_old, v_old
    # attention over the compacted pool still matches the oracle (tables rebuilt from the remap)
    bt, sl = kv.build_block_table(w.seq_ids)
    w.block_table, w.cache_seqlens = bt.clone(), sl.clone()
    chk = LayerCheck(w, 13)
    out = torch.full_like(w.q[13], float("nan"))
    _call(w, 13, out)
    chk.check(out, "config5 verify after compaction, layer 13")
    del chk, w
    _free()
