"""Seeded random sweep of the drop-in attention op against the fp64 oracle (through the C ABI).

Each case draws a batch, ragged context lengths (zeros included), a page size, a Qwen2.5 head
geometry (whole model or a tensor-parallel shard), s_q (decode and verify rows, or prefill
chunks of 16-512 tokens), causal or not, append or not, and a fragmented page pool; the library picks its kernel and merge as it would for Prism.  Checked:
outputs within the north_star bf16 tolerance of the fp64 oracle, and both caches bit-exact after
the append (whole pools compared).  The draws are fixed by the seed list, so a failure names a
reproducible case.
"""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close, make_paged_case

pytestmark = pytest.mark.gpu

# (n_heads, n_kv, head_dim): Qwen2.5 0.5B / 7B / 14B and their tensor-parallel shards
GEOMETRIES = [(14, 2, 64), (7, 1, 64), (28, 4, 128), (14, 2, 128), (7, 1, 128), (40, 8, 128), (20, 4, 128),
              (10, 2, 128)]
PAGE_SIZES = [16, 32, 64, 128, 256]
S_Q = [1, 1, 1, 2, 4, 5]


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    batch = int(rng.integers(1, 41))
    ctx = rng.integers(0, 3000, size=batch)
    ctx[rng.random(batch) < 0.1] = 0
    return dict(batch=batch, ctx=[int(c) for c in ctx], page_size=int(PAGE_SIZES[rng.integers(len(PAGE_SIZES))]),
                n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=int(S_Q[rng.integers(len(S_Q))]),
                causal=bool(rng.random() < 0.8), append=bool(rng.random() < 0.8), seed=seed)


@pytest.mark.parametrize("seed", range(48))
def test_random_case_matches_oracle(gpu, seed):
    c = draw(seed)
    print(f"random case {seed}: B={c['batch']} ctx[:6]={c['ctx'][:6]} P={c['page_size']} h={c['n_heads']} "
          f"kv={c['n_kv']} hd={c['head_dim']} s_q={c['s_q']} causal={c['causal']} append={c['append']}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=c["batch"], ctx=c["ctx"], page_size=c["page_size"], n_kv=c["n_kv"],
                               n_heads=c["n_heads"], head_dim=c["head_dim"], s_q=c["s_q"], seed=seed)
    k = dev["k"] if c["append"] else None
    v = dev["v"] if c["append"] else None
    out = torch.full_like(dev["q"], float("nan"))
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], k, v,
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=c["causal"], out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if c["append"] else None,
        cpu["v"] if c["append"] else None, cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
        causal=c["causal"])
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random case {seed}")


def draw_prefill(seed):
    rng = np.random.default_rng(5000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    batch = int(rng.integers(1, 7))
    ctx = rng.integers(0, 2500, size=batch)
    ctx[rng.random(batch) < 0.2] = 0
    s_q = int([16, 33, 64, 100, 128, 256, 512][rng.integers(7)])
    return dict(batch=batch, ctx=[int(c) for c in ctx], page_size=int(PAGE_SIZES[rng.integers(len(PAGE_SIZES))]),
                n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q, causal=bool(rng.random() < 0.85),
                append=bool(rng.random() < 0.85), seed=seed)


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill_chunk_matches_oracle(gpu, seed):
    """Chunks (s_q * n_heads / n_kv > 64) take the prefill kernels through the same drop-in call."""
    c = draw_prefill(seed)
    print(f"random prefill case {seed}: B={c['batch']} ctx={c['ctx']} P={c['page_size']} h={c['n_heads']} "
          f"kv={c['n_kv']} hd={c['head_dim']} s_q={c['s_q']} causal={c['causal']} append={c['append']}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=c["batch"], ctx=c["ctx"], page_size=c["page_size"], n_kv=c["n_kv"],
                               n_heads=c["n_heads"], head_dim=c["head_dim"], s_q=c["s_q"], seed=seed)
    k = dev["k"] if c["append"] else None
    v = dev["v"] if c["append"] else None
    out = torch.full_like(dev["q"], float("nan"))
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], k, v,
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=c["causal"], out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if c["append"] else None,
        cpu["v"] if c["append"] else None, cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
        causal=c["causal"])
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random prefill case {seed}")


def draw_cascade(seed):
    rng = np.random.default_rng(9000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    batch = int(rng.integers(2, 49))
    P = int([32, 64, 128, 256][rng.integers(4)])
    shared_pages = int(rng.integers(1, 5))
    suffix = rng.integers(0, 900, size=batch)
    suffix[rng.random(batch) < 0.15] = 0
    return dict(suffix=[int(x) for x in suffix], shared_pages=shared_pages, page_size=P,
                s_q=int([1, 2, 4, 5, 8][rng.integers(5)]), n_heads=nh, n_kv=n_kv, hd=hd, seed=seed,
                causal=bool(rng.random() < 0.75))


@pytest.mark.parametrize("seed", range(32))
def test_random_cascade_matches_oracle(gpu, seed):
    """Batches sharing a random number of prefix pages, declared through shared_prefix_tokens."""
    from test_gpu_cascade import _shared_case
    c = draw_cascade(seed)
    print(f"random cascade case {seed}: B={len(c['suffix'])} shared={c['shared_pages']}x{c['page_size']} "
          f"h={c['n_heads']} kv={c['n_kv']} hd={c['hd']} s_q={c['s_q']} causal={c['causal']}", flush=True)
    cpu, dev, shared = _shared_case(gpu, suffix=c["suffix"], shared_pages=c["shared_pages"], page_size=c["page_size"],
                                    s_q=c["s_q"], n_heads=c["n_heads"], n_kv=c["n_kv"], hd=c["hd"], seed=seed)
    out = torch.full_like(dev["q"], float("nan"))
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                      cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                      causal=c["causal"], shared_prefix_tokens=shared, out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                                 cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                                 causal=c["causal"])
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random cascade case {seed}")
    assert prism_amd.read_status(gpu) == 0


def draw_rope(seed):
    rng = np.random.default_rng(13000 + seed)
    # shapes the fused rotary launch takes: R + 2 s_q <= 16 rows per KV head, a page of a tile or more
    nh, n_kv, hd = [(28, 4, 128), (40, 8, 128), (14, 2, 128), (7, 1, 128), (14, 2, 64), (20, 4, 128)][rng.integers(6)]
    g = nh // n_kv
    s_q = 2 if g <= 5 and rng.random() < 0.4 else 1
    heads_per_tile = 4 if n_kv % 4 == 0 else (2 if n_kv % 2 == 0 else 1)
    tile = 32 * (4 // heads_per_tile) * (128 // hd)  # tokens per tile of the balanced kernel
    P = int(max(tile, [32, 64, 128, 256][rng.integers(4)]))
    batch = int(rng.integers(1, 49))
    ctx = rng.integers(0, 3000, size=batch)
    ctx[rng.random(batch) < 0.1] = 0
    return dict(batch=batch, ctx=[int(c) for c in ctx], page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                seed=seed)


@pytest.mark.parametrize("seed", range(16))
def test_random_rope_decode_matches_reference_step(gpu, seed):
    """The fused rotary + append + attention launch against the reference's bf16 rotary expression
    and the fp64 attention oracle."""
    from oracle import epilogue as ep
    c = draw_rope(seed)
    B, nh, nkv, hd, s = c["batch"], c["n_heads"], c["n_kv"], c["head_dim"], c["s_q"]
    print(f"random rope case {seed}: B={B} P={c['page_size']} h={nh} kv={nkv} hd={hd} s_q={s}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=B, ctx=c["ctx"], page_size=c["page_size"], n_kv=nkv, n_heads=nh,
                               head_dim=hd, s_q=s, seed=seed)
    g = torch.Generator().manual_seed(77 + seed)
    qkv = torch.randn((B, s, (nh + 2 * nkv) * hd), generator=g).to(torch.bfloat16)
    cos, sin = ep.rope_tables(hd, 4096)
    q_ref, k_ref, v_ref = ep.qkv_split_rope(qkv, np.array(c["ctx"], dtype=np.int32), cos, sin, nh, nkv)
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(q_ref, cpu["k_cache"], cpu["v_cache"], k_ref, v_ref,
                                                 cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                                 causal=True)
    out = torch.full((B, s, nh, hd), float("nan"), dtype=torch.bfloat16, device=gpu)
    prism_amd.rope_decode_attention(qkv.to(gpu), dev["k_cache"], dev["v_cache"], cos.to(gpu), sin.to(gpu),
                                    cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                    n_heads=nh, n_kv=nkv, out=out)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "appended (rotated) K not bit-exact"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "appended V not bit-exact"
    assert_attn_close(out, ref, f"random rope case {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_random_page_copies_match_oracle(gpu, seed):
    """Batched page copies between two caches (whole or partial pages, direct and staged), whole
    pools bit-exact against oracle/page_ops.py."""
    from oracle import page_ops
    from prism_amd import FlashAttnKVCache
    rng = np.random.default_rng(17000 + seed)
    layers = int(rng.integers(1, 5))
    P = int([16, 32, 64, 256][rng.integers(4)])
    n_kv, hd = [(2, 64), (4, 128), (8, 128), (1, 128)][rng.integers(4)]
    pages = int(rng.integers(8, 60))
    n = int(rng.integers(1, pages // 2 + 1))
    staged = bool(rng.random() < 0.3)
    print(f"random page copies {seed}: layers={layers} P={P} kv={n_kv} hd={hd} pages={pages} n={n} staged={staged}",
          flush=True)
    caches = []
    for k in range(2):
        kv = FlashAttnKVCache(layers, n_kv, hd, pages, P, str(gpu), torch.bfloat16)
        g = torch.Generator(device=gpu).manual_seed(seed * 2 + k)
        kv.k_pool.normal_(generator=g)
        kv.v_pool.normal_(generator=g)
        caches.append(kv)
    src, dst = caches
    src_ids = [int(x) for x in rng.choice(pages, size=n, replace=False)]
    dst_ids = [int(x) for x in rng.choice(pages, size=n, replace=False)]
    fill = [int(x) for x in rng.integers(1, P + 1, size=n)] if rng.random() < 0.6 else None
    pools = lambda kv: [pa.bf16_bits(t) for t in kv.k_caches] + [pa.bf16_bits(t) for t in kv.v_caches]
    before_src, before_dst = pools(src), pools(dst)
    prism_amd.copy_pages(src, dst, src_ids, dst_ids, fill, staged=staged)
    torch.cuda.synchronize()
    expect = page_ops.copy_pages(before_src, before_dst, src_ids, dst_ids, fill)
    for got, exp in zip(pools(dst), expect):
        assert np.array_equal(got, exp)
    for got, exp in zip(pools(src), before_src):
        assert np.array_equal(got, exp), "source pool changed"


def draw_options(seed):
    rng = np.random.default_rng(21000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    g = nh // n_kv
    s_q = int(rng.integers(1, 64 // g + 1))
    batch = int(rng.integers(1, 33))
    ctx = rng.integers(0, 2500, size=batch)
    ctx[rng.random(batch) < 0.1] = 0
    return dict(batch=batch, ctx=[int(c) for c in ctx], page_size=int(PAGE_SIZES[rng.integers(len(PAGE_SIZES))]),
                n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q, causal=bool(rng.random() < 0.7),
                append=bool(rng.random() < 0.8), kernel=["auto", "auto", "heads"][rng.integers(3)],
                split=int([0, 0, 32, 64, 256, 4096][rng.integers(6)]),
                two_pass=[None, None, True, False][rng.integers(4)],
                # an explicit scale around the default 1/sqrt(head_dim) (Prism passes the default;
                # the bf16 P of the PV product puts scales several times larger past 1e-2)
                scale=None if rng.random() < 0.5 else float(rng.uniform(0.5, 1.5) / np.sqrt(hd)),
                strided=bool(rng.random() < 0.5), seed=seed)


@pytest.mark.parametrize("seed", range(32))
def test_random_call_options_match_oracle(gpu, seed):
    """The decode / verify call with the options Prism and flash_attn expose: split lengths, the
    per-head kernel, either merge, an explicit softmax scale, q / k / v as strided views of one
    fused projection buffer, and up to 64 query rows per KV head."""
    c = draw_options(seed)
    B, nh, n_kv, hd, s = c["batch"], c["n_heads"], c["n_kv"], c["head_dim"], c["s_q"]
    print(f"random options case {seed}: {c}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=B, ctx=c["ctx"], page_size=c["page_size"], n_kv=n_kv, n_heads=nh,
                               head_dim=hd, s_q=s, seed=seed)
    q, k, v = dev["q"], dev["k"], dev["v"]
    if c["strided"]:
        qs, kvs = nh * hd, n_kv * hd
        qkv = torch.cat([q.reshape(B, s, qs), k.reshape(B, s, kvs), v.reshape(B, s, kvs)], dim=-1)
        q = qkv[:, :, :qs].view(B, s, nh, hd)
        k = qkv[:, :, qs:qs + kvs].view(B, s, n_kv, hd)
        v = qkv[:, :, qs + kvs:].view(B, s, n_kv, hd)
    if not c["append"]:
        k = v = None
    out = torch.full_like(dev["q"], float("nan"))
    out = prism_amd.flash_attn_with_kvcache(q, dev["k_cache"], dev["v_cache"], k, v,
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=c["causal"], softmax_scale=c["scale"], split_tokens=c["split"],
                                            kernel=c["kernel"], two_pass=c["two_pass"], out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if c["append"] else None,
        cpu["v"] if c["append"] else None, cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
        causal=c["causal"], softmax_scale=c["scale"])
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random options case {seed}")


def _ulp_close(got, ref, what, ulps=1.0):
    g = got.float().cpu().numpy().astype(np.float64)
    tol = ulps * np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7 + 1e-30
    bad = np.abs(g - ref) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond {ulps} bf16 unit(s)"


@pytest.mark.parametrize("seed", range(16))
def test_random_epilogue_kernels_match_oracle(gpu, seed):
    """rope_qk (bit-exact to the reference's bf16 expression), add + RMSNorm and SiLU-mul (within one
    bf16 unit of fp64) at random row counts and widths, strided gate / up views included."""
    from oracle import epilogue as ep
    rng = np.random.default_rng(25000 + seed)
    g = torch.Generator().manual_seed(seed)
    rnd = lambda shape, scale=1.0: (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    B, s = int(rng.integers(1, 65)), int([1, 1, 2, 5, 17, 64][rng.integers(6)])
    print(f"random epilogue case {seed}: B={B} s={s} h={nh} kv={n_kv} hd={hd}", flush=True)
    qkv = rnd((B, s, (nh + 2 * n_kv) * hd), 2.0)
    pos = rng.integers(0, 6000, size=B).astype(np.int32)
    cos, sin = ep.rope_tables(hd, 6100)
    q_ref, k_ref, _ = ep.qkv_split_rope(qkv, pos, cos, sin, nh, n_kv)
    q, k = prism_amd.rope_qk(qkv.to(gpu), torch.from_numpy(pos).to(gpu), cos.to(gpu), sin.to(gpu), nh, n_kv)
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), q_ref) and torch.equal(k.cpu(), k_ref), "rope_qk not bit-exact"
    rows, hidden = int(rng.integers(1, 70)), int([896, 1536, 2048, 3584, 5120, 8192][rng.integers(6)])
    x, w = rnd((rows, hidden), 3.0), rnd((hidden,))
    resid = bool(rng.random() < 0.5)
    r = rnd((rows, hidden)) if resid else None
    ref, h_ref = ep.rms_norm_f64(x.float().numpy(), w.float().numpy(), 1e-6, r.float().numpy() if resid else None)
    res = prism_amd.rms_norm(x.to(gpu), w.to(gpu), 1e-6, residual=r.to(gpu) if resid else None)
    torch.cuda.synchronize()
    _ulp_close(res[0] if resid else res, ep.round_bf16(ref), "rms_norm")
    if resid:
        assert np.array_equal(res[1].float().cpu().numpy(), h_ref), "residual sum not bit-exact"
    m = int([4864, 8960, 13824, 18944, 1000][rng.integers(5)])
    gu = rnd((rows, 2 * m), 3.0)
    sref = ep.silu_mul_ref(gu[:, :m].float().numpy(), gu[:, m:].float().numpy())
    d = gu.to(gpu)
    out = prism_amd.silu_mul(d[:, :m], d[:, m:])
    torch.cuda.synchronize()
    _ulp_close(out, sref, "silu_mul")


@pytest.mark.parametrize("seed", range(16))
def test_random_launch_shapes_match_oracle(gpu, seed):
    """The balanced kernel on an explicit number of workgroups (1 to 600, so ranges from hundreds
    of tiles down to none), flash_attn's num_splits, and batches past the balanced kernel's 256."""
    rng = np.random.default_rng(29000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    g = nh // n_kv
    s_q = int(rng.integers(1, 16 // g + 2)) if g < 16 else 1
    mode = ["grid", "grid", "splits", "big"][rng.integers(4)]
    batch = int(rng.integers(257, 301)) if mode == "big" else int(rng.integers(1, 41))
    ctx = rng.integers(0, 600 if mode == "big" else 2500, size=batch)
    ctx[rng.random(batch) < 0.1] = 0
    heads_per_tile = 4 if n_kv % 4 == 0 else (2 if n_kv % 2 == 0 else 1)
    P = int(max(32 * (4 // heads_per_tile) * (128 // hd), [16, 32, 64, 128, 256][rng.integers(5)]))
    grid = int([1, 2, 3, 7, 33, 100, 256, 300, 600][rng.integers(9)]) if mode == "grid" else 0
    num_splits = int(rng.integers(1, 9)) if mode == "splits" else 0
    two_pass = [None, True, False][rng.integers(3)]
    print(f"random launch case {seed}: mode={mode} B={batch} P={P} h={nh} kv={n_kv} hd={hd} s_q={s_q} grid={grid} "
          f"num_splits={num_splits} two_pass={two_pass}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=batch, ctx=[int(c) for c in ctx], page_size=P, n_kv=n_kv, n_heads=nh,
                               head_dim=hd, s_q=s_q, seed=seed)
    out = torch.full_like(dev["q"], float("nan"))
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=True, grid=grid, num_splits=num_splits, two_pass=two_pass,
                                            out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                                 cache_seqlens=cpu["cache_seqlens"],
                                                 block_table=cpu["block_table"], causal=True)
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random launch case {seed}")
    assert prism_amd.read_status(gpu) == 0


@pytest.mark.parametrize("seed", range(24))
def test_random_forced_prefill_kernel_matches_oracle(gpu, seed):
    """prefill_attention (the row-parallel prefill kernels, whatever s_q) at small and odd shapes:
    1-300 query tokens, causal or not, append or not, every page size and head geometry."""
    rng = np.random.default_rng(33000 + seed)
    nh, n_kv, hd = GEOMETRIES[rng.integers(len(GEOMETRIES))]
    batch = int(rng.integers(1, 9))
    ctx = rng.integers(0, 2000, size=batch)
    ctx[rng.random(batch) < 0.2] = 0
    s_q = int(rng.integers(1, 301))
    P = int(PAGE_SIZES[rng.integers(len(PAGE_SIZES))])
    causal, append = bool(rng.random() < 0.7), bool(rng.random() < 0.7)
    print(f"random forced prefill case {seed}: B={batch} ctx={list(ctx)} P={P} h={nh} kv={n_kv} hd={hd} s_q={s_q} "
          f"causal={causal} append={append}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=batch, ctx=[int(c) for c in ctx], page_size=P, n_kv=n_kv, n_heads=nh,
                               head_dim=hd, s_q=s_q, seed=seed)
    k = dev["k"] if append else None
    v = dev["v"] if append else None
    out = torch.full_like(dev["q"], float("nan"))
    out = prism_amd.prefill_attention(dev["q"], dev["k_cache"], dev["v_cache"], k, v,
                                      cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                      causal=causal, out=out)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if append else None, cpu["v"] if append else None,
        cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"], causal=causal)
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, f"random forced prefill case {seed}")


@pytest.mark.parametrize("seed", range(6))
def test_random_cache_lifecycle_keeps_every_sequence_exact(gpu, seed):
    """A random life of one FlashAttnKVCache on the device: sequences created, grown by decode and
    chunk appends through the drop-in attention call (which appends), forked (shared pages,
    copy-on-write on the next write), freed and compacted.  A host mirror keeps each sequence's
    K / V rows; after every step each live sequence's rows, gathered through its page list, are
    bit-identical to the mirror, and every attention output is bit-identical to the same call on
    a fresh cache holding the mirror's rows in consecutive pages (the attention arithmetic itself
    is checked against the oracle by the other sweeps)."""
    from prism_amd import FlashAttnKVCache
    rng = np.random.default_rng(37000 + seed)
    nh, n_kv, hd = [(28, 4, 128), (14, 2, 64), (40, 8, 128), (7, 1, 128)][seed % 4]
    P = int([16, 32, 64, 256][rng.integers(4)])
    kv = FlashAttnKVCache(1, n_kv, hd, 160 if P >= 64 else 600, P, str(gpu), torch.bfloat16)
    kv.k_pool.zero_()
    kv.v_pool.zero_()
    mirror_k: dict[int, np.ndarray] = {}
    mirror_v: dict[int, np.ndarray] = {}
    next_id = 0

    def gather(sid):
        L = kv.seq_len[sid]
        pages = kv.seq_pages[sid]
        kc, vc = pa.bf16_bits(kv.k_caches[0]), pa.bf16_bits(kv.v_caches[0])
        rows = [(pages[t // P], t % P) for t in range(L)]
        return (np.array([kc[p, r] for p, r in rows]).reshape(L, n_kv, hd),
                np.array([vc[p, r] for p, r in rows]).reshape(L, n_kv, hd))

    for step in range(14):
        live = sorted(mirror_k)
        op = rng.random()
        if not live or (op < 0.25 and len(live) < 6):
            kv.new_sequence(next_id)
            kv.seq_len[next_id] = 0
            mirror_k[next_id] = np.zeros((0, n_kv, hd), np.uint16)
            mirror_v[next_id] = np.zeros((0, n_kv, hd), np.uint16)
            next_id += 1
        elif op < 0.35 and len(live) < 6:
            src = int(rng.choice(live))
            if kv.seq_len[src] > 0:
                kv.fork_sequence(src, next_id)
                mirror_k[next_id], mirror_v[next_id] = mirror_k[src].copy(), mirror_v[src].copy()
                next_id += 1
        elif op < 0.45 and len(live) > 1:
            victim = int(rng.choice(live))
            kv.free_sequence(victim)
            del mirror_k[victim], mirror_v[victim]
        elif op < 0.55:
            kv.compact()
        live = sorted(mirror_k)
        # one attention call that appends s_q new rows to a batch of the live sequences
        batch = [int(x) for x in rng.choice(live, size=int(rng.integers(1, len(live) + 1)), replace=False)]
        s_q = int([1, 1, 1, 3, 17, 40][rng.integers(6)])
        if kv.pages_free < len(batch) * (s_q // P + 2) + 2:
            continue
        kv.prepare_append(batch, s_q)
        bt, sl = kv.build_block_table(batch)
        g = torch.Generator().manual_seed(seed * 100 + step)
        q = torch.randn(len(batch), s_q, nh, hd, generator=g).to(torch.bfloat16)
        k = torch.randn(len(batch), s_q, n_kv, hd, generator=g).to(torch.bfloat16)
        v = torch.randn(len(batch), s_q, n_kv, hd, generator=g).to(torch.bfloat16)
        out = prism_amd.flash_attn_with_kvcache(q.to(gpu), kv.k_caches[0], kv.v_caches[0], k.to(gpu), v.to(gpu),
                                                cache_seqlens=sl, block_table=bt, causal=True)
        # the same call on a fresh cache holding the mirror's rows in consecutive pages: the kernels'
        # arithmetic depends on lengths and token positions only, so the outputs must match bit for
        # bit whatever pages, forks, copies and compactions the first cache went through
        lens = [len(mirror_k[sid]) for sid in batch]
        need = [-(-(L + s_q) // P) for L in lens]
        fk = torch.zeros(sum(need), P, n_kv, hd, dtype=torch.bfloat16)
        fv = torch.zeros_like(fk)
        fbt = torch.zeros(len(batch), max(need), dtype=torch.int32)
        base = 0
        for i, sid in enumerate(batch):
            L = lens[i]
            fbt[i, :need[i]] = torch.arange(base, base + need[i], dtype=torch.int32)
            rows_k = torch.from_numpy(mirror_k[sid].astype(np.int16)).view(torch.bfloat16)
            rows_v = torch.from_numpy(mirror_v[sid].astype(np.int16)).view(torch.bfloat16)
            fk.view(-1, n_kv, hd)[base * P: base * P + L] = rows_k
            fv.view(-1, n_kv, hd)[base * P: base * P + L] = rows_v
            base += need[i]
        out2 = prism_amd.flash_attn_with_kvcache(q.to(gpu), fk.to(gpu), fv.to(gpu), k.to(gpu), v.to(gpu),
                                                 cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=gpu),
                                                 block_table=fbt.to(gpu), causal=True)
        torch.cuda.synchronize()
        assert torch.equal(out, out2), f"lifecycle {seed} step {step}: output depends on the page layout"
        kv.update_seqlens(batch, s_q)
        for i, sid in enumerate(batch):
            mirror_k[sid] = np.concatenate([mirror_k[sid], pa.bf16_bits(k[i])])
            mirror_v[sid] = np.concatenate([mirror_v[sid], pa.bf16_bits(v[i])])
        for sid in mirror_k:
            gk, gv = gather(sid)
            assert np.array_equal(gk, mirror_k[sid]) and np.array_equal(gv, mirror_v[sid]), \
                f"lifecycle {seed} step {step}: sequence {sid} rows differ"


# Seeds of the draws above (beyond their committed ranges) whose worst rows land past 1e-2: rows of
# an empty-cache sequence that see 2-7 keys, where the bf16 output's own rounding (half an ulp,
# 0.0156 at |o| > 4) or bf16 P (flash_attn's rounding for the PV product) decides the last bit.
EDGE_SEEDS = [("decode", 5283), ("decode", 5856), ("prefill", 292), ("prefill", 701), ("prefill", 817)]


@pytest.mark.parametrize("kind,seed", EDGE_SEEDS)
def test_tolerance_edge_rows_stay_within_one_output_ulp(gpu, kind, seed):
    """Every element within max(1e-2, one bf16 ulp of the exact value); the elements past 1e-2 only
    on rows that see at most 8 keys; mean-abs within 1e-3."""
    c = draw(seed) if kind == "decode" else draw_prefill(seed)
    print(f"edge case {kind} {seed}: B={c['batch']} s_q={c['s_q']} h={c['n_heads']} kv={c['n_kv']}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=c["batch"], ctx=c["ctx"], page_size=c["page_size"], n_kv=c["n_kv"],
                               n_heads=c["n_heads"], head_dim=c["head_dim"], s_q=c["s_q"], seed=seed)
    k = dev["k"] if c["append"] else None
    v = dev["v"] if c["append"] else None
    out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], k, v,
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=c["causal"])
    torch.cuda.synchronize()
    ref, _, _ = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if c["append"] else None,
        cpu["v"] if c["append"] else None, cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
        causal=c["causal"])
    err = np.abs(out.float().cpu().numpy() - ref)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert (err <= np.maximum(1e-2, ulp)).all(), f"max error over the bound {float((err - np.maximum(1e-2, ulp)).max())}"
    assert err.mean() <= 1e-3
    L = cpu["cache_seqlens"].numpy() + (c["s_q"] if c["append"] else 0)
    seen = L[:, None] - c["s_q"] + np.arange(c["s_q"])[None, :] + 1          # keys row r of sequence b sees
    b, r = np.nonzero(err.max(axis=(2, 3)) > 1e-2)
    assert (seen[b, r] <= 8).all(), f"rows past 1e-2 that see many keys: {sorted(set(seen[b, r].tolist()))}"
    print(f"  max-abs {err.max():.4f}; rows past 1e-2: {len(b)}, keys seen {sorted(set(seen[b, r].tolist()))}",
          flush=True)
