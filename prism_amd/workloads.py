"""Seeded synthetic workloads for the five benchmark configurations of the paged KV path.

Shapes are Qwen2.5's: 0.5B nh=14 / n_kv=2 / hd=64; 7B 28 / 4 / 128 (28 layers); 14B 40 / 8 / 128
(48 layers); page size 256; bf16 K/V/Q ~ N(0, 1).  Pools are sized like Prism's scheduler does
(engine/scheduler.py:99-103): bytes_per_page = 2 * P * n_kv * hd * 2 * L, max_pages =
int(budget_gb * 1e9 / bytes_per_page) -- 2043 pages for 7B at 30 GB, 596 for 14B.

Lengths and page permutations come from numpy's default_rng(seed); tensors from a torch.Generator
on the target device seeded with the same seed.  Everything is built through the product's own
FlashAttnKVCache (allocation by LIFO pop after a seeded free-list order), so the block tables are
exactly what a serving run would hand the kernels.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from .kv_cache import FlashAttnKVCache

SHAPES = {
    "0.5B": dict(n_heads=14, n_kv=2, head_dim=64, layers=24),
    "7B": dict(n_heads=28, n_kv=4, head_dim=128, layers=28),
    "14B": dict(n_heads=40, n_kv=8, head_dim=128, layers=48),
    # one GPU's share of the 7B model under 4-way tensor parallelism (KV heads split across GPUs)
    "7B-tp4": dict(n_heads=7, n_kv=1, head_dim=128, layers=28),
}
PAGE = 256


def pages_for_budget(budget_gb: float, layers: int, n_kv: int, head_dim: int, page_size: int = PAGE) -> int:
    """engine/scheduler.py:100-103 page budget."""
    bytes_per_page = 2 * page_size * n_kv * head_dim * 2 * layers
    return max(int(budget_gb * 1e9 / bytes_per_page), 16)


@dataclass
class PagedWorkload:
    """One batch of sequences over a paged pool, with per-layer new K/V rows and queries."""
    name: str
    kv: FlashAttnKVCache
    seq_ids: list[int]
    ctx: np.ndarray              # cache length of each sequence before this step's append
    s_q: int                     # query / appended rows per sequence
    n_heads: int
    q: list[torch.Tensor]        # per layer [B, s_q, n_heads, hd]
    k: list[torch.Tensor]        # per layer [B, s_q, n_kv, hd]
    v: list[torch.Tensor]
    block_table: torch.Tensor    # [B, max_blocks] int32 (device)
    cache_seqlens: torch.Tensor  # [B] int32 (device), = ctx
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return len(self.seq_ids)

    @property
    def layers(self) -> int:
        return len(self.q)

    def keys_total(self) -> np.ndarray:
        return self.ctx.astype(np.int64) + self.s_q

    def decode_bytes_per_layer(self) -> int:
        """Algorithmic HBM bytes of one append + attention call (bf16, int32 tables):
        K+V rows read, Q read + O written, new K+V rows written, block-table entries + seqlens."""
        kv = self.kv
        keys = self.keys_total()
        row = kv.num_kv_heads * kv.head_dim * 2
        pages = np.ceil(keys / kv.page_size).astype(np.int64)
        return int(keys.sum() * row * 2
                   + self.batch * self.s_q * self.n_heads * kv.head_dim * 2 * 2
                   + self.batch * self.s_q * row * 2
                   + 4 * (pages.sum() + self.batch))

    def attention_flops_per_layer(self) -> int:
        """4 * n_heads * hd * sum_b sum_j (visible keys of query j), causal-exact."""
        keys = self.keys_total()
        vis = (keys[:, None] - self.s_q + np.arange(self.s_q)[None, :] + 1).clip(min=0).sum()
        return int(4 * self.n_heads * self.kv.head_dim * vis)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _fill_pool(kv: FlashAttnKVCache, g: torch.Generator) -> None:
    for t in (kv.k_pool, kv.v_pool):
        for layer in range(t.shape[0]):
            t[layer].normal_(0.0, 1.0, generator=g)


def _rand(shape, g, device) -> torch.Tensor:
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


def _finish(name, kv, seq_ids, ctx, s_q, n_heads, g, device, meta) -> PagedWorkload:
    B = len(seq_ids)
    L = kv.num_layers
    q = [_rand((B, s_q, n_heads, kv.head_dim), g, device) for _ in range(L)]
    k = [_rand((B, s_q, kv.num_kv_heads, kv.head_dim), g, device) for _ in range(L)]
    v = [_rand((B, s_q, kv.num_kv_heads, kv.head_dim), g, device) for _ in range(L)]
    bt, sl = kv.build_block_table(seq_ids)
    return PagedWorkload(name, kv, list(seq_ids), np.asarray(ctx, dtype=np.int64), s_q, n_heads, q, k, v,
                         bt.clone(), sl.clone(), meta)


def _alloc(kv: FlashAttnKVCache, seq_ids, ctx, s_new: int) -> None:
    """Allocate pages by LIFO pop so each sequence holds ctx + s_new rows; seq_len = ctx."""
    for sid, c in zip(seq_ids, ctx):
        kv.new_sequence(sid)
        kv._ensure_capacity(sid, int(c) + s_new)
        kv.seq_len[sid] = int(c)


def config1(device="cuda", seed=0) -> PagedWorkload:
    """0.5B shape, 1 layer, B=4, ctx ~ U{1..1024}, tables consecutive from randperm(64)."""
    s = SHAPES["0.5B"]
    rng = np.random.default_rng(seed)
    kv = FlashAttnKVCache(1, s["n_kv"], s["head_dim"], 64, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    ctx = rng.integers(1, 1025, size=4)
    perm = rng.permutation(64)
    kv.free_pages = [int(p) for p in perm[::-1]]   # pop() hands out perm[0], perm[1], ...
    _alloc(kv, range(4), ctx, 1)
    return _finish("config1", kv, list(range(4)), ctx, 1, s["n_heads"], g, device, {"shape": "0.5B"})


def config2(device="cuda", seed=0, layers=None, max_pages=None, batch=8, ctx_len=2048) -> PagedWorkload:
    """7B full decode step: B=8 at context 2048, pages scattered over a 30 GB pool."""
    s = SHAPES["7B"]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = max_pages or pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    kv.free_pages = [int(p) for p in rng.permutation(mp)]
    ctx = np.full(batch, ctx_len, dtype=np.int64)
    _alloc(kv, range(batch), ctx, 1)
    return _finish("config2", kv, list(range(batch)), ctx, 1, s["n_heads"], g, device, {"shape": "7B"})


def lognormal_ctx(rng, batch, median=1500.0, sigma=1.0, lo=16, hi=32768) -> np.ndarray:
    return np.clip(np.round(rng.lognormal(math.log(median), sigma, size=batch)), lo, hi).astype(np.int64)


def config3(device="cuda", seed=0, layers=None, max_pages=None, batch=32, churn=0.4) -> PagedWorkload:
    """Headline: 7B ragged decode, B=32, ctx lognormal(median 1500, sigma 1) in [16, 32768], pool
    fragmented by freeing a seeded 40% of a fully used pool in random order, then LIFO allocation."""
    s = SHAPES["7B"]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = max_pages or pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    ctx = lognormal_ctx(rng, batch)
    # all pages in use, then a seeded 40% freed in random order (the free list is that order)
    freed = rng.permutation(mp)[: int(round(churn * mp))]
    need = int(np.ceil((ctx + 1) / PAGE).sum())
    if need > len(freed):
        raise RuntimeError(f"config3 seed {seed}: {need} pages needed > {len(freed)} free")
    kv.free_pages = [int(p) for p in freed]
    _alloc(kv, range(batch), ctx, 1)
    return _finish("config3", kv, list(range(batch)), ctx, 1, s["n_heads"], g, device,
                   {"shape": "7B", "pool_pages": mp, "free_after_churn": len(freed)})


def ragged_decode(shape: str, device="cuda", seed=0, layers=None, max_pages=None, batch=32, churn=0.4,
                  budget_gb=30.0, force: dict[int, int] | None = None, name: str | None = None) -> PagedWorkload:
    """config3's ragged decode batch (lognormal lengths, churned pool, LIFO allocation) at another
    model shape: the Qwen2.5-14B (8 KV heads) and 0.5B (2 KV heads, head_dim 64) decode steps, and
    the 7B step on one GPU of a 4-way tensor-parallel group (1 KV head).  The pool is the model's
    30 GB budget, capped at 4096 pages.  force {index: context} replaces drawn lengths (the long
    end of config 3's [16, 32768] range)."""
    s = SHAPES[shape]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = max_pages or min(pages_for_budget(budget_gb, s["layers"], s["n_kv"], s["head_dim"]), 4096)
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    ctx = lognormal_ctx(rng, batch)
    for i, c in (force or {}).items():
        ctx[i] = c
    freed = rng.permutation(mp)[: int(round(churn * mp))]
    need = int(np.ceil((ctx + 1) / PAGE).sum())
    if need > len(freed):
        raise RuntimeError(f"ragged_decode {shape} seed {seed}: {need} pages needed > {len(freed)} free")
    kv.free_pages = [int(p) for p in freed]
    _alloc(kv, range(batch), ctx, 1)
    return _finish(name or f"decode-{shape}", kv, list(range(batch)), ctx, 1, s["n_heads"], g, device,
                   {"shape": shape, "pool_pages": mp})


# config 3's long end: a sequence at the 32768-token clip (32767 keys before the append) beside a
# 12000-token one, in the seed's ragged batch; and one sequence alone at the clip (the B = 1 graph)
LONG_FORCE = {0: 32767, 1: 12000}


def long_decode(device="cuda", seed=0, layers=None, shape: str = "7B", batch: int = 32) -> PagedWorkload:
    """Decode past the executor's 32-page graph limit (engine/executor.py:343, :385-386): config 3's
    ragged 7B batch with sequence 0 at 32767 cached keys and sequence 1 at 12000 (batch > 1), or a
    single sequence at 32767 keys (batch = 1)."""
    force = {0: LONG_FORCE[0]} if batch == 1 else dict(LONG_FORCE)
    name = f"long-decode-{shape}-b{batch}"
    return ragged_decode(shape, device, seed=seed, layers=layers, batch=batch, force=force, name=name)


def prompt_prefill(device="cuda", seed=0, layers=None, shape: str = "7B", prompt: int = 4096,
                   batch: int = 1) -> PagedWorkload:
    """Whole-prompt prefill (engine/executor.py:97-120): `batch` sequences with no cached prefix, each
    appending and attending a `prompt`-token chunk (causal), on the model's 30 GB pool with pages
    scattered by a seeded permutation of the free list."""
    s = SHAPES[shape]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    kv.free_pages = [int(p) for p in rng.permutation(mp)]
    ctx = np.zeros(batch, dtype=np.int64)
    _alloc(kv, range(batch), ctx, prompt)
    return _finish(f"prefill-{shape}-{prompt}", kv, list(range(batch)), ctx, prompt, s["n_heads"], g, device,
                   {"shape": shape})


def config4(device="cuda", seed=0, layers=None, max_pages=None, batch=8, chunk=512, max_prefix=4096) -> PagedWorkload:
    """14B varlen chunked prefill: B=8 chunks of 512 onto prefixes ~ U{0..4096}."""
    s = SHAPES["14B"]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = max_pages or pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    kv.free_pages = [int(p) for p in rng.permutation(mp)]
    ctx = rng.integers(0, max_prefix + 1, size=batch)
    _alloc(kv, range(batch), ctx, chunk)
    return _finish("config4", kv, list(range(batch)), ctx, chunk, s["n_heads"], g, device, {"shape": "14B"})


def config5(device="cuda", seed=0, layers=None, max_pages=None, batch=64, prefix=2048, max_suffix=1024,
            draft=5, prefix_cache=None, before_cow=None) -> PagedWorkload:
    """7B prefix sharing + speculative verify.

    A root sequence holds a shared prefix of 2048 - r tokens (r seeded in [1, 255], so the last
    prefix page is partially filled); its full pages are stored in the prefix cache when one is
    given.  `batch` sequences fork the root (sharing all its pages), the root is freed, and each
    child grows by a private suffix ~ U{0..1024}: the first write into the shared boundary page
    copies it (one batched copy-on-write launch).  The step then verifies `draft` tokens per
    sequence (s_q = 5, causal within the 5).  before_cow(kv), when given, runs right before that
    copy-on-write (a parity test snapshots the pool there).
    """
    s = SHAPES["7B"]
    L = layers or s["layers"]
    rng = np.random.default_rng(seed)
    mp = max_pages or pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    kv = FlashAttnKVCache(L, s["n_kv"], s["head_dim"], mp, PAGE, device, torch.bfloat16)
    g = _gen(device, seed)
    _fill_pool(kv, g)
    kv.free_pages = [int(p) for p in rng.permutation(mp)]
    r = int(rng.integers(1, PAGE))
    shared = prefix - r
    root = 10_000
    kv.new_sequence(root, owner="target")
    kv._ensure_capacity(root, shared)
    kv.seq_len[root] = shared
    if prefix_cache is not None:
        # the cache cooperates with this pool: its pages stay off the free list while cached
        prefix_cache.kv = kv
        kv.prefix_cache = prefix_cache
        tokens = rng.integers(0, 150_000, size=shared).tolist()
        prefix_cache.store(tokens, kv.seq_pages[root], "target")
    ids = list(range(batch))
    root_pages = list(kv.seq_pages[root])  # the prefix's pages, the last one partially filled
    for sid in ids:
        kv.fork_sequence(root, sid)
    kv.free_sequence(root)
    suffix = rng.integers(0, max_suffix + 1, size=batch)
    if before_cow is not None:
        before_cow(kv)
    n_cow = kv.prepare_append(ids, [int(x) for x in suffix])
    for sid, x in zip(ids, suffix):
        kv.seq_len[sid] += int(x)
    kv.prepare_append(ids, draft)
    ctx = np.array([kv.seq_len[sid] for sid in ids], dtype=np.int64)
    return _finish("config5", kv, ids, ctx, draft, s["n_heads"], g, device,
                   {"shape": "7B", "shared_prefix": shared, "cow_copies": n_cow, "boundary_fill": shared % PAGE,
                    "root_pages": root_pages})
