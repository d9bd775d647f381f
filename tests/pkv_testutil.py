"""Shared helpers for the parity tests (inputs, tolerance checks).

The attention tolerance is the one BASELINE.json's north_star states for bf16 outputs versus an
fp32-accumulated reference: max-abs <= 1e-2 and mean-abs <= 1e-3, measured between the kernel's
bf16 output and the unrounded fp64 oracle.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import paged_attention as pa


ATOL_MAX = 1e-2
ATOL_MEAN = 1e-3


def attn_errors(out: torch.Tensor, ref64: np.ndarray) -> tuple[float, float]:
    got = out.detach().float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref64)
    return float(err.max(initial=0.0)), float(err.mean()) if err.size else 0.0


def assert_attn_close(out: torch.Tensor, ref64: np.ndarray, what: str = "") -> None:
    assert out.shape == ref64.shape, (out.shape, ref64.shape)
    got = out.detach().float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    mx, mean = attn_errors(out, ref64)
    assert mx <= ATOL_MAX and mean <= ATOL_MEAN, f"{what}: max-abs {mx:.3g} mean-abs {mean:.3g}"


def make_paged_case(device, *, batch, ctx, page_size, n_kv, n_heads, head_dim, s_q, num_pages=None,
                    seed=0, fragment=True, extra_cols=0):
    """Random pool + disjoint shuffled page assignment; returns dict of device tensors."""
    g = torch.Generator().manual_seed(seed)
    ctx = np.asarray(ctx, dtype=np.int64)
    need = np.ceil((ctx + s_q) / page_size).astype(np.int64).clip(min=1)
    total = int(need.sum())
    num_pages = num_pages or total + 5
    kc = torch.randn(num_pages, page_size, n_kv, head_dim, generator=g).to(torch.bfloat16)
    vc = torch.randn(num_pages, page_size, n_kv, head_dim, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_pages, generator=g) if fragment else torch.arange(num_pages)
    width = int(need.max()) + extra_cols
    bt = torch.zeros(batch, width, dtype=torch.int32)
    off = 0
    for b in range(batch):
        bt[b, : need[b]] = perm[off: off + need[b]].to(torch.int32)
        off += int(need[b])
    q = torch.randn(batch, s_q, n_heads, head_dim, generator=g).to(torch.bfloat16)
    k = torch.randn(batch, s_q, n_kv, head_dim, generator=g).to(torch.bfloat16)
    v = torch.randn(batch, s_q, n_kv, head_dim, generator=g).to(torch.bfloat16)
    sl = torch.tensor(ctx, dtype=torch.int32)
    cpu = dict(q=q, k=k, v=v, k_cache=kc, v_cache=vc, block_table=bt, cache_seqlens=sl)
    dev = {n: t.to(device) for n, t in cpu.items()}
    return cpu, dev


def free_cached():
    """Return the caching allocator's free blocks (the callers drop their references first)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _referenced(bt: np.ndarray, keys: np.ndarray, P: int) -> np.ndarray:
    """Sorted page ids of the columns each sequence needs for `keys[b]` keys."""
    used = set()
    for b in range(bt.shape[0]):
        n = max(1, -(-int(keys[b]) // P))
        used.update(int(x) for x in bt[b, :n])
    return np.array(sorted(used), dtype=np.int64)


class LayerCheck:
    """Snapshot of one layer's referenced pages (and the whole pool, on the device) before a call,
    then the oracle comparison after it."""

    def __init__(self, w, layer: int, kv_heads=None):
        kv = w.kv
        self.w, self.layer, self.kv_heads = w, layer, kv_heads
        P = kv.page_size
        self.bt = w.block_table.cpu().numpy().astype(np.int64)
        self.sl = w.cache_seqlens.cpu().numpy().astype(np.int64)
        self.used = _referenced(self.bt, self.sl + w.s_q, P)
        assert (self.used >= 0).all() and (self.used < kv.max_pages).all()
        remap = np.full(kv.max_pages, -1, dtype=np.int64)
        remap[self.used] = np.arange(len(self.used))
        self.bt_mini = np.where(self.bt >= 0, remap[self.bt.clip(min=0)], -1)
        self.idx = torch.from_numpy(self.used).to(kv.k_pool.device)
        self.k_pre = kv.k_caches[layer].index_select(0, self.idx).cpu()
        self.v_pre = kv.v_caches[layer].index_select(0, self.idx).cpu()
        self.k_full = kv.k_caches[layer].clone()
        self.v_full = kv.v_caches[layer].clone()

    def check(self, out: torch.Tensor, what: str, append: bool = True, rows=None) -> tuple[float, float]:
        """rows: a sorted sample of query positions the fp64 oracle checks (all when None)."""
        w, kv, l = self.w, self.w.kv, self.layer
        torch.cuda.synchronize()
        q, k, v = w.q[l].cpu(), w.k[l].cpu(), w.v[l].cpu()
        bt = torch.from_numpy(self.bt_mini.clip(min=0).astype(np.int32))
        sl = torch.from_numpy(self.sl.astype(np.int32))
        # bit-exact append on the referenced pages (every head)
        kb, vb = pa.append_kv(pa.bf16_bits(self.k_pre), pa.bf16_bits(self.v_pre), pa.bf16_bits(k),
                              pa.bf16_bits(v), self.bt_mini.clip(min=0), self.sl) if append else \
            (pa.bf16_bits(self.k_pre), pa.bf16_bits(self.v_pre))
        got_k = pa.bf16_bits(kv.k_caches[l].index_select(0, self.idx))
        got_v = pa.bf16_bits(kv.v_caches[l].index_select(0, self.idx))
        assert np.array_equal(got_k, kb), f"{what}: K pages not bit-exact after append"
        assert np.array_equal(got_v, vb), f"{what}: V pages not bit-exact after append"
        # every other page of the pool untouched
        keep = torch.ones(kv.max_pages, dtype=torch.bool, device=self.idx.device)
        keep[self.idx] = False
        assert torch.equal(kv.k_caches[l][keep], self.k_full[keep]), f"{what}: a K page outside the batch changed"
        assert torch.equal(kv.v_caches[l][keep], self.v_full[keep]), f"{what}: a V page outside the batch changed"
        # attention against the fp64 oracle (optionally on a sample of KV heads)
        kc, vc = pa.bits_to_bf16(kb), pa.bits_to_bf16(vb)
        got = out.detach().cpu()
        if self.kv_heads is not None:
            g = w.n_heads // kv.num_kv_heads
            qh = [h for kh in self.kv_heads for h in range(kh * g, (kh + 1) * g)]
            q, got = q[:, :, qh], got[:, :, qh]
            kc, vc = kc[:, :, self.kv_heads].contiguous(), vc[:, :, self.kv_heads].contiguous()
        if rows is not None:
            got = got[:, rows]
        ref = pa.attention_fp64(pa.bf16_bits(q), pa.bf16_bits(kc), pa.bf16_bits(vc), bt.numpy().astype(np.int64),
                                self.sl + w.s_q, True, rows=rows)
        assert_attn_close(got, ref, what)
        mx, mean = attn_errors(got, ref)
        print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e} over {got.numel()} outputs", flush=True)
        return mx, mean
