"""Shared helpers for the parity tests (inputs, tolerance checks).

The attention tolerance is the one BASELINE.json's north_star states for bf16 outputs versus an
fp32-accumulated reference: max-abs <= 1e-2 and mean-abs <= 1e-3, measured between the kernel's
bf16 output and the unrounded fp64 oracle.
"""
from __future__ import annotations

import numpy as np
import torch


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
