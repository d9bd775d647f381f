"""ORACLE (test infrastructure): CPU restatement of flash_attn_with_kvcache as Prism uses it.

Prism calls the third-party flash_attn op (flash-attn "2.8+", README.md:198; unpinned
`pip install flash-attn`, Dockerfile:15) at engine/executor.py:119-120, :151-153, :260-261,
:385-386 and engine/speculative_executor.py:150-153 with
    flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens=sl,
                            block_table=bt, causal=True)
on the paged layout of engine/kv_cache.py:37-46 ([num_pages, page_size, n_kv, head_dim]) and
block tables of engine/kv_cache.py:123-153.  flash_attn is absent from /root/reference and from
this image, so its published semantics are restated here:
  * append: new row j of sequence b goes to slot cache_seqlens[b] + j, i.e. page
    block_table[b, slot // P], row slot % P (docs/architecture.md:129-147);
  * keys of sequence b: L_b = cache_seqlens[b] (+ s_q when k/v are appended);
  * causal mask aligned bottom-right: query j sees keys t <= L_b - s_q + j;
  * GQA: query head h reads KV head h // (n_heads / n_kv);
  * softmax_scale defaults to 1/sqrt(head_dim); a query row with no visible key outputs 0.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

import math

import numpy as np
import torch

# ------------------------------------------------------------------------------------------
# bf16 <-> bits helpers (numpy has no bfloat16; caches are handled as uint16 bit patterns)
# ------------------------------------------------------------------------------------------


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 ndarray of its bit patterns (CPU copy)."""
    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def bits_to_f64(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def bits_to_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp64/fp32 -> bf16 (round to nearest even, torch's rule) -> fp64 values."""
    t = torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.to(torch.float64).numpy()


# ------------------------------------------------------------------------------------------
# slot mapping and append (bit-exact index work)
# ------------------------------------------------------------------------------------------


def slot_mapping(block_table: np.ndarray, cache_seqlens: np.ndarray, s_new: int, page_size: int) -> np.ndarray:
    """Flat slot (page * page_size + row) of every appended row, int64 [B, s_new].

    slot of token t of sequence b = block_table[b, t // P] * P + t % P, t = cache_seqlens[b] + j
    (engine/kv_cache.py:123-153 table format; docs/architecture.md:140-147).
    """
    bt = np.asarray(block_table, dtype=np.int64)
    sl = np.asarray(cache_seqlens, dtype=np.int64)
    t = sl[:, None] + np.arange(s_new, dtype=np.int64)[None, :]
    pages = np.take_along_axis(bt, t // page_size, axis=1)
    return pages * page_size + t % page_size


def append_kv(k_bits: np.ndarray, v_bits: np.ndarray, k_new_bits: np.ndarray, v_new_bits: np.ndarray,
              block_table: np.ndarray, cache_seqlens: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Return copies of the [num_pages, P, n_kv, hd] uint16 caches with the new rows written."""
    num_pages, P, n_kv, hd = k_bits.shape
    B, s_new = k_new_bits.shape[:2]
    slots = slot_mapping(block_table, cache_seqlens, s_new, P)
    kf = k_bits.reshape(num_pages * P, n_kv, hd).copy()
    vf = v_bits.reshape(num_pages * P, n_kv, hd).copy()
    kf[slots.reshape(-1)] = k_new_bits.reshape(B * s_new, n_kv, hd)
    vf[slots.reshape(-1)] = v_new_bits.reshape(B * s_new, n_kv, hd)
    return kf.reshape(k_bits.shape), vf.reshape(v_bits.shape)


def append_kv_loop(k_bits, v_bits, k_new_bits, v_new_bits, block_table, cache_seqlens):
    """Per-row brute force of append_kv (pure Python loops; small cases only)."""
    k_out, v_out = k_bits.copy(), v_bits.copy()
    P = k_bits.shape[1]
    for b in range(k_new_bits.shape[0]):
        for j in range(k_new_bits.shape[1]):
            t = int(cache_seqlens[b]) + j
            page = int(block_table[b][t // P])
            k_out[page, t % P] = k_new_bits[b, j]
            v_out[page, t % P] = v_new_bits[b, j]
    return k_out, v_out


# ------------------------------------------------------------------------------------------
# attention
# ------------------------------------------------------------------------------------------


def causal_visible(s_q: int, L: int) -> np.ndarray:
    """Bool [s_q, L]: query j sees key t iff t <= L - s_q + j (bottom-right aligned)."""
    j = np.arange(s_q)[:, None]
    t = np.arange(L)[None, :]
    return t <= (L - s_q + j)


def gather_seq(cache_bits: np.ndarray, block_table_row: np.ndarray, L: int) -> np.ndarray:
    """Rows [0, L) of one sequence from a paged cache, uint16 [L, n_kv, hd]."""
    P = cache_bits.shape[1]
    t = np.arange(L)
    pages = np.asarray(block_table_row, dtype=np.int64)[t // P]
    return cache_bits[pages, t % P]


def attention_fp64(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, block_table: np.ndarray,
                   seqlens_k: np.ndarray, causal: bool, softmax_scale: float | None = None,
                   rows: np.ndarray | None = None) -> np.ndarray:
    """fp64 paged attention. q [B, s_q, nh, hd] bits; caches [pages, P, n_kv, hd] bits.

    seqlens_k[b] is the number of keys of sequence b (after any append).  Returns fp64
    [B, s_q, nh, hd]; rows with no visible key are 0.  With `rows` (sorted query positions),
    only those rows are computed and the result is [B, len(rows), nh, hd] (a long prefill chunk
    checked on a sample of its rows; the causal mask still counts every row's true position).
    """
    B, s_q, nh, hd = q_bits.shape
    n_kv = k_bits.shape[2]
    g = nh // n_kv
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(hd)
    sel = np.arange(s_q) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.zeros((B, len(sel), nh, hd), dtype=np.float64)
    for b in range(B):
        L = int(seqlens_k[b])
        if L <= 0:
            continue
        K = bits_to_f64(gather_seq(k_bits, block_table[b], L))  # [L, n_kv, hd]
        V = bits_to_f64(gather_seq(v_bits, block_table[b], L))
        Q = bits_to_f64(q_bits[b][sel])                         # [rows, nh, hd]
        vis = (causal_visible(s_q, L) if causal else np.ones((s_q, L), dtype=bool))[sel]
        for h in range(nh):
            kvh = h // g
            s = (Q[:, h, :] @ K[:, kvh, :].T) * scale          # [s_q, L]
            s = np.where(vis, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            has = np.isfinite(m[:, 0])
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.exp(s - m)
            denom = p.sum(axis=1, keepdims=True)
            o = (p @ V[:, kvh, :]) / np.where(denom > 0, denom, 1.0)
            out[b, :, h, :] = np.where(has[:, None], o, 0.0)
    return out


def flash_attn_with_kvcache_ref(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                k: torch.Tensor | None = None, v: torch.Tensor | None = None, *,
                                cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                                causal: bool = False, softmax_scale: float | None = None):
    """Oracle of the whole op: returns (out fp64 ndarray, k_cache bits, v_cache bits) after append."""
    qb = bf16_bits(q)
    kb, vb = bf16_bits(k_cache), bf16_bits(v_cache)
    bt = block_table.detach().cpu().numpy().astype(np.int64)
    sl = cache_seqlens.detach().cpu().numpy().astype(np.int64)
    s_q = q.shape[1]
    if k is not None:
        kb, vb = append_kv(kb, vb, bf16_bits(k), bf16_bits(v), bt, sl)
        lk = sl + s_q
    else:
        lk = sl
    out = attention_fp64(qb, kb, vb, bt, lk, causal, softmax_scale)
    return out, kb, vb


# ------------------------------------------------------------------------------------------
# torch-CPU reference path (the CPU baseline): index_select page gather + fp32 SDPA with GQA
# ------------------------------------------------------------------------------------------


def flash_attn_cpu(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   k: torch.Tensor | None = None, v: torch.Tensor | None = None, *,
                   cache_seqlens: torch.Tensor, block_table: torch.Tensor, causal: bool = False,
                   softmax_scale: float | None = None) -> torch.Tensor:
    """CPU torch path: append via flat index_copy_, gather pages via index_select, fp32 SDPA.

    Mutates k_cache/v_cache (CPU bf16) in place like the GPU op; returns fp32 [B, s_q, nh, hd].
    """
    B, s_q, nh, hd = q.shape
    num_pages, P, n_kv, _ = k_cache.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(hd)
    sl = cache_seqlens.to(torch.int64)
    bt = block_table.to(torch.int64)
    kf = k_cache.view(num_pages * P, n_kv, hd)
    vf = v_cache.view(num_pages * P, n_kv, hd)
    if k is not None:
        t = sl[:, None] + torch.arange(s_q)[None, :]
        slots = torch.gather(bt, 1, t // P) * P + t % P
        kf.index_copy_(0, slots.reshape(-1), k.reshape(B * s_q, n_kv, hd))
        vf.index_copy_(0, slots.reshape(-1), v.reshape(B * s_q, n_kv, hd))
        lk = sl + s_q
    else:
        lk = sl
    out = torch.zeros((B, s_q, nh, hd), dtype=torch.float32)
    for b in range(B):
        L = int(lk[b])
        if L <= 0:
            continue
        n_pages = -(-L // P)
        pages = bt[b, :n_pages]
        Kb = k_cache.index_select(0, pages).reshape(n_pages * P, n_kv, hd)[:L].float()
        Vb = v_cache.index_select(0, pages).reshape(n_pages * P, n_kv, hd)[:L].float()
        qh = q[b].float().transpose(0, 1)          # [nh, s_q, hd]
        kh = Kb.transpose(0, 1)                    # [n_kv, L, hd]
        vh = Vb.transpose(0, 1)
        if causal:
            j = torch.arange(s_q)[:, None]
            tt = torch.arange(L)[None, :]
            mask = tt <= (L - s_q + j)
        else:
            mask = None
        o = torch.nn.functional.scaled_dot_product_attention(
            qh, kh, vh, attn_mask=mask, scale=scale, enable_gqa=True)
        if causal:
            o = torch.where(mask.any(dim=1)[None, :, None], o, torch.zeros_like(o))
        out[b] = o.transpose(0, 1)
    return out
