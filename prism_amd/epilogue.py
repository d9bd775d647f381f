"""Drop-ins for the elementwise steps around Prism's paged attention, over the gfx950 kernels.

Each decoder layer of Prism's executor (engine/executor.py:104-127, :140-160, :250-275) runs:

    hidden = fused_rms_norm(hidden, input_ln_w)                     -> rms_norm
    qkv = F.linear(hidden, qkv_w, qkv_b)
    q, k, v = split(qkv); [q, k = fused_rms_norm(q | k, q/k_norm_w)] ; q, k = rope(q | k)
                                                                  -> rope_qk (+ the paged append)
    attn = flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, ...)
    hidden = residual + F.linear(attn, o_w); fused_rms_norm(hidden)  -> rms_norm(..., residual=)
    F.silu(gu[..., :m]) * gu[..., m:]                               -> silu_mul

The GEMMs stay with torch/hipBLASLt; these functions replace the eager elementwise chains in
between (about six launches per layer for the QKV split and rotary alone).  Results follow the
reference's bf16 rounding points; see include/prism_kv.h for the exact contract of each kernel.
Every call is asynchronous on the current stream and has no CPU fallback.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import _BF16, _require_gpu, _stream_ptr, status_tensor


def rope_tables(head_dim: int, n_pos: int, theta: float = 10000.0,
                device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin tables [n_pos, head_dim] bf16, built exactly as engine/executor.py:45-57 builds
    its [1, max_pos, 1, head_dim] tables (fp32 inv_freq and angles, bf16 cos / sin of the half
    dimension repeated for both halves), for any n_pos: the reference caps max_pos at 4096."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    t = torch.arange(n_pos, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    cos = freqs.cos().to(torch.bfloat16)
    sin = freqs.sin().to(torch.bfloat16)
    return torch.cat([cos, cos], dim=-1).contiguous(), torch.cat([sin, sin], dim=-1).contiguous()


def _bf16_rows(t: torch.Tensor, name: str) -> None:
    _require_gpu(t, name)
    if t.dtype != _BF16:
        raise RuntimeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.stride(-1) != 1:
        raise RuntimeError(f"{name} must be contiguous in its last dimension")


def rope_qk(qkv: torch.Tensor, positions: torch.Tensor | int, cos: torch.Tensor, sin: torch.Tensor,
            n_heads: int, n_kv: int, *, q_norm_w: torch.Tensor | None = None,
            k_norm_w: torch.Tensor | None = None, eps: float = 1e-6, return_k: bool = True,
            k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
            block_table: torch.Tensor | None = None, cache_seqlens: torch.Tensor | None = None,
            q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None,
            status: torch.Tensor | None = None):
    """QKV split + optional QK-norm + RoPE of Prism's executor for qkv [B, s, (n_heads + 2 n_kv) * hd].

    ``positions`` (int32 [B] or an int) is the position of token 0 of each sequence; token j uses
    row positions[b] + j of ``cos`` / ``sin`` ([n_pos, hd], see rope_tables).  Returns
    (q [B, s, n_heads, hd], k [B, s, n_kv, hd] or None) with the rotated heads.  With
    ``k_cache``/``v_cache``/``block_table``/``cache_seqlens`` the rotated k and the unrotated v are
    also appended at cache_seqlens[b] + j (the append half of flash_attn_with_kvcache), so the
    attention call can follow with k = v = None and cache_seqlens + s."""
    _bf16_rows(qkv, "qkv")
    if qkv.dim() != 3:
        raise RuntimeError(f"qkv must be [B, s, (n_heads + 2 n_kv) * head_dim], got {tuple(qkv.shape)}")
    batch, s_new, width = qkv.shape
    if width % (n_heads + 2 * n_kv):
        raise RuntimeError(f"qkv width {width} is not a multiple of n_heads + 2 n_kv = {n_heads + 2 * n_kv}")
    hd = width // (n_heads + 2 * n_kv)
    device = qkv.device
    for name, t in (("cos", cos), ("sin", sin)):
        _bf16_rows(t, name)
        if t.dim() != 2 or t.shape[1] != hd or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous [n_pos, {hd}] table")
    if cos.shape != sin.shape:
        raise RuntimeError("cos and sin tables differ in shape")
    for name, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        if t is not None:
            _bf16_rows(t, name)
            if t.numel() != hd or not t.is_contiguous():
                raise RuntimeError(f"{name} must be a contiguous [{hd}] vector")
    if isinstance(positions, int):
        positions = torch.full((batch,), positions, dtype=torch.int32, device=device)
    if positions.dtype != torch.int32 or positions.device != device or positions.numel() != batch:
        raise RuntimeError("positions must be int32 [B] on the qkv device")
    if q_out is None:
        q_out = torch.empty((batch, s_new, n_heads, hd), dtype=_BF16, device=device)
    if k_out is None and return_k:
        k_out = torch.empty((batch, s_new, n_kv, hd), dtype=_BF16, device=device)
    for name, t, nh in (("q_out", q_out, n_heads), ("k_out", k_out, n_kv)):
        if t is not None:
            _bf16_rows(t, name)
            if tuple(t.shape) != (batch, s_new, nh, hd):
                raise RuntimeError(f"{name} must be [{batch}, {s_new}, {nh}, {hd}]")
    append = k_cache is not None
    if append:
        if v_cache is None or block_table is None or cache_seqlens is None:
            raise RuntimeError("the append needs k_cache, v_cache, block_table and cache_seqlens")
        from .attention import _check_cache, _check_table
        num_pages, page_size, cache_kv, cache_hd = _check_cache(k_cache, v_cache)
        if (cache_kv, cache_hd) != (n_kv, hd):
            raise RuntimeError(f"cache heads {cache_kv} x {cache_hd} != n_kv {n_kv} x head_dim {hd}")
        _check_table(block_table, cache_seqlens, batch, device)
        cache_args = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), block_table.data_ptr(),
                      block_table.stride(0), cache_seqlens.data_ptr())
        page_args = (page_size, num_pages, block_table.shape[1])
    else:
        cache_args = (0, 0, 0, 0, 0, 0)
        page_args = (256, 1, 1)
    st = status if status is not None else status_tensor(device)
    lib = _lib.load()
    rc = lib.pkv_rope_qk(
        qkv.data_ptr(), qkv.stride(0), qkv.stride(1), positions.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        q_norm_w.data_ptr() if q_norm_w is not None else 0, k_norm_w.data_ptr() if k_norm_w is not None else 0,
        float(eps),
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1), q_out.stride(2),
        k_out.data_ptr() if k_out is not None else 0,
        *((k_out.stride(0), k_out.stride(1), k_out.stride(2)) if k_out is not None else (0, 0, 0)),
        *cache_args, batch, s_new, n_heads, n_kv, hd, *page_args, st.data_ptr(), _stream_ptr(device))
    _lib.check(rc, "pkv_rope_qk")
    return q_out, k_out


def _rows2d(t: torch.Tensor, name: str) -> torch.Tensor:
    _bf16_rows(t, name)
    t2 = t.reshape(-1, t.shape[-1])
    if t2.data_ptr() != t.data_ptr() or (t2.shape[0] > 1 and t2.stride(0) < t2.shape[1]):
        raise RuntimeError(f"{name} must flatten to rows without a copy")
    return t2


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, *,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
             h_out: torch.Tensor | None = None):
    """engine/fused_kernels.py:fused_rms_norm(x, weight, eps) over the last dimension.  With
    ``residual``, normalises h = x + residual (bf16) instead and returns (out, h): the executor's
    ``hidden = residual + ...; fused_rms_norm(hidden)`` in one pass."""
    x2 = _rows2d(x, "x")
    hidden = x2.shape[1]
    _bf16_rows(weight, "weight")
    if weight.numel() != hidden or not weight.is_contiguous():
        raise RuntimeError(f"weight must be a contiguous [{hidden}] vector")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    o2 = _rows2d(out, "out")
    r2 = h2 = None
    if residual is not None:
        if residual.shape != x.shape:
            raise RuntimeError("residual must have x's shape")
        r2 = _rows2d(residual, "residual")
        if h_out is None:
            h_out = torch.empty_like(x, memory_format=torch.contiguous_format)
        h2 = _rows2d(h_out, "h_out")
    elif h_out is not None:
        raise RuntimeError("h_out needs a residual")
    if o2.shape != x2.shape:
        raise RuntimeError("out must have x's shape")
    lib = _lib.load()
    rc = lib.pkv_rms_norm(x2.data_ptr(), x2.stride(0), r2.data_ptr() if r2 is not None else 0,
                          r2.stride(0) if r2 is not None else 0, h2.data_ptr() if h2 is not None else 0,
                          h2.stride(0) if h2 is not None else 0, weight.data_ptr(), o2.data_ptr(), o2.stride(0),
                          x2.shape[0], hidden, float(eps), _stream_ptr(x.device))
    _lib.check(rc, "pkv_rms_norm")
    return out if residual is None else (out, h_out)


def fused_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Same name and arguments as engine/fused_kernels.py:fused_rms_norm."""
    return rms_norm(x, weight, eps)


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """F.silu(gate) * up on bf16 rows (engine/executor.py:127, with gate = gu[..., :m] and
    up = gu[..., m:] views of the fused gate/up projection)."""
    if gate.shape != up.shape:
        raise RuntimeError("gate and up must have the same shape")
    m = gate.shape[-1]
    for name, t in (("gate", gate), ("up", up)):
        _bf16_rows(t, name)
    rows = gate.numel() // m if m else 0
    g2, u2 = gate.reshape(-1, m), up.reshape(-1, m)
    if g2.data_ptr() != gate.data_ptr() or u2.data_ptr() != up.data_ptr():
        raise RuntimeError("gate/up must flatten to rows without a copy")
    if out is None:
        out = torch.empty(gate.shape, dtype=_BF16, device=gate.device)
    o2 = _rows2d(out, "out")
    lib = _lib.load()
    rc = lib.pkv_silu_mul(g2.data_ptr(), g2.stride(0) if rows > 1 else m, u2.data_ptr(),
                          u2.stride(0) if rows > 1 else m, o2.data_ptr(), o2.stride(0) if rows > 1 else m,
                          rows, m, _stream_ptr(gate.device))
    _lib.check(rc, "pkv_silu_mul")
    return out


def fused_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Same name and arguments as engine/fused_kernels.py:fused_silu_mul."""
    return silu_mul(gate, up)
