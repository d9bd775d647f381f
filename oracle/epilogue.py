"""ORACLE (test infrastructure): CPU restatement of the elementwise steps around Prism's paged
attention -- rotary tables, QKV split + QK-norm + RoPE, RMSNorm (with the residual add before it)
and SiLU(gate) * up.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.

Followed from the reference:
  rope_tables          engine/executor.py:45-57 (fp32 inv_freq and angles, bf16 cos / sin of the
                       half dimension, concatenated for both halves; the reference caps positions
                       at 4096, the restatement takes any count).
  rope_bf16            engine/executor.py:18-21 (_rotate_half) and :116-118 / :146-147
                       (q * cos + _rotate_half(q) * sin on bf16 tensors: each torch op computes in
                       fp32 and rounds to bf16).
  rope_bf16_loop       the same expression element by element with explicit rounding (an
                       independent restatement used to pin rope_bf16).
  rms_norm_f64         engine/fused_kernels.py:31-65 (x * rsqrt(mean(x^2) + eps) * w over the last
                       dimension), in fp64; with a residual, h = bf16(x + residual) first
                       (engine/executor.py:121-122, :127-131).
  silu_mul_ref         engine/executor.py:127 (F.silu(gate) * up on bf16: silu rounded to bf16,
                       then the product rounded), silu in fp64.
  qkv_split_rope       engine/executor.py:108-118: the split of the fused QKV row, optional per-head
                       QK-norm (rounded to bf16), then RoPE.
"""
from __future__ import annotations

import numpy as np
import torch


def rope_tables(head_dim: int, n_pos: int, theta: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    """[n_pos, head_dim] bf16 cos / sin tables by the engine/executor.py:47-57 formula (CPU)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(n_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos = freqs.cos().to(torch.bfloat16)
    sin = freqs.sin().to(torch.bfloat16)
    return torch.cat([cos, cos], dim=-1), torch.cat([sin, sin], dim=-1)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """engine/executor.py:18-21."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def rope_bf16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin on bf16 CPU tensors (x [..., hd]; cos/sin broadcastable)."""
    assert x.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16
    return (x * cos) + (rotate_half(x) * sin)


def _bf16(v: float) -> float:
    return float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16).to(torch.float32))


def rope_bf16_loop(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """rope_bf16 for one vector, element by element: out[i] = bf16(bf16(x[i] cos[i]) +
    bf16(r[i] sin[i])) with r = (-x[h:], x[:h]); x, cos, sin are fp32 values of bf16 numbers."""
    hd = len(x)
    h = hd // 2
    out = np.zeros(hd, dtype=np.float64)
    for i in range(hd):
        r = -x[i + h] if i < h else x[i - h]
        a = _bf16(float(np.float32(x[i]) * np.float32(cos[i])))
        b = _bf16(float(np.float32(r) * np.float32(sin[i])))
        out[i] = _bf16(float(np.float32(a) + np.float32(b)))
    return out


def rope_f64(x: np.ndarray, pos: np.ndarray, head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """The rotation itself in fp64: pair (x[i], x[i + hd/2]) is the complex number x[i] + i x[i+hd/2]
    multiplied by exp(i pos theta^(-2i/hd)).  x [..., hd], pos broadcast over the leading dims."""
    h = head_dim // 2
    inv = theta ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.asarray(pos, dtype=np.float64)[..., None] * inv
    z = (x[..., :h] + 1j * x[..., h:]) * np.exp(1j * ang)
    return np.concatenate([z.real, z.imag], axis=-1)


def rms_norm_f64(x: np.ndarray, w: np.ndarray, eps: float, residual: np.ndarray | None = None):
    """RMSNorm over the last axis in fp64; x, w, residual hold bf16 values.  Returns (out, h) with
    h = bf16(x + residual) when a residual is given (else h = x); out is not rounded."""
    h = x.astype(np.float64)
    if residual is not None:
        h = round_bf16(h + residual.astype(np.float64))
    ms = np.mean(h * h, axis=-1, keepdims=True)
    return h / np.sqrt(ms + eps) * w.astype(np.float64), h


def silu_mul_ref(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """bf16(bf16(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in fp64; inputs hold bf16 values."""
    g = gate.astype(np.float64)
    s = round_bf16(g / (1.0 + np.exp(-g)))
    return round_bf16(s * up.astype(np.float64))


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp64 -> (fp32 ->) bf16, round to nearest even -> fp64 values (torch's conversion)."""
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def qkv_split_rope(qkv: torch.Tensor, positions: np.ndarray, cos: torch.Tensor, sin: torch.Tensor,
                   n_heads: int, n_kv: int, q_norm_w: torch.Tensor | None = None,
                   k_norm_w: torch.Tensor | None = None, eps: float = 1e-6):
    """engine/executor.py:108-118 on CPU bf16 tensors: qkv [B, s, (nh + 2 nkv) hd] -> (q, k, v)
    [B, s, heads, hd] bf16 with RoPE at positions[b] + j (and QK-norm when weights are given)."""
    B, s, width = qkv.shape
    hd = width // (n_heads + 2 * n_kv)
    qs, kvs = n_heads * hd, n_kv * hd
    q = qkv[:, :, :qs].reshape(B, s, n_heads, hd)
    k = qkv[:, :, qs:qs + kvs].reshape(B, s, n_kv, hd)
    v = qkv[:, :, qs + kvs:].reshape(B, s, n_kv, hd)
    if q_norm_w is not None:
        q = _norm_bf16(q, q_norm_w, eps)
    if k_norm_w is not None:
        k = _norm_bf16(k, k_norm_w, eps)
    pos = torch.as_tensor(np.asarray(positions, dtype=np.int64))[:, None] + torch.arange(s)[None, :]
    c = cos[pos][:, :, None, :]  # [B, s, 1, hd]
    sn = sin[pos][:, :, None, :]
    return rope_bf16(q, c, sn), rope_bf16(k, c, sn), v


def _norm_bf16(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    out, _ = rms_norm_f64(x.float().numpy(), w.float().numpy(), eps)
    return torch.from_numpy(out.astype(np.float32)).to(torch.bfloat16)


def cpu_epilogue_ref(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     n_heads: int, n_kv: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's eager torch path on CPU (timed as the CPU baseline): split, then
    q * cos + rotate_half(q) * sin for q and k."""
    B, s, width = qkv.shape
    hd = width // (n_heads + 2 * n_kv)
    qs, kvs = n_heads * hd, n_kv * hd
    q = qkv[:, :, :qs].view(B, s, n_heads, hd)
    k = qkv[:, :, qs:qs + kvs].view(B, s, n_kv, hd)
    pos = positions.long()[:, None] + torch.arange(s)[None, :]
    c = cos[pos][:, :, None, :]
    sn = sin[pos][:, :, None, :]
    return (q * c) + (rotate_half(q) * sn), (k * c) + (rotate_half(k) * sn)


__all__ = ["rope_tables", "rotate_half", "rope_bf16", "rope_bf16_loop", "rope_f64", "rms_norm_f64", "silu_mul_ref",
           "round_bf16", "qkv_split_rope", "cpu_epilogue_ref"]
