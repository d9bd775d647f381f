"""CPU pins of oracle/epilogue.py (rotary tables and RoPE, RMSNorm, SiLU-mul), each checked against
an independent formulation or a closed form, not against a retyped copy of itself."""
import math

import numpy as np
import torch

from oracle import epilogue as ep


def _bf16_rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def test_rope_tables_match_cos_sin():
    cos, sin = ep.rope_tables(128, 5000)
    assert cos.shape == (5000, 128) and cos.dtype == torch.bfloat16
    assert torch.equal(cos[:, :64], cos[:, 64:]) and torch.equal(sin[:, :64], sin[:, 64:])
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    for pos, i in [(1, 0), (7, 3), (4095, 10), (4999, 63)]:
        ang = pos * 10000.0 ** (-2 * i / 128)
        assert abs(float(cos[pos, i]) - math.cos(ang)) <= 2 ** -8 * 1.01
        assert abs(float(sin[pos, i]) - math.sin(ang)) <= 2 ** -8 * 1.01


def test_rope_bf16_matches_elementwise_restatement():
    cos, sin = ep.rope_tables(128, 300)
    x = _bf16_rand((6, 128), 1, 3.0)
    pos = [0, 1, 17, 100, 255, 299]
    out = ep.rope_bf16(x, cos[pos], sin[pos]).float().numpy()
    for r, p in enumerate(pos):
        ref = ep.rope_bf16_loop(x[r].float().numpy(), cos[p].float().numpy(), sin[p].float().numpy())
        assert np.array_equal(out[r], ref), r


def test_rope_position_zero_is_identity_and_rotation_matches_fp64():
    cos, sin = ep.rope_tables(64, 2048)
    x = _bf16_rand((32, 64), 2)
    out0 = ep.rope_bf16(x, cos[0], sin[0])
    assert torch.equal(out0, x)
    pos = np.arange(0, 2048, 64)
    out = ep.rope_bf16(x, cos[pos], sin[pos]).double().numpy()
    ref = ep.rope_f64(x.double().numpy(), pos, 64)
    # three bf16 roundings per element plus the tables' own bf16 rounding
    assert np.max(np.abs(out - ref)) <= 0.05 * np.max(np.abs(ref))
    # a rotation keeps each (x_i, x_{i+h}) pair's length
    h = 32
    n_out = np.hypot(out[:, :h], out[:, h:])
    n_in = np.hypot(x.double().numpy()[:, :h], x.double().numpy()[:, h:])
    assert np.max(np.abs(n_out - n_in)) <= 0.02 * np.max(n_in)


def test_rms_norm_against_torch_and_closed_forms():
    x = _bf16_rand((5, 3584), 3, 2.0).float().numpy()
    w = _bf16_rand((3584,), 4).float().numpy()
    out, h = ep.rms_norm_f64(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (3584,), torch.from_numpy(w).double(), 1e-6)
    assert np.allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)
    c = np.full((1, 64), 0.75)
    oc, _ = ep.rms_norm_f64(c, np.ones(64), 0.0)
    assert np.allclose(oc, 1.0)
    o2, _ = ep.rms_norm_f64(4.0 * x, w, 0.0)
    o1, _ = ep.rms_norm_f64(x, w, 0.0)
    assert np.allclose(o1, o2, rtol=1e-12)
    r = _bf16_rand((5, 3584), 5).float().numpy()
    _, hr = ep.rms_norm_f64(x, w, 1e-6, residual=r)
    assert np.array_equal(hr, ep.round_bf16(x.astype(np.float64) + r))


def test_silu_mul_against_torch_and_limits():
    g = _bf16_rand((4, 1024), 6, 4.0).float().numpy()
    u = _bf16_rand((4, 1024), 7).float().numpy()
    out = ep.silu_mul_ref(g, u)
    s = torch.nn.functional.silu(torch.from_numpy(g).double()).float().to(torch.bfloat16).double()
    ref = (s * torch.from_numpy(u).double()).float().to(torch.bfloat16).double().numpy()
    assert np.array_equal(out, ref)
    z = ep.silu_mul_ref(np.array([0.0, 60.0, -60.0]), np.array([1.0, 1.0, 1.0]))
    assert z[0] == 0.0 and z[1] == 60.0 and abs(z[2]) < 1e-20


def test_qkv_split_rope_layout_and_qk_norm():
    nh, nkv, hd = 4, 2, 64
    qkv = _bf16_rand((2, 3, (nh + 2 * nkv) * hd), 8)
    cos, sin = ep.rope_tables(hd, 64)
    q, k, v = ep.qkv_split_rope(qkv, np.array([0, 10]), cos, sin, nh, nkv)
    assert torch.equal(v, qkv[:, :, (nh + nkv) * hd:].reshape(2, 3, nkv, hd))
    # sequence 0, token 0 is at position 0: q and k unchanged
    assert torch.equal(q[0, 0], qkv[0, 0, :nh * hd].reshape(nh, hd))
    assert torch.equal(k[0, 0], qkv[0, 0, nh * hd:(nh + nkv) * hd].reshape(nkv, hd))
    # token 2 of sequence 1 is at position 12
    exp = ep.rope_bf16(qkv[1, 2, :hd], cos[12], sin[12])
    assert torch.equal(q[1, 2, 0], exp)
    wq = torch.ones(hd, dtype=torch.bfloat16)
    qn, _, _ = ep.qkv_split_rope(qkv, np.array([0, 0]), cos, sin, nh, nkv, q_norm_w=wq)
    rms = qn[0, 0].float().pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=0.02)
