"""GPU parity of the pre-attention epilogue (QKV split + QK-norm + RoPE + paged append), RMSNorm and
SiLU-mul against oracle/epilogue.py, through the C ABI.  RoPE and the appended cache rows are
bit-exact (the reference's bf16 expression is exact in fp32 up to its roundings); QK-norm, RMSNorm
and SiLU-mul agree to one bf16 unit (rsqrt / exp differ in the last fp32 bits)."""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import epilogue as ep
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close, make_paged_case

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(device)


def _ulp_close(got: torch.Tensor, ref: np.ndarray, what: str, ulps: float = 1.0):
    """|got - ref| <= ulps bf16 units of ref (2^-8 relative, with a floor for tiny values)."""
    g = got.float().cpu().numpy().astype(np.float64)
    tol = ulps * np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7 + 1e-30
    bad = np.abs(g - ref) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond {ulps} bf16 unit(s), max diff {np.max(np.abs(g - ref)):.3g}"


ROPE_CASES = [
    # (batch, s_new, n_heads, n_kv, head_dim, qk_norm)
    (32, 1, 28, 4, 128, False),   # 7B decode
    (3, 37, 40, 8, 128, False),   # 14B chunk
    (4, 5, 14, 2, 64, False),     # 0.5B verify
    (2, 9, 16, 8, 128, True),     # QK-norm (Qwen3-style)
    (1, 3, 14, 2, 64, True),
]


@pytest.mark.parametrize("case", ROPE_CASES, ids=[f"r{i}" for i in range(len(ROPE_CASES))])
def test_rope_qk_matches_reference_expression(gpu, case):
    B, s, nh, nkv, hd, qkn = case
    print(f"rope case {case}", flush=True)
    qkv = _rand((B, s, (nh + 2 * nkv) * hd), 11 + B, 2.0)
    pos = np.array([(97 * b + 5) % 5000 for b in range(B)], dtype=np.int32)
    cos, sin = ep.rope_tables(hd, 5100)
    qw = _rand((hd,), 1) if qkn else None
    kw = _rand((hd,), 2) if qkn else None
    q_ref, k_ref, _ = ep.qkv_split_rope(qkv, pos, cos, sin, nh, nkv, qw, kw)
    dcos, dsin = cos.to(gpu), sin.to(gpu)
    q, k = prism_amd.rope_qk(qkv.to(gpu), torch.from_numpy(pos).to(gpu), dcos, dsin, nh, nkv,
                             q_norm_w=qw.to(gpu) if qkn else None, k_norm_w=kw.to(gpu) if qkn else None)
    torch.cuda.synchronize()
    if not qkn:
        assert torch.equal(q.cpu(), q_ref), "q not bit-exact"
        assert torch.equal(k.cpu(), k_ref), "k not bit-exact"
    else:
        # one-unit differences of the normalised inputs can move the rotated value by a little more
        _ulp_close(q, q_ref.double().numpy(), "q (QK-norm)", 3.0)
        _ulp_close(k, k_ref.double().numpy(), "k (QK-norm)", 3.0)


def test_rope_qk_appends_into_pages_then_attends(gpu):
    # the fused epilogue's append + attention without k/v equals attention with the reference path
    B, s, nh, nkv, hd, P = 3, 4, 28, 4, 128, 256
    ctx = [0, 300, 1023]
    cpu, dev = make_paged_case(gpu, batch=B, ctx=ctx, page_size=P, n_kv=nkv, n_heads=nh, head_dim=hd, s_q=s,
                               seed=5)
    qkv = _rand((B, s, (nh + 2 * nkv) * hd), 21, 1.0)
    pos = np.array(ctx, dtype=np.int32)
    cos, sin = ep.rope_tables(hd, 2048)
    q_ref, k_ref, v_ref = ep.qkv_split_rope(qkv, pos, cos, sin, nh, nkv)
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(q_ref, cpu["k_cache"], cpu["v_cache"], k_ref, v_ref,
                                                 cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                                 causal=True)
    dcos, dsin = cos.to(gpu), sin.to(gpu)
    sl = dev["cache_seqlens"]
    q, _ = prism_amd.rope_qk(qkv.to(gpu), sl, dcos, dsin, nh, nkv, return_k=False, k_cache=dev["k_cache"],
                             v_cache=dev["v_cache"], block_table=dev["block_table"], cache_seqlens=sl)
    out = prism_amd.flash_attn_with_kvcache(q, dev["k_cache"], dev["v_cache"], cache_seqlens=sl + s,
                                            block_table=dev["block_table"], causal=True)
    torch.cuda.synchronize()
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "appended K not bit-exact"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "appended V not bit-exact"
    assert_attn_close(out, ref, "rope+append+attention")
    assert prism_amd.read_status(gpu) == 0


ROPE_ATTN_CASES = [
    # (batch, ctx, page, n_kv, n_heads, hd, s_q, grid, two_pass)
    (32, [(i * 397) % 3000 for i in range(32)], 256, 4, 28, 128, 1, 0, None),   # 7B decode
    (32, [(i * 397) % 3000 for i in range(32)], 256, 4, 28, 128, 1, 9, False),  # in-launch merge
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 8, 40, 128, 2, 0, None),          # 14B, 2 new rows, R = 10
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 2, 14, 64, 1, 7, None),           # 0.5B (hd 64, two phases)
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 1, 7, 128, 1, 5, None),           # 7B on 4 TP ranks
    (40, [(i * 37) % 300 for i in range(40)], 64, 2, 14, 128, 1, 3, None),     # 64-token pages, 2 phases
    (3, [0, 255, 256], 256, 4, 28, 128, 1, 0, None),                           # page edges, empty cache
    (70, [(i * 53) % 900 for i in range(70)], 256, 4, 28, 128, 1, 0, None),    # over 64 sequences
    (70, [(i * 53) % 900 for i in range(70)], 256, 2, 14, 64, 1, 0, None),
]


@pytest.mark.parametrize("case", ROPE_ATTN_CASES, ids=[f"r{i}" for i in range(len(ROPE_ATTN_CASES))])
def test_rope_decode_attention_matches_the_reference_step(gpu, case):
    # one launch for the reference's q / k rotation, append and paged attention: the cache rows
    # bit-identical to the reference expression's (and so to rope_qk's), the output within the
    # attention tolerance of the fp64 oracle and of the two-launch path (rope_qk + attention)
    B, ctx, P, nkv, nh, hd, s, grid, two_pass = case
    print(f"rope_decode_attention B={B} P={P} kv={nkv} h={nh} hd={hd} s={s} grid={grid}", flush=True)
    cpu, dev = make_paged_case(gpu, batch=B, ctx=ctx, page_size=P, n_kv=nkv, n_heads=nh, head_dim=hd, s_q=s,
                               seed=B + nkv)
    qkv = _rand((B, s, (nh + 2 * nkv) * hd), 31 + nkv, 1.0)
    pos = np.array(ctx, dtype=np.int32)
    cos, sin = ep.rope_tables(hd, 8192)
    q_ref, k_ref, v_ref = ep.qkv_split_rope(qkv, pos, cos, sin, nh, nkv)
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(q_ref, cpu["k_cache"], cpu["v_cache"], k_ref, v_ref,
                                                 cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                                 causal=True)
    dcos, dsin = cos.to(gpu), sin.to(gpu)
    kc0, vc0 = dev["k_cache"].clone(), dev["v_cache"].clone()
    out = torch.full((B, s, nh, hd), float("nan"), dtype=torch.bfloat16, device=gpu)
    prism_amd.rope_decode_attention(qkv.to(gpu), dev["k_cache"], dev["v_cache"], dcos, dsin,
                                    cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                    n_heads=nh, n_kv=nkv, grid=grid, two_pass=two_pass, out=out)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == 0
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "appended (rotated) K not bit-exact"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "appended V not bit-exact"
    assert_attn_close(out, ref, f"rope_decode_attention {case[:1] + case[2:]}")
    sl = dev["cache_seqlens"]
    q2, _ = prism_amd.rope_qk(qkv.to(gpu), sl, dcos, dsin, nh, nkv, return_k=False, k_cache=kc0, v_cache=vc0,
                              block_table=dev["block_table"], cache_seqlens=sl)
    two = prism_amd.flash_attn_with_kvcache(q2, kc0, vc0, cache_seqlens=sl + s, block_table=dev["block_table"],
                                            causal=True)
    torch.cuda.synchronize()
    assert torch.equal(kc0, dev["k_cache"]) and torch.equal(vc0, dev["v_cache"]), "caches differ from rope_qk's"
    assert float((two.float() - out.float()).abs().max()) <= 1e-2


def test_rope_decode_attention_flags_positions_and_rejects_other_shapes(gpu):
    B, nh, nkv, hd, P = 2, 28, 4, 128, 256
    cpu, dev = make_paged_case(gpu, batch=B, ctx=[10, 40], page_size=P, n_kv=nkv, n_heads=nh, head_dim=hd, s_q=1,
                               seed=3)
    qkv = _rand((B, 1, (nh + 2 * nkv) * hd), 4).to(gpu)
    cos, sin = prism_amd.rope_tables(hd, 32, device=gpu)   # position 40 is past the table
    prism_amd.rope_decode_attention(qkv, dev["k_cache"], dev["v_cache"], cos, sin,
                                    cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                    n_heads=nh, n_kv=nkv)
    torch.cuda.synchronize()
    assert prism_amd.read_status(gpu) == prism_amd._lib.PKV_STATUS_BAD_POSITION
    # verify rows (R + 2 s_q > 16) are not fused: the call is refused before anything runs
    cpu, dev = make_paged_case(gpu, batch=B, ctx=[10, 40], page_size=P, n_kv=nkv, n_heads=nh, head_dim=hd, s_q=3,
                               seed=3)
    with pytest.raises(prism_amd._lib.PrismKVError, match="fused into the balanced decode kernel"):
        prism_amd.rope_decode_attention(_rand((B, 3, (nh + 2 * nkv) * hd), 5).to(gpu), dev["k_cache"],
                                        dev["v_cache"], cos, sin, cache_seqlens=dev["cache_seqlens"],
                                        block_table=dev["block_table"], n_heads=nh, n_kv=nkv)


def test_device_rope_tables_match_the_cpu_formula(gpu):
    # the reference builds its tables on the device (engine/executor.py:49-55); device and host
    # cos / sin may differ in the last fp32 bit, so bf16 entries agree to one unit
    for hd in (64, 128):
        cos, sin = ep.rope_tables(hd, 6000)
        dcos, dsin = prism_amd.rope_tables(hd, 6000, device=gpu)
        for name, a, b in (("cos", dcos, cos), ("sin", dsin, sin)):
            diff = (a.float().cpu() - b.float()).abs()
            assert float(diff.max()) <= 2.0 ** -8 * 1.01, f"{name} hd={hd}: max diff {float(diff.max())}"
            assert float((diff == 0).float().mean()) > 0.99, f"{name} hd={hd}: too many differing entries"


def test_rope_qk_flags_positions_past_the_table(gpu):
    qkv = _rand((2, 2, 8 * 64), 3).to(gpu)
    cos, sin = prism_amd.rope_tables(64, 16, device=gpu)
    prism_amd.rope_qk(qkv, torch.tensor([3, 15], dtype=torch.int32, device=gpu), cos, sin, 4, 2)
    assert prism_amd.read_status(gpu) == 2
    with pytest.raises(RuntimeError):
        prism_amd.rope_qk(qkv[..., :-8], 0, cos, sin, 4, 2)


@pytest.mark.parametrize("hidden,rows,resid", [(3584, 33, False), (5120, 7, True), (896, 1, True), (8192, 3, False)])
def test_rms_norm_matches_fp64(gpu, hidden, rows, resid):
    x = _rand((rows, hidden), hidden + rows, 3.0)
    w = _rand((hidden,), 4)
    r = _rand((rows, hidden), 5) if resid else None
    ref, h_ref = ep.rms_norm_f64(x.float().numpy(), w.float().numpy(), 1e-6,
                                 r.float().numpy() if resid else None)
    res = prism_amd.rms_norm(x.to(gpu), w.to(gpu), 1e-6, residual=r.to(gpu) if resid else None)
    torch.cuda.synchronize()
    out = res[0] if resid else res
    _ulp_close(out, ep.round_bf16(ref), f"rms_norm {hidden}x{rows}", 1.0)
    if resid:
        assert np.array_equal(res[1].float().cpu().numpy(), h_ref), "residual sum not bit-exact"


def test_silu_mul_matches_reference(gpu):
    rows, m = 37, 18944
    gu = _rand((rows, 2 * m), 9, 3.0)
    ref = ep.silu_mul_ref(gu[:, :m].float().numpy(), gu[:, m:].float().numpy())
    d = gu.to(gpu)
    out = prism_amd.silu_mul(d[:, :m], d[:, m:])
    torch.cuda.synchronize()
    _ulp_close(out, ref, "silu_mul", 1.0)
    exact = np.mean(out.float().cpu().numpy() == ref)
    assert exact > 0.99, f"only {exact:.4f} of outputs bit-exact"
