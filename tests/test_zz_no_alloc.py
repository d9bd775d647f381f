"""pkv_decode_attn_noalloc, the allocation-free variant of pkv_decode_attn, through the C ABI.

The variant takes no workspace: its split-K counters and partials live in the library's static
device array.  On the same inputs it must give pkv_decode_attn's results bit for bit (output and
appended cache rows), on two calls in a row, the second with a smaller input: the array keeps the
previous call's contents, so a stale partial or a counter left non-zero would show.  Covered: the
balanced kernel for decode (R = 7) and verify (R = 35), with its two-pass and in-launch merges,
and the per-head kernel with several splits per sequence (its in-launch merge counts arrivals in
the array).  A call needing more scratch than the array holds is rejected before anything runs.
Through the drop-in, a forked-branch table that would send the default call to cascade attention
(which needs the module's workspace) runs the allocation-free path and allocates nothing.  A
fresh process whose first allocation-free call is made under graph capture (the scratch lookup and
its counter clearing then happen inside the capture) replays to the eager call's output.
"""

import pytest
import torch

from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close, make_paged_case
from prism_amd import _lib

pytestmark = pytest.mark.gpu


def _common(d, out):
    q, k, v, kc, vc, bt, sl = (d[n] for n in ("q", "k", "v", "k_cache", "v_cache", "block_table", "cache_seqlens"))
    B, s_q, nh, hd = q.shape
    num_pages, P, n_kv, _ = kc.shape
    head = (q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            kc.data_ptr(), vc.data_ptr(), kc.stride(0),
            bt.data_ptr(), bt.stride(0), sl.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2))
    sizes = (B, s_q, nh, n_kv, hd, P, num_pages, bt.shape[1])
    return head, sizes


def _run(lib, d, *, noalloc, flags=0, split=0, status):
    out = torch.full_like(d["q"], float("nan"))
    head, sizes = _common(d, out)
    hd = sizes[4]
    stream = torch.cuda.current_stream().cuda_stream
    tail = (1, 1.0 / hd ** 0.5, split, flags, status.data_ptr(), stream)
    if noalloc:
        rc = lib.pkv_decode_attn_noalloc(*head, *sizes, *tail)
        _lib.check(rc, "pkv_decode_attn_noalloc")
    else:
        nbytes = lib.pkv_decode_workspace_bytes(sizes[0], sizes[1], sizes[2], sizes[3], sizes[4], sizes[5],
                                                sizes[7], split)
        ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=out.device)
        rc = lib.pkv_decode_attn(*head, ws.data_ptr(), ws.numel(), *sizes, *tail)
        _lib.check(rc, "pkv_decode_attn")
    torch.cuda.synchronize()
    return out


CASES = [
    # (name, first call, second (smaller) call, flags, split_tokens); calls are
    # (batch, ctx, page, n_kv, n_heads, head_dim, s_q)
    ("balanced decode", (32, [(i * 911) % 5000 + 16 for i in range(32)], 256, 4, 28, 128, 1),
     (5, [40, 3000, 1, 700, 257], 256, 4, 28, 128, 1), 0, 0),
    ("balanced verify", (64, [2027 + (i * 97) % 1024 for i in range(64)], 256, 4, 28, 128, 5),
     (3, [517, 2, 90], 256, 4, 28, 128, 5), 0, 0),
    ("balanced in-launch merge", (32, [(i * 577) % 4000 + 1 for i in range(32)], 256, 4, 28, 128, 1),
     (4, [3000, 17, 4100, 800], 256, 4, 28, 128, 1), _lib.PKV_DECODE_FUSED_MERGE, 0),
    ("per-head kernel, in-launch split merge", (6, [3000, 17, 4100, 800, 1, 2500], 256, 2, 14, 64, 1),
     (2, [1500, 600], 256, 2, 14, 64, 1), 0, 256),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0].replace(" ", "_").replace(",", "") for c in CASES])
def test_noalloc_matches_workspace_entry_point(gpu, case):
    name, first, second, flags, split = case
    lib = _lib.load()
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    for i, (B, ctx, P, n_kv, nh, hd, s_q) in enumerate((first, second)):
        print(f"noalloc {name} call {i}: B={B} P={P} kv={n_kv} h={nh} hd={hd} s_q={s_q} flags={flags} "
              f"split={split}", flush=True)
        cpu, d1 = make_paged_case(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd,
                                  s_q=s_q, seed=17 + i)
        d2 = {n: t.clone() for n, t in d1.items()}
        ref = _run(lib, d1, noalloc=False, flags=flags, split=split, status=status)
        got = _run(lib, d2, noalloc=True, flags=flags, split=split, status=status)
        assert int(status.item()) == 0
        assert torch.equal(got, ref), f"{name} call {i}: output differs from pkv_decode_attn"
        assert torch.equal(d2["k_cache"], d1["k_cache"]) and torch.equal(d2["v_cache"], d1["v_cache"]), \
            f"{name} call {i}: appended cache differs from pkv_decode_attn"
        exp, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                                   cache_seqlens=cpu["cache_seqlens"],
                                                   block_table=cpu["block_table"], causal=True)
        assert_attn_close(got, exp, f"noalloc {name} call {i}")


def test_noalloc_rejects_a_call_beyond_its_scratch(gpu):
    # the per-head kernel with 256 sequences x 8 KV heads x 32 splits x 40 rows needs ~1.4 GB of
    # partials: rejected with PKV_ENOSPC and a message, nothing launched (out stays NaN).  Every
    # sequence is empty and every table entry is page 0, so even a launch would stay in bounds.
    lib = _lib.load()
    B, s_q, nh, n_kv, hd, P, max_blocks = 256, 8, 40, 8, 128, 256, 64
    q = torch.randn(B, s_q, nh, hd, device=gpu).to(torch.bfloat16)
    kc = torch.zeros(1, P, n_kv, hd, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    d = dict(q=q, k=torch.zeros(B, s_q, n_kv, hd, dtype=torch.bfloat16, device=gpu),
             v=torch.zeros(B, s_q, n_kv, hd, dtype=torch.bfloat16, device=gpu), k_cache=kc, v_cache=vc,
             block_table=torch.zeros(B, max_blocks, dtype=torch.int32, device=gpu),
             cache_seqlens=torch.zeros(B, dtype=torch.int32, device=gpu))
    out = torch.full_like(q, float("nan"))
    head, sizes = _common(d, out)
    need = lib.pkv_decode_workspace_bytes(B, s_q, nh, n_kv, hd, P, max_blocks, 512)
    assert need > 48 << 20
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    rc = lib.pkv_decode_attn_noalloc(*head, *sizes, 1, 1.0 / hd ** 0.5, 512, 0, status.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == _lib.PKV_ENOSPC
    msg = lib.pkv_last_error().decode()
    assert "static scratch" in msg and str(need) in msg, msg
    assert torch.isnan(out.float()).all()
    assert int(status.item()) == 0


def test_noalloc_never_takes_the_cascade(gpu):
    # a forked-branch verify batch whose table would send the default call to cascade attention
    # (which needs a workspace of the module's): with noalloc it runs the allocation-free decode
    # entry point, allocates nothing and matches the oracle
    import numpy as np

    import prism_amd
    from prism_amd import shared_prefix_of

    P, n_kv, hd, nh, s_q = 256, 4, 128, 28, 5
    kv = prism_amd.FlashAttnKVCache(1, n_kv, hd, 64, P, str(gpu))
    g = torch.Generator().manual_seed(11)
    kv.k_pool.copy_(torch.randn(kv.k_pool.shape, generator=g).to(torch.bfloat16))
    kv.v_pool.copy_(torch.randn(kv.v_pool.shape, generator=g).to(torch.bfloat16))
    kv.new_sequence(0)
    kv._ensure_capacity(0, 2400)
    kv.seq_len[0] = 2400
    ids = list(range(8))
    for sid in ids[1:]:
        kv.fork_sequence(0, sid)
    for sid in ids:
        grow = (sid * 53) % 300
        kv.prepare_append([sid], grow)
        kv.update_seqlens([sid], grow)
    bt, sl = kv.build_block_table(ids)
    assert shared_prefix_of(bt, sl, s_q=s_q, appends=False) >= prism_amd.attention.AUTO_CASCADE_MIN_TOKENS
    q = torch.randn(len(ids), s_q, nh, hd, generator=g).to(torch.bfloat16).to(gpu)
    out = torch.full_like(q, float("nan"))
    kw = dict(cache_seqlens=sl, block_table=bt, causal=True, noalloc=True, out=out)
    print(f"noalloc forked branches B={len(ids)} s_q={s_q}", flush=True)
    prism_amd.flash_attn_with_kvcache(q, kv.k_caches[0], kv.v_caches[0], **kw)  # first use: status words
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(gpu)
    out.fill_(float("nan"))
    prism_amd.flash_attn_with_kvcache(q, kv.k_caches[0], kv.v_caches[0], **kw)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(gpu) == before, "the noalloc call allocated device memory"
    ref, _, _ = pa.flash_attn_with_kvcache_ref(q.cpu(), kv.k_caches[0].cpu(), kv.v_caches[0].cpu(),
                                               cache_seqlens=sl.cpu(), block_table=bt.cpu(), causal=True)
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert_attn_close(out, ref, "noalloc forked branches")
    assert prism_amd.read_status(gpu) == 0


def test_noalloc_inside_a_captured_graph(gpu):
    # the drop-in's noalloc path captured on a fresh stream (nothing allocated during capture);
    # replays equal the eager call, with eager calls on the shared scratch between the replays
    import prism_amd

    cpu, d = make_paged_case(gpu, batch=32, ctx=[(i * 397) % 3000 + 1 for i in range(32)], page_size=256, n_kv=4,
                             n_heads=28, head_dim=128, s_q=5, seed=23)
    kw = dict(cache_seqlens=d["cache_seqlens"], block_table=d["block_table"], causal=True, noalloc=True)
    eager = prism_amd.flash_attn_with_kvcache(d["q"], d["k_cache"], d["v_cache"], d["k"], d["v"], **kw)
    torch.cuda.synchronize()
    out = torch.full_like(eager, float("nan"))
    cap = torch.cuda.Stream(device=gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            prism_amd.flash_attn_with_kvcache(d["q"], d["k_cache"], d["v_cache"], d["k"], d["v"], out=out, **kw)
    torch.cuda.current_stream(gpu).wait_stream(cap)
    for rep in range(3):
        out.fill_(float("nan"))
        graph.replay()
        other = prism_amd.flash_attn_with_kvcache(d["q"][:4], d["k_cache"], d["v_cache"],
                                                  cache_seqlens=d["cache_seqlens"][:4],
                                                  block_table=d["block_table"][:4], causal=True, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager call"
        assert torch.isfinite(other.float()).all()
    exp, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"], cpu["v"],
                                               cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                               causal=True)
    assert_attn_close(out, exp, "noalloc captured verify")
    assert prism_amd.read_status(gpu) == 0


_FIRST_CALL_CAPTURED = r"""
import sys, torch
sys.path[:0] = [{repo!r}, {tests!r}]
import numpy as np, prism_amd
from oracle import paged_attention as pa
from pkv_testutil import attn_errors, make_paged_case
gpu = torch.device("cuda:0")
cpu, d = make_paged_case(gpu, batch=16, ctx=[(i * 397) % 3000 + 1 for i in range(16)], page_size=256, n_kv=4,
                         n_heads=28, head_dim=128, s_q=1, seed=31)
kw = dict(cache_seqlens=d["cache_seqlens"], block_table=d["block_table"], causal=True, noalloc=True)
out = torch.full_like(d["q"], float("nan"))
torch.cuda.synchronize()
print("capturing the process's first noalloc call", flush=True)
cap = torch.cuda.Stream(device=gpu)
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(cap):
    with torch.cuda.graph(graph, stream=cap):
        prism_amd.flash_attn_with_kvcache(d["q"], d["k_cache"], d["v_cache"], out=out, **kw)
torch.cuda.current_stream(gpu).wait_stream(cap)
exp, _, _ = pa.flash_attn_with_kvcache_ref(cpu["q"], cpu["k_cache"], cpu["v_cache"],
                                           cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"],
                                           causal=True)
first = None
for rep in range(3):
    out.fill_(float("nan"))
    graph.replay()
    eager = prism_amd.flash_attn_with_kvcache(d["q"], d["k_cache"], d["v_cache"], **kw)
    torch.cuda.synchronize()
    mx, mean = attn_errors(out, exp)
    print(f"replay {{rep}}: max-abs {{mx:.3g}} mean-abs {{mean:.3g}}", flush=True)
    assert mx <= 1e-2 and mean <= 1e-3
    assert torch.equal(out, eager), "replay differs from the eager call"
assert prism_amd.read_status(gpu) == 0
print("ok", flush=True)
"""


def test_noalloc_first_call_under_capture():
    # a fresh process whose first noalloc call is made under graph capture: the scratch lookup and
    # its counter clearing (a kernel recorded into the graph) happen inside the capture
    import os
    import subprocess
    import sys
    tests = os.path.dirname(os.path.abspath(__file__))
    script = _FIRST_CALL_CAPTURED.format(repo=os.path.dirname(tests), tests=tests)
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.rstrip().endswith("ok")
