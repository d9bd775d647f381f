"""Benchmark: paged decode attention (append + attention) at the Qwen2.5-7B shape, batch 32.

Default workload (the metric's configuration): 28 layers, 28 query /
4 KV heads, head_dim 128, bf16, 256-token pages in a 2043-page (30 GB) pool fragmented by freeing
a seeded 40% of it, 32 sequences with context lengths lognormal(median 1500, sigma 1) clipped to
[16, 32768].  One step = for each of the 28 layers, append one new K/V row per sequence and run
paged decode attention over it (prism_amd.flash_attn_with_kvcache, the drop-in for Prism's
per-layer call at engine/executor.py:260-261).  Inputs are resident in HBM before timing; every
layer reads its own cache, so a step streams the whole working set and the 256 MB Infinity Cache
cannot serve it.

The step is captured once in a HIP graph and replayed (as Prism's executor runs decode); HIP events
on the replay stream bracket the K timed replays.  Prints one JSON line: value = algorithmic HBM
bytes per step / step time (GB/s), the per-call roofline (step time / layers) and a CPU baseline
(the oracle's torch-CPU reference path on a bounded sample of the same workload, N=1 only).

--workload config2 / config4 / config5 measures the other configurations the same way (decode at
b=8 ctx 2048; 14B chunked prefill, MFMA-bound, in TFLOP/s; 7B shared-prefix speculative verify in
GB/s of unique KV bytes, the shared prefix counted once, on the ordinary and the cascade path,
plus its copy-on-write and a compaction of every live page into a fresh pool).  --workload
epilogue times the elementwise kernels on either side of attention (QKV split + RoPE + paged
append, RMSNorm with the residual add, SiLU-mul) at the 14B prefill-chunk and 7B decode scales,
and config 3's decode step from the QKV projection on as two launches (rope_qk, attention) and as
one (rope_decode_attention).
--workload tables times the per-step host staging of a graph-captured decode batch (block table,
lengths, rotary rows) at config 3's batch: DecodeBatch against the reference's refill.
--workload decode-14B / decode-0.5B / decode-7B-tp4 run config 3's ragged batch at other model
shapes.  --workload peak measures the streaming-read ceiling of the decode kernels' copy pattern
(libpkv_probe.so) that the roofline's published 8 TB/s is checked against.  --workload
tile-stamps reads the timeline of config 3's decode launch from the stamps build of the library
(libprism_kv_stamps.so): when each workgroup starts, when each of its tiles lands, when its range
ends and its parts arrive, and when the merges complete.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_PROFILE = ROOT / "profiles" / "decode_config3_traffic.md"
VERIFY_TRAFFIC_PROFILE = ROOT / "profiles" / "verify_config5_traffic.md"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--workload", choices=["config2", "config3", "config4", "config5", "decode-14B", "decode-0.5B",
                                           "decode-7B-tp4", "long-decode", "long-decode-b1", "prefill-4096",
                                           "epilogue", "tables", "peak", "tile-stamps"], default="config3")
    ap.add_argument("--split", type=int, default=0, help="split_tokens (0 = library choice)")
    ap.add_argument("--grid", type=int, default=0, help="workgroups of the balanced kernel (0 = one per CU)")
    ap.add_argument("--layers", type=int, default=0, help="layers (0 = the model's)")
    ap.add_argument("--batch", type=int, default=0, help="config2's batch at context 2048 (0 = its own 8)")
    ap.add_argument("--merge", choices=["auto", "two-pass", "fused"], default="auto",
                    help="split-K merge of the per-head kernel: library choice, second launch, in-launch")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=4, help="layers in the CPU baseline sample")
    ap.add_argument("--stamp-calls", type=int, default=10, help="stamped calls read by --workload tile-stamps")
    ap.add_argument("--stamps-of", choices=["config3", "config2", "config5", "decode-0.5B", "decode-7B-tp4"],
                    default="config3",
                    help="the decode workload --workload tile-stamps records")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after timing, copy this many MiB of pages once (counter calibration)")
    return ap.parse_args()


def profiled_traffic(args, w, key="traffic_bytes_per_call"):
    """HBM bytes per call from the committed FETCH_SIZE / WRITE_SIZE counter passes over this same
    workload (config 3 or 5, default seed, 28 layers, library-chosen kernel); None otherwise."""
    profile = {"config3": TRAFFIC_PROFILE, "config5": VERIFY_TRAFFIC_PROFILE}.get(args.workload)
    if (profile is None or args.seed != 0 or w.layers != 28 or args.split or args.grid or args.merge != "auto"
            or not profile.exists()):
        return None, None
    for line in profile.read_text().splitlines():
        if line.startswith(key + ":"):
            return int(line.split(":", 1)[1]), str(profile.relative_to(ROOT))
    return None, None


def cpu_baseline(w, n_layers: int, metric_unit: str, gpu_outs=None) -> tuple[dict, dict | None]:
    """The oracle's torch-CPU path (index_select page gather + fp32 SDPA) on n_layers of the workload,
    timed, and its first run's results used as the parity check of the GPU run that preceded it.

    gpu_outs: {name: per-layer GPU outputs} of the timed run(s).  The GPU already appended this call's
    rows, and the CPU path appends the same rows again (the call is idempotent), so the append was
    bit-exact iff the CPU append leaves the gathered pages unchanged; the GPU outputs are compared with
    the fp32 CPU outputs at the north_star tolerance (max-abs <= 1e-2, mean-abs <= 1e-3)."""
    import torch

    from oracle import paged_attention as pa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kv = w.kv
    bt = w.block_table.cpu()
    sl = w.cache_seqlens.cpu()
    # keep only the referenced pages on the host, with the block table remapped onto them
    used = sorted({int(p) for b in range(w.batch) for p in bt[b, : -(-(int(sl[b]) + w.s_q) // kv.page_size)]})
    remap = torch.full((kv.max_pages,), 0, dtype=torch.int64)
    remap[torch.tensor(used)] = torch.arange(len(used))
    bt_host = remap[bt.long().clamp(min=0)].to(torch.int32)
    idx = torch.tensor(used, device=kv.k_pool.device)
    layers = []
    for l in range(n_layers):
        layers.append((kv.k_caches[l].index_select(0, idx).cpu(), kv.v_caches[l].index_select(0, idx).cpu(),
                       w.q[l].cpu(), w.k[l].cpu(), w.v[l].cpu()))

    def run():
        return [pa.flash_attn_cpu(q, kc, vc, k, v, cache_seqlens=sl, block_table=bt_host, causal=True)
                for kc, vc, q, k, v in layers]

    parity = None
    if gpu_outs:
        pre = [(kc.clone(), vc.clone()) for kc, vc, _, _, _ in layers]
        ref = run()
        exact = all(torch.equal(kc, a) and torch.equal(vc, b) for (kc, vc, _, _, _), (a, b) in zip(layers, pre))
        del pre
        parity = {"reference": "oracle.flash_attn_cpu: index_select page gather + fp32 SDPA (enable_gqa), "
                               "bottom-right causal", "layers": list(range(n_layers)),
                  "append_bit_exact": bool(exact), "tol_max_abs": 1e-2, "tol_mean_abs": 1e-3}
        for name, outs in gpu_outs.items():
            errs = [(outs[l].float().cpu() - ref[l]).abs() for l in range(n_layers)]
            finite = all(bool(torch.isfinite(outs[l].float()).all()) for l in range(n_layers))
            mx = max(float(e.max()) for e in errs)
            mean = sum(float(e.sum()) for e in errs) / sum(e.numel() for e in errs)
            parity[name] = {"max_abs": float(f"{mx:.3e}"), "mean_abs": float(f"{mean:.3e}"),
                            "pass": finite and mx <= 1e-2 and mean <= 1e-3}
        parity["pass"] = exact and all(v["pass"] for k, v in parity.items() if isinstance(v, dict))
        print(f"[bench] parity vs CPU reference on {n_layers} layers: "
              + ", ".join(f"{k} max-abs {v['max_abs']} mean-abs {v['mean_abs']}" for k, v in parity.items()
                          if isinstance(v, dict))
              + f", append bit-exact {exact}", file=sys.stderr, flush=True)

    reps = 5 if w.s_q == 1 else 2
    warm = min(3, reps)
    for _ in range(warm):
        run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times) / n_layers
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    value = (w.decode_bytes_per_layer() / per_layer / 1e9 if metric_unit == "GB/s"
             else w.attention_flops_per_layer() / per_layer / 1e12)
    return {
        "value": round(value, 4),
        "unit": metric_unit,
        "cores": cores,
        "kind": "port",
        "us_per_step": round(per_layer * w.layers * 1e6, 1),
        "sample": f"{n_layers} of {w.layers} layers, all {w.batch} sequences, referenced pages only; "
                  f"{warm} warm-ups, median of {reps}; torch {torch.__version__} CPU, {model}",
    }, parity


def time_graph(fn, args, dev) -> float:
    """Capture fn() once in a HIP graph and replay it; HIP events on the replay stream bracket the
    K timed replays.  Returns ms per replay."""
    import torch

    fn()  # eager call: sizes the split-K workspace before capture
    torch.cuda.synchronize()
    cap = torch.cuda.Stream(device=dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            fn()
    torch.cuda.current_stream(dev).wait_stream(cap)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} graph replays)", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream(dev)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    t_end.record(stream)
    torch.cuda.synchronize()
    return t_start.elapsed_time(t_end) / args.steps


def time_eager(fn, reps: int) -> float:
    """ms per call of fn() (one launch), HIP events around reps back-to-back calls."""
    import torch

    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def config5_page_ops(prism_amd, w, dev) -> dict:
    """Copy-on-write of the shared boundary page into every child (one launch) and compaction of
    every live page into a fresh pool (one launch), each timed on its own."""
    kv = w.kv
    L = w.layers
    out = {}
    fill = w.meta["boundary_fill"]
    if fill:
        bidx = w.meta["shared_prefix"] // kv.page_size
        first = kv.seq_pages[w.seq_ids[0]][bidx]
        dst = [kv.seq_pages[s][bidx] for s in w.seq_ids[1:]]
        src = [first] * len(dst)   # the same copy shape: fill slots of one page into every other child
        ms = time_eager(lambda: prism_amd.copy_pages(kv, kv, src, dst, [fill] * len(dst)), 20)
        slot_bytes = kv.num_kv_heads * kv.head_dim * 2
        # HBM must move the source slots once and write every copy: (pages + 1) x fill slots per
        # tensor; the kernel issues a read per copy, but 62 of the 63 reads of the one source page
        # are cache hits, so they are not counted
        nbytes = (len(dst) + 1) * fill * slot_bytes * 2 * L
        issued = 2 * len(dst) * fill * slot_bytes * 2 * L
        out["copy_on_write"] = {"pages": len(dst), "fill_slots": fill, "us": round(ms * 1e3, 2), "bytes": nbytes,
                                "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                "pct_of_peak_hbm": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                                "bytes_issued": issued}
    live = kv.live_pages()
    fresh = prism_amd.FlashAttnKVCache(L, kv.num_kv_heads, kv.head_dim, len(live), kv.page_size, str(dev))
    ms = time_eager(lambda: prism_amd.copy_pages(kv, fresh, live, list(range(len(live))), None), 5)
    nbytes = 2 * len(live) * kv.bytes_per_page * 2 * L
    out["compaction"] = {"pages": len(live), "us": round(ms * 1e3, 1), "bytes": nbytes,
                         "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    # the disaggregated transfer path on one device: one child's pages (every layer, K and V)
    # gathered into staging, copied once as a block (the xGMI peer copy between GPUs), scattered
    # into another cache; bytes = the pages' bytes once (what a transfer moves)
    sid = w.seq_ids[-1]
    n = -(-kv.seq_len[sid] // kv.page_size)
    pages = kv.seq_pages[sid][:n]
    target = prism_amd.FlashAttnKVCache(L, kv.num_kv_heads, kv.head_dim, n, kv.page_size, str(dev))
    ms = time_eager(lambda: prism_amd.copy_pages(kv, target, pages, list(range(n)), None, staged=True), 5)
    nbytes = 2 * n * kv.bytes_per_page * L
    out["staged_transfer"] = {"pages": n, "tokens": kv.seq_len[sid], "us": round(ms * 1e3, 1), "bytes": nbytes,
                              "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    return out


def epilogue_bench(args, dev) -> dict:
    """QKV split + RoPE + paged append, residual add + RMSNorm and SiLU-mul per layer: 20 calls over
    8 per-layer buffer sets (8 x 100-340 MB at the prefill scale: the 256 MB Infinity Cache cannot
    serve a repeat) captured in a HIP graph and replayed, HIP events around the replays.  Bytes are the algorithmic ones: every input
    element read once, every output written once (cos / sin: one table row per token)."""
    import torch

    import prism_amd

    sets = 8
    scales = {
        # name: (model, tokens as (B, s), n_heads, n_kv, hidden, intermediate, page_size, pool pages)
        "prefill14b": ("Qwen2.5-14B chunk 8x512", (8, 512), 40, 8, 5120, 13824),
        "decode7b": ("Qwen2.5-7B decode b=32", (32, 1), 28, 4, 3584, 18944),
    }
    hd, P = 128, 256
    g = torch.Generator(device=dev).manual_seed(args.seed)
    res = {}
    for key, (model, (B, s), nh, nkv, H, M) in scales.items():
        T = B * s
        width = (nh + 2 * nkv) * hd
        pages_per_seq = -(-(4096 + s) // P)
        n_pages = B * pages_per_seq
        cos, sin = prism_amd.rope_tables(hd, 4096 + s, device=dev)
        pos = torch.randint(0, 4096, (B,), generator=g, device=dev, dtype=torch.int32)
        bufs = []
        for _ in range(sets):
            kc = torch.zeros(n_pages, P, nkv, hd, dtype=torch.bfloat16, device=dev)
            bufs.append(dict(
                qkv=torch.randn(B, s, width, generator=g, device=dev).to(torch.bfloat16),
                q=torch.empty(B, s, nh, hd, dtype=torch.bfloat16, device=dev),
                kc=kc, vc=torch.zeros_like(kc),
                x=torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16),
                r=torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16),
                o=torch.empty(T, H, dtype=torch.bfloat16, device=dev),
                h=torch.empty(T, H, dtype=torch.bfloat16, device=dev),
                gu=torch.randn(T, 2 * M, generator=g, device=dev).to(torch.bfloat16),
                a=torch.empty(T, M, dtype=torch.bfloat16, device=dev)))
        w = torch.randn(H, generator=g, device=dev).to(torch.bfloat16)
        bt = torch.randperm(n_pages, generator=g, device=dev).to(torch.int32).view(B, pages_per_seq)
        sl = pos.clone()
        ops = {
            "rope_qk_append": (lambda b: prism_amd.rope_qk(b["qkv"], pos, cos, sin, nh, nkv, return_k=False,
                                                           q_out=b["q"], k_cache=b["kc"], v_cache=b["vc"],
                                                           block_table=bt, cache_seqlens=sl),
                               T * (width + 2 * hd + nh * hd + 2 * nkv * hd) * 2),
            "add_rms_norm": (lambda b: prism_amd.rms_norm(b["x"], w, 1e-6, residual=b["r"], out=b["o"], h_out=b["h"]),
                             (4 * T * H + H) * 2),
            "silu_mul": (lambda b: prism_amd.silu_mul(b["gu"][:, :M], b["gu"][:, M:], out=b["a"]), 3 * T * M * 2),
        }
        out = {"model": model, "tokens": T}
        for name, (fn, nbytes) in ops.items():
            reps = 20

            def calls(fn=fn):
                for i in range(reps):
                    fn(bufs[i % sets])

            # replayed as one HIP graph of 20 calls: the time is the kernels', not Python's
            us = time_graph(calls, argparse.Namespace(warmup=2, steps=5), dev) * 1e3 / reps
            out[name] = {"us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                         "pct_of_peak_hbm": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)}
            print(f"[bench] {key} {name}: {us:.2f} us, {out[name]['gbs']} GB/s", file=sys.stderr, flush=True)
        res[key] = out
        del bufs
        torch.cuda.empty_cache()
    if prism_amd.read_status(dev):
        print("[bench] WARNING: kernel status flags set", file=sys.stderr)
    return res


def decode_step_bench(args, dev) -> dict:
    """Config 3's decode batch from the fused QKV projection on, per layer: rope_qk (split + RoPE
    + append) followed by attention over cache_seqlens + 1, against rope_decode_attention (the
    same in one launch), with the plain append + attention call (rotated q / k given) beside them.
    Each is a graph of the 28-layer step; HIP events around the replays, per layer = step / 28."""
    import torch

    import prism_amd
    from prism_amd import workloads

    w = workloads.config3(dev, seed=args.seed)
    kv, L, B = w.kv, w.layers, w.batch
    nh, nkv, hd = w.n_heads, kv.num_kv_heads, kv.head_dim
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    qkv = [torch.randn(B, 1, (nh + 2 * nkv) * hd, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    cos, sin = prism_amd.rope_tables(hd, int(w.ctx.max()) + 2, device=dev)
    sl, sl1, bt = w.cache_seqlens, w.cache_seqlens + 1, w.block_table
    qbuf = [torch.empty(B, 1, nh, hd, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    outs = [torch.empty(B, 1, nh, hd, dtype=torch.bfloat16, device=dev) for _ in range(L)]

    def two_launch():
        for l in range(L):
            prism_amd.rope_qk(qkv[l], sl, cos, sin, nh, nkv, return_k=False, q_out=qbuf[l],
                              k_cache=kv.k_caches[l], v_cache=kv.v_caches[l], block_table=bt, cache_seqlens=sl)
            prism_amd.flash_attn_with_kvcache(qbuf[l], kv.k_caches[l], kv.v_caches[l], cache_seqlens=sl1,
                                              block_table=bt, causal=True, out=outs[l])

    def fused():
        for l in range(L):
            prism_amd.rope_decode_attention(qkv[l], kv.k_caches[l], kv.v_caches[l], cos, sin, cache_seqlens=sl,
                                            block_table=bt, n_heads=nh, n_kv=nkv, out=outs[l])

    def attention_only():
        for l in range(L):
            prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                              cache_seqlens=sl, block_table=bt, causal=True, out=outs[l])

    res = {"layers": L, "batch": B}
    for name, fn in (("rope_qk_then_attention", two_launch), ("rope_decode_attention", fused),
                     ("append_attention_rotated_inputs", attention_only)):
        us = time_graph(fn, args, dev) * 1e3 / L
        res[name + "_us"] = round(us, 2)
        print(f"[bench] config3 step {name}: {us:.2f} us per layer", file=sys.stderr, flush=True)
    if prism_amd.read_status(dev):
        print("[bench] WARNING: kernel status flags set", file=sys.stderr)
    del w, kv
    torch.cuda.empty_cache()
    return res


def epilogue_cpu_baseline(seed: int) -> dict:
    """The reference's eager torch expressions on the host cores (engine/executor.py:108-127 with
    the Triton norms restated in torch), on 1/8 of the 14B chunk (512 tokens)."""
    import torch

    from oracle import epilogue as ep

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(seed)
    T, nh, nkv, hd, H, M = 512, 40, 8, 128, 5120, 13824
    qkv = torch.randn(1, T, (nh + 2 * nkv) * hd, generator=g).to(torch.bfloat16)
    cos, sin = ep.rope_tables(hd, 4096 + T)
    pos = torch.tensor([1000], dtype=torch.int32)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.randn(H, generator=g).to(torch.bfloat16)
    gu = torch.randn(T, 2 * M, generator=g).to(torch.bfloat16)

    def run():
        ep.cpu_epilogue_ref(qkv, pos, cos, sin, nh, nkv)
        hsum = r + x
        hf = hsum.float()
        (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).to(torch.bfloat16)
        torch.nn.functional.silu(gu[:, :M]) * gu[:, M:]

    for _ in range(2):
        run()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    width = (nh + 2 * nkv) * hd
    nbytes = T * (width + 2 * hd + nh * hd + 2 * nkv * hd) * 2 + (4 * T * H + H) * 2 + 3 * T * M * 2
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the three steps on 512 of the chunk's 4096 tokens (14B shape), eager torch CPU bf16; "
                      f"2 warm-ups, median of 5; torch {torch.__version__}"}


def tables_bench(args, dev) -> dict:
    """Per-step staging of a captured decode batch's inputs at config 3's batch (Qwen2.5-7B shape,
    32 sequences, context lognormal(1500, 1), 2043-page pool with a shuffled free list), each path
    running decode steps of one token per sequence from the same start:

      DecodeBatch      step() + advance(): grow, one packet of changed lengths / pages, one H2D
                       copy, one pkv_table_update launch (rotary positions are cache_seqlens)
      drop-in          the executor's refill (engine/executor.py:345-356: grow, build_block_table,
                       zero + copy the static bt / sl, one cos / sin row copy per sequence) on
                       prism_amd's build_block_table (one H2D copy of the whole table)
      reference        the same refill on the reference's element-by-element build_block_table
                       (engine/kv_cache.py:147-151, restated in the oracle), on device tensors

    Host wall clock around the steps with a device synchronisation at the end (so copies and
    launches are included), median of 3 runs."""
    import numpy as np
    import torch

    import prism_amd
    from oracle.kv_state import graph_staging_elementwise
    from prism_amd import workloads

    s = workloads.SHAPES["7B"]
    mp = workloads.pages_for_budget(30.0, s["layers"], s["n_kv"], s["head_dim"])
    ctx = workloads.lognormal_ctx(np.random.default_rng(args.seed), 32)
    B, hd = len(ctx), s["head_dim"]
    cos, sin = prism_amd.rope_tables(hd, 40000, device=dev)

    def fresh_cache():
        kv = prism_amd.FlashAttnKVCache(1, s["n_kv"], hd, mp, workloads.PAGE, str(dev))
        kv.free_pages = [int(p) for p in np.random.default_rng(args.seed + 1).permutation(mp)]
        for b, c in enumerate(ctx):
            kv.new_sequence(b)
            kv.seq_len[b] = 0
            kv._ensure_capacity(b, int(c))
            kv.seq_len[b] = int(c)
        return kv

    ids = list(range(B))

    def run_decode_batch(n):
        kv = fresh_cache()
        db = prism_amd.DecodeBatch(kv, max_batch=B)
        db.step(ids, 1, graph_batch=B)
        db.advance()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            db.step(ids, 1, graph_batch=B)
            db.advance()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    def run_refill(n, elementwise):
        kv = fresh_cache()
        g_bt = torch.zeros(B, 32, dtype=torch.int32, device=dev)   # engine/executor.py:282
        g_sl = torch.zeros(B, dtype=torch.int32, device=dev)
        g_cos = torch.zeros(B, 1, hd, dtype=torch.bfloat16, device=dev)
        g_sin = torch.zeros(B, 1, hd, dtype=torch.bfloat16, device=dev)
        bt_buf = torch.zeros(B, 32, dtype=torch.int32, device=dev)  # build_block_table's buffers
        sl_buf = torch.zeros(B, dtype=torch.int32, device=dev)

        def one():
            for sid in ids:
                kv._ensure_capacity(sid, kv.seq_len[sid] + 1)
            if elementwise:
                graph_staging_elementwise(bt_buf, sl_buf, g_bt, g_sl, kv.seq_pages, kv.seq_len, ids,
                                          cos, sin, g_cos, g_sin)
            else:
                bt, sl = kv.build_block_table(ids)
                nb = bt.shape[1]
                g_bt[:] = 0
                g_bt[:B, :nb] = bt
                g_sl[:] = 0
                g_sl[:B] = sl
                for i, sid in enumerate(ids):
                    g_cos[i, 0].copy_(cos[kv.seq_len[sid]])
                    g_sin[i, 0].copy_(sin[kv.seq_len[sid]])
            for sid in ids:
                kv.seq_len[sid] += 1

        one()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            one()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    ours = statistics.median(run_decode_batch(512) for _ in range(3))
    print(f"[bench] DecodeBatch {ours:.1f} us/step", file=sys.stderr, flush=True)
    drop_in = statistics.median(run_refill(128, False) for _ in range(3))
    print(f"[bench] drop-in refill {drop_in:.1f} us/step", file=sys.stderr, flush=True)
    ref = None
    if not args.no_cpu_baseline:
        ref = statistics.median(run_refill(16, True) for _ in range(3))
        print(f"[bench] reference refill {ref:.1f} us/step", file=sys.stderr, flush=True)

    # device time of one table update (32 lengths + 1 page entry): 20 launches on the uploaded
    # packet captured in a HIP graph and replayed (host launch overhead excluded)
    kv = fresh_cache()
    db = prism_amd.DecodeBatch(kv, max_batch=B)
    db.step(ids, 1, graph_batch=B)
    packet = np.concatenate([np.stack([np.arange(B), np.asarray(ctx, dtype=np.int64)], 1).ravel(),
                             np.array([0, 0, kv.seq_pages[0][0]])]).astype(np.int32)
    db.apply(packet, B, 1)
    lib = prism_amd._lib.load()
    st = prism_amd.status_tensor(dev)

    def launches():
        for _ in range(20):
            rc = lib.pkv_table_update(db._packet_dev.data_ptr(), B, 1, db.block_table.data_ptr(),
                                      db.block_table.stride(0), db.cache_seqlens.data_ptr(), B, db.max_blocks,
                                      mp, st.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
            prism_amd._lib.check(rc, "pkv_table_update")

    upd_us = time_graph(launches, argparse.Namespace(warmup=2, steps=10), dev) * 1e3 / 20
    return {"decode_batch_us": round(ours, 1), "drop_in_us": round(drop_in, 1),
            "reference_us": None if ref is None else round(ref, 1), "update_us": round(upd_us, 2),
            "packet_bytes": int(packet.nbytes), "batch": B, "pool_pages": mp,
            "max_pages_per_seq": max(len(kv.seq_pages[b]) for b in ids)}


def peak_bench(args, dev) -> dict:
    """Streaming-read rates of the decode kernels' copy pattern (global->LDS, 1 KiB per wave
    instruction, one 4-wave workgroup per CU) from a buffer far larger than the caches, read once
    (HBM), and from a 64 MiB window re-read by every workgroup (last-level cache): the measured
    ceiling that the HBM roofline's published 8 TB/s is checked against."""
    import ctypes

    import torch

    from prism_amd.build import PROBE_LIB_PATH

    if not PROBE_LIB_PATH.exists():
        raise RuntimeError(f"{PROBE_LIB_PATH} is not built: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(PROBE_LIB_PATH))
    lib.pkv_probe_stream_read.restype = ctypes.c_int
    lib.pkv_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    per_wg = 32 << 20  # 32 MiB per workgroup: 8 GiB over 256 CUs
    buf = torch.randint(0, 255, (grid * per_wg,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for name, window, policy in (("hbm_nt", grid * per_wg, 2), ("hbm_default", grid * per_wg, 0),
                                 ("llc_64mib", 64 << 20, 0)):
        def launch():
            rc = lib.pkv_probe_stream_read(buf.data_ptr(), window, per_wg, grid, policy, sink.data_ptr(),
                                           stream.cuda_stream)
            if rc:
                raise RuntimeError(f"pkv_probe_stream_read returned {rc}")

        for _ in range(2):
            launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            launch()
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.steps
        res[name] = {"bytes": grid * per_wg, "us": round(us, 1), "gbs": round(grid * per_wg / (us * 1e-6) / 1e9, 1)}
        print(f"[bench] peak {name}: {res[name]}", file=sys.stderr, flush=True)
    del buf
    return res


def tile_stamps_bench(args, dev) -> dict:
    """Timeline of a decode launch (decode_lean_kernel with its in-launch merge; config 3 unless
    --stamps-of names another decode workload) from
    libprism_kv_stamps.so: per-call time of both builds (graph replays), then eager calls whose
    stamps are read back.  Times are us from the first decode workgroup's start (100 MHz clock).
    Also bounds what a pool of tail tiles could gain on these measured timelines: the shortest
    ranges of a static split (per - 1 tiles, as many as the tile count leaves) assigned to the
    ranges that reach iteration k last (a claim made k tiles into the range, as a pool's copy
    pipeline would need), or, as the bound, to the ranges that actually end last."""
    import numpy as np
    import torch

    import prism_amd
    from prism_amd import _lib, workloads
    from prism_amd.build import LIB_PATH, STAMPS_LIB_PATH

    if not STAMPS_LIB_PATH.exists():
        raise RuntimeError(f"{STAMPS_LIB_PATH} is not built: run __graft_entry__.build() first")
    if args.stamps_of.startswith("decode-"):
        w = workloads.ragged_decode(args.stamps_of[len("decode-"):], dev, seed=args.seed)
    elif args.stamps_of == "config2" and args.batch:
        w = workloads.config2(dev, seed=args.seed, batch=args.batch)
    else:
        w = getattr(workloads, args.stamps_of)(dev, seed=args.seed)
    kv, L = w.kv, w.layers
    outs = [torch.empty_like(q) for q in w.q]

    def call(l):
        prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                          cache_seqlens=w.cache_seqlens, block_table=w.block_table, causal=True,
                                          out=outs[l])

    def step():
        for l in range(L):
            call(l)

    us_plain = time_graph(step, args, dev) * 1e3 / L
    lib = _lib.use(STAMPS_LIB_PATH)
    try:
        import ctypes

        lib.pkv_tile_stamp_words.restype = ctypes.c_int
        lib.pkv_tile_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.pkv_tile_stamps_clear.argtypes = [ctypes.c_void_p]
        us_stamped = time_graph(step, args, dev) * 1e3 / L
        n_words = lib.pkv_tile_stamp_words()
        host = torch.zeros(n_words, dtype=torch.int64).pin_memory()
        stream = torch.cuda.current_stream(dev).cuda_stream
        calls = []
        for i in range(4 + args.stamp_calls):
            if lib.pkv_tile_stamps_clear(ctypes.c_void_p(stream)) != 0:
                raise RuntimeError("pkv_tile_stamps_clear failed")
            call(i % L)
            if lib.pkv_tile_stamps(ctypes.c_void_p(host.data_ptr()), n_words * 8, ctypes.c_void_p(stream)) != 0:
                raise RuntimeError("pkv_tile_stamps failed")
            torch.cuda.synchronize()
            if i >= 4:
                calls.append(host.numpy().copy())
        status = prism_amd.read_status(dev)
    finally:
        _lib.use(LIB_PATH)
    if status:
        raise RuntimeError(f"status word {status} after the stamped calls")

    WG_WORDS, N_WG, N_MERGE = 32, 1024, 4096
    per_call = []
    for a in calls:
        d = a[:N_WG * WG_WORDS].reshape(N_WG, WG_WORDS)
        m = a[N_WG * WG_WORDS:N_WG * WG_WORDS + 4 * N_MERGE].reshape(N_MERGE, 4)
        dec = np.nonzero(d[:, 0] > 0)[0]
        t0 = d[dec, 0].min()
        us = lambda x: (x - t0) / 100.0
        full = [wg for wg in dec if d[wg, 3] > 0]
        per = int(max(d[wg, 3] for wg in full))
        rows = []
        for wg in full:
            n = int(d[wg, 3])
            t = us(d[wg, 8:8 + min(n, 24)].astype(np.float64))
            rows.append({"wg": int(wg), "n": n, "start": us(d[wg, 0]), "tiles": t, "end": us(d[wg, 1]),
                         "arrival": us(d[wg, 2]) if d[wg, 2] else None, "segs": bin(int(d[wg, 4])).count("1"),
                         "mask": int(d[wg, 4])})
        mu = np.nonzero(m[:, 0] > 0)[0]
        per_call.append({"rows": rows, "per": per, "grid": len(dec), "tiles": sum(r["n"] for r in rows),
                         "merge_ready": us(m[mu, 1].max()) if len(mu) else None,
                         "merge_done": us(m[mu, 2].max()) if len(mu) else None,
                         "last_arrival": max((r["arrival"] for r in rows if r["arrival"] is not None), default=None)})

    def med(xs):
        return round(float(np.median(xs)), 2)

    def pct(xs, q):
        return round(float(np.percentile(xs, q)), 2)

    first, plain, after_end, ends_by_seg, xcd_end = [], [], [], {}, {}
    for c in per_call:
        for r in c["rows"]:
            t = r["tiles"]
            first.append(t[0])
            for j in range(1, len(t)):
                (after_end if r["mask"] >> (j - 1) & 1 else plain).append(t[j] - t[j - 1])
            ends_by_seg.setdefault(r["segs"], []).append(r["end"])
            xcd_end.setdefault(r["wg"] % 8, []).append(r["end"])
    # the tail-pool bound, per call: ranges of `per` tiles only
    pool = {}
    for c in per_call:
        full = [r for r in c["rows"] if r["n"] == c["per"] and len(r["tiles"]) == c["per"]]
        n_short = c["grid"] * c["per"] - c["tiles"]  # ranges a static split of per - 1 tiles leaves short
        if c["per"] < 3 or n_short <= 0 or n_short >= len(full):
            continue
        T = np.array([r["tiles"] for r in full])
        E = np.array([r["end"] for r in full])
        end_short = T[:, -2] + (E - T[:, -1])  # the same range one tile shorter
        for key, order in [(f"claim_at_tile_{k}", np.argsort(T[:, k])) for k in range(1, c["per"] - 2)] + \
                          [("bound_slowest_known", np.argsort(E))]:
            short, rest = order[-n_short:], order[:-n_short]
            for cost in (0.3, 1.0):
                new_last = max((E[rest] + cost).max(), end_short[short].max())
                pool.setdefault(f"{key}_cost_{cost}", []).append(new_last - E.max())
    return {
        "us_per_call_plain": round(us_plain, 2), "us_per_call_stamped": round(us_stamped, 2),
        "calls": len(per_call), "grid": per_call[0]["grid"], "tiles": per_call[0]["tiles"],
        "tiles_per_range": per_call[0]["per"],
        "start_spread_p90": med([pct([r["start"] for r in c["rows"]], 90) for c in per_call]),
        "first_tile": {"median": med(first), "p90": pct(first, 90)},
        "tile_interval": {"median": med(plain), "p90": pct(plain, 90)},
        "tile_after_segment_end": {"median": med(after_end), "p90": pct(after_end, 90)} if after_end else None,
        "range_end_by_segment_ends": {str(k): {"ranges": len(v), "median": med(v), "p90": pct(v, 90),
                                               "max": round(float(np.max(v)), 2)}
                                      for k, v in sorted(ends_by_seg.items())},
        "range_end_median_by_xcd": {str(k): med(v) for k, v in sorted(xcd_end.items())},
        "end_vs_first_tile_corr": round(float(np.corrcoef([r["end"] for c in per_call for r in c["rows"]],
                                                          [r["tiles"][0] for c in per_call for r in c["rows"]])[0, 1]), 2),
        "last_range_end": med([max(r["end"] for r in c["rows"]) for c in per_call]),
        "last_arrival": med([c["last_arrival"] for c in per_call if c["last_arrival"] is not None]),
        "last_merge_ready": med([c["merge_ready"] for c in per_call if c["merge_ready"] is not None]),
        "last_merge_done": med([c["merge_done"] for c in per_call if c["merge_done"] is not None]),
        "tail_pool_change_of_last_range_end_us": {k: med(v) for k, v in pool.items()},
    }


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs on a single MI355X and has no multi-GPU "
              "path (the paged KV hot path would shard by KV head, each rank running its heads' "
              "shard of every call unchanged). Use --gpus 1.",
              file=sys.stderr)
        return 2
    import torch

    import prism_amd
    from prism_amd import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "epilogue":
        res = epilogue_bench(args, dev)
        pf = res["prefill14b"]
        names = ("rope_qk_append", "add_rms_norm", "silu_mul")
        tot_b = sum(pf[n]["bytes"] for n in names)
        tot_us = sum(pf[n]["us"] for n in names)
        dom = max(names, key=lambda n: pf[n]["bytes"])
        result = {
            "metric": "attention epilogue kernels HBM GB/s (% of peak), Qwen2.5-14B prefill chunk 8x512 per layer",
            "value": round(tot_b / (tot_us * 1e-6) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": 20,
            "warmup": 1, "ms_per_step": round(tot_us / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "epilogue: QKV split + RoPE + paged append, residual add + RMSNorm, SiLU-mul "
                                   "per layer at the 14B prefill chunk (4096 tokens) and the 7B decode batch "
                                   "(32 tokens)", "seed": args.seed},
            "roofline": {"bound": "hbm", "achieved": pf[dom]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pf[dom]["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": f"{dom} (the largest of the three) at the 14B prefill chunk; HIP events around "
                                   "graph replays of 20 calls over 8 per-layer buffer sets",
                         "bytes_per_call": pf[dom]["bytes"], "avg_call_us": pf[dom]["us"]},
            "kernels": res,
            "decode_step_config3": decode_step_bench(args, dev),
        }
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = epilogue_cpu_baseline(args.seed)
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "peak":
        res = peak_bench(args, dev)
        best = max(res["hbm_nt"]["gbs"], res["hbm_default"]["gbs"])
        result = {
            "metric": "streaming HBM read GB/s of the decode kernels' global->LDS copy pattern (8 GiB, read once)",
            "value": best, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 2,
            "ms_per_step": round(res["hbm_nt"]["us"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "peak: one 4-wave workgroup per CU streams 32 MiB of an 8 GiB buffer into LDS "
                                   "(1 KiB per wave copy, 32 KiB stages, two in flight), non-temporal and default "
                                   "cache policy, then a 64 MiB window every workgroup re-reads"},
            "roofline": {"bound": "hbm", "achieved": best, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(best / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "stream_read_kernel (libpkv_probe.so); HIP events around K launches",
                         "bytes_per_call": res["hbm_nt"]["bytes"], "avg_call_us": res["hbm_nt"]["us"]},
            "detail": res,
        }
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "tile-stamps":
        res = tile_stamps_bench(args, dev)
        result = {
            "metric": f"{args.stamps_of} decode call timeline (decode_lean_kernel + in-launch merge), us from the "
                      "first workgroup's start",
            "value": res["last_merge_done"], "unit": "us", "n_gpus": 1, "steps": args.stamp_calls, "warmup": 4,
            "ms_per_step": round(res["us_per_call_stamped"] / 1e3, 5), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": f"tile-stamps: {args.stamps_of}'s call (layer i, eager) on the stamps build "
                                   "(libprism_kv_stamps.so)", "seed": args.seed, "batch": args.batch or None},
            "detail": res,
        }
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "tables":
        res = tables_bench(args, dev)
        result = {
            "metric": "decode-step input staging us per step (block table, lengths, rotary rows), "
                      "Qwen2.5-7B b=32, 2043-page pool",
            "value": res["decode_batch_us"], "unit": "us/step", "n_gpus": 1, "steps": 512, "warmup": 1,
            "ms_per_step": round(res["decode_batch_us"] / 1e3, 4), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "int32", "data": "synthetic",
            "config": {"workload": "tables: DecodeBatch.step + advance per decode step of 32 sequences (config 3 "
                                   "lengths), against the executor's per-step refill of its graph buffers",
                       "seed": args.seed},
            # a few hundred bytes per launch: the update kernel is launch-bound, not HBM-bound
            "roofline": {"bound": "hbm", "achieved": round(res["packet_bytes"] * 2 / (res["update_us"] * 1e-6) / 1e9, 4),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(res["packet_bytes"] * 2 / (res["update_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 8),
                         "traffic": None,
                         "kernel": "pkv_table_update (32 lengths + 1 page entry: packet read + entries written); "
                                   "HIP events around graph replays of 20 launches; launch-bound",
                         "avg_call_us": res["update_us"]},
            "drop_in_refill_us_per_step": res["drop_in_us"],
            "detail": res,
        }
        if res["reference_us"] is not None:
            result["cpu_baseline"] = {"value": res["reference_us"], "unit": "us/step", "cores": 1, "kind": "port",
                                      "sample": "16 decode steps of the reference's element-by-element refill "
                                                "(oracle restatement of engine/kv_cache.py:147-151 and "
                                                "engine/executor.py:345-356) on device tensors, median of 3"}
        print(json.dumps(result), flush=True)
        return 0
    print(f"[bench] building {args.workload} workload (seed={args.seed})", file=sys.stderr, flush=True)
    if args.workload.startswith("decode-"):
        w = workloads.ragged_decode(args.workload[len("decode-"):], dev, seed=args.seed, layers=args.layers or None)
    elif args.workload.startswith("long-decode"):
        w = workloads.long_decode(dev, seed=args.seed, layers=args.layers or None,
                                  batch=1 if args.workload.endswith("-b1") else 32)
    elif args.workload == "prefill-4096":
        w = workloads.prompt_prefill(dev, seed=args.seed, layers=args.layers or None, prompt=4096)
    elif args.workload == "config2" and args.batch:
        w = workloads.config2(dev, seed=args.seed, layers=args.layers or None, batch=args.batch)
    else:
        w = getattr(workloads, args.workload)(dev, seed=args.seed, layers=args.layers or None)
    L = w.layers
    outs = [torch.empty_like(q) for q in w.q]
    kv = w.kv
    two_pass = {"auto": None, "two-pass": True, "fused": False}[args.merge]

    def step():
        for l in range(L):
            prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                              cache_seqlens=w.cache_seqlens, block_table=w.block_table,
                                              causal=True, out=outs[l], split_tokens=args.split, grid=args.grid,
                                              two_pass=two_pass)

    step_ms = time_graph(step, args, dev)
    status = prism_amd.read_status(dev)
    if status:
        print(f"[bench] WARNING: kernel status flags {status}", file=sys.stderr)
    call_us = step_ms * 1e3 / L
    bytes_layer = w.decode_bytes_per_layer()
    flops_layer = w.attention_flops_per_layer()
    gbs = bytes_layer / (call_us * 1e-6) / 1e9
    tflops = flops_layer / (call_us * 1e-6) / 1e12
    print(f"[bench] step {step_ms * 1e3:.1f} us, call avg {call_us:.2f} us, {gbs:.0f} GB/s, {tflops:.1f} TFLOP/s",
          file=sys.stderr, flush=True)

    if args.copy_probe_mib:
        n_pages = max(1, args.copy_probe_mib * (1 << 20) // (kv.bytes_per_page * 2 * L))
        src = list(range(min(n_pages, kv.max_pages)))
        probe = prism_amd.FlashAttnKVCache(L, kv.num_kv_heads, kv.head_dim, len(src), kv.page_size, str(dev))
        prism_amd.copy_pages(kv, probe, src, list(range(len(src))), None)
        torch.cuda.synchronize()
        print(f"[bench] copy probe: {len(src) * kv.bytes_per_page * 2 * L} bytes read and written by "
              f"copy_pages_kernel", file=sys.stderr, flush=True)

    common = {
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4), "us_per_step": round(step_ms * 1e3, 1),
        "tokens_per_s": round(w.batch * w.s_q / (step_ms * 1e-3), 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
    }
    cfg = {"workload": "", "batch": w.batch, "layers": L, "n_heads": w.n_heads, "n_kv": kv.num_kv_heads,
           "head_dim": kv.head_dim, "page_size": kv.page_size, "pool_pages": kv.max_pages, "s_q": w.s_q,
           "sum_ctx": int(w.ctx.sum()), "max_ctx": int(w.ctx.max()), "seed": args.seed,
           "split_tokens": args.split or "auto", "grid": args.grid or "auto", "merge": args.merge}
    per_call = f"HIP events around K graph replays of the {L}-call step, per call = step / {L}"
    decode_like = args.workload in ("config2", "config3") or args.workload.startswith(("decode-", "long-decode"))
    if decode_like:
        traffic, traffic_src = profiled_traffic(args, w)
        if args.workload == "config3":
            metric = "paged decode attn HBM GB/s (% of peak) + us/step, Qwen2.5-7B shape b=32"
            cfg["workload"] = ("config3: Qwen2.5-7B paged decode (append + attention), 28 layers, b=32, ctx "
                               "lognormal(1500, 1) in [16, 32768], 2043-page 30 GB pool, 40% churn")
        elif args.workload.startswith("long-decode"):
            metric = f"paged decode attn HBM GB/s (% of peak) + us/step, Qwen2.5-7B shape b={w.batch}, long contexts"
            cfg["workload"] = (f"{args.workload}: " + (
                "config3's ragged batch (b=32, ctx lognormal(1500, 1), 40% churn) with sequence 0 at 32767 cached "
                "keys and sequence 1 at 12000" if w.batch > 1 else "one sequence at 32767 cached keys (the B = 1 "
                "decode graph)") + f", Qwen2.5-7B shape, {L} layers, {kv.max_pages}-page pool")
        elif args.workload.startswith("decode-"):
            shape = w.meta["shape"]
            metric = f"paged decode attn HBM GB/s (% of peak) + us/step, Qwen2.5-{shape} shape b={w.batch}"
            cfg["workload"] = (f"{args.workload}: config3's ragged batch (b={w.batch}, ctx lognormal(1500, 1), 40% "
                               f"churn) at the Qwen2.5-{shape} shape, {L} layers, {kv.max_pages}-page pool")
        else:
            metric = f"paged decode attn HBM GB/s (% of peak) + us/step, Qwen2.5-7B shape b={w.batch} ctx 2048"
            cfg["workload"] = (f"config2: Qwen2.5-7B paged decode (append + attention), 28 layers, b={w.batch}, "
                               "ctx 2048, 2043-page 30 GB pool")
        result = {
            "metric": metric, "value": round(bytes_layer * L / (step_ms * 1e-3) / 1e9, 2), "unit": "GB/s",
            **common, "pct_of_peak_hbm": round(100 * gbs / HBM_PEAK_GBS, 2), "config": cfg,
            "roofline": {
                "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "kernel": "one pkv_decode_attn call = decode_lean_kernel (append + balanced paged attention, "
                          "split-K partials merged by workgroups appended to the launch; a second "
                          "combine_lean_kernel launch when those exceed one per CU); " + per_call,
                "bytes_per_call": bytes_layer, "avg_call_us": round(call_us, 3),
            },
        }
        unit = "GB/s"
    elif args.workload in ("config4", "prefill-4096"):
        if args.workload == "config4":
            cfg["workload"] = ("config4: Qwen2.5-14B varlen chunked prefill over paged KV, 48 layers, b=8 chunks of "
                               "512 appended onto prefixes ~U{0..4096}, causal, 596-page 30 GB pool")
            metric = "chunked prefill attn TFLOP/s (% of bf16 MFMA peak), Qwen2.5-14B shape b=8 chunk 512"
        else:
            cfg["workload"] = ("prefill-4096: Qwen2.5-7B whole-prompt prefill (engine/executor.py:97-120), b=1, a "
                               f"4096-token prompt with no prefix appended and attended causally, {L} layers, "
                               f"{kv.max_pages}-page 30 GB pool")
            metric = "whole-prompt prefill attn TFLOP/s (% of bf16 MFMA peak), Qwen2.5-7B shape b=1 prompt 4096"
        result = {
            "metric": metric,
            "value": round(flops_layer * L / (step_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", **common,
            "config": cfg,
            "roofline": {
                "bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                "kernel": "one pkv_prefill_attn call = append_kernel + prefill_lds_kernel<2,4,4,1> (LDS-staged KV tiles in 4 stages, 128 query rows per workgroup); " + per_call,
                "flops_per_call": flops_layer, "bytes_per_call": bytes_layer, "avg_call_us": round(call_us, 3),
                "hbm_gbs": round(gbs, 1),
            },
        }
        unit = "TFLOP/s"
    else:
        cfg["workload"] = ("config5: Qwen2.5-7B shared 2048-token prefix (ref-counted, copy-on-write boundary "
                           "page) + speculative verify of 5 draft tokens, 28 layers, b=64, suffix ~U{0..1024}")
        cfg.update({k: v for k, v in w.meta.items() if k not in ("shape", "root_pages")})
        outs_cascade = [torch.empty_like(q) for q in w.q]
        # cascade attention over the pages every child shares (the full pages of the prefix; the
        # boundary page was copied into each child): the prefix read once per layer for the batch
        shared_tokens = (w.meta["shared_prefix"] // kv.page_size) * kv.page_size

        def cascade_step():
            for l in range(L):
                prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                                  cache_seqlens=w.cache_seqlens, block_table=w.block_table,
                                                  causal=True, out=outs_cascade[l],
                                                  shared_prefix_tokens=shared_tokens)

        cascade_ms = time_graph(cascade_step, args, dev)
        c_status = prism_amd.read_status(dev)
        if c_status:
            print(f"[bench] WARNING: cascade status flags {c_status}", file=sys.stderr)
        c_us = cascade_ms * 1e3 / L
        unique_layer = bytes_layer - (w.batch - 1) * shared_tokens * kv.num_kv_heads * kv.head_dim * 2 * 2
        print(f"[bench] cascade: call avg {c_us:.2f} us ({shared_tokens} shared tokens)", file=sys.stderr, flush=True)
        cascade = {"shared_tokens": shared_tokens, "avg_call_us": round(c_us, 3), "ms_per_step": round(cascade_ms, 4),
                   "speedup": round(call_us / c_us, 3), "unique_bytes_per_call": unique_layer,
                   "gbs_unique": round(unique_layer / (c_us * 1e-6) / 1e9, 1),
                   "frac_unique": round(unique_layer / (c_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                   "mfma_tflops": round(flops_layer / (c_us * 1e-6) / 1e12, 2),
                   "mfma_frac": round(flops_layer / (c_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                   "kernels": "prefill_lds_kernel (prefix pass, key splits) + decode_lean_kernel<3> (suffixes) + "
                              "combine_lean_kernel; HIP events around graph replays"}
        # the same verify where the shared prefix dominates (8192-token prompt, suffixes <= 256)
        wl = workloads.config5(dev, seed=args.seed, prefix=8192, max_suffix=256)
        shared_l = (wl.meta["shared_prefix"] // wl.kv.page_size) * wl.kv.page_size
        outs_l = [torch.empty_like(q) for q in wl.q]

        def long_step(sp):
            def f():
                for l in range(wl.layers):
                    prism_amd.flash_attn_with_kvcache(wl.q[l], wl.kv.k_caches[l], wl.kv.v_caches[l], k=wl.k[l],
                                                      v=wl.v[l], cache_seqlens=wl.cache_seqlens,
                                                      block_table=wl.block_table, causal=True, out=outs_l[l],
                                                      shared_prefix_tokens=sp)
            return f

        plain_l = time_graph(long_step(0), args, dev) * 1e3 / wl.layers
        casc_l = time_graph(long_step(shared_l), args, dev) * 1e3 / wl.layers
        print(f"[bench] long prefix: plain {plain_l:.2f} us, cascade {casc_l:.2f} us", file=sys.stderr, flush=True)
        cascade["long_prefix"] = {"prefix": 8192, "max_suffix": 256, "shared_tokens": shared_l,
                                  "plain_us": round(plain_l, 3), "cascade_us": round(casc_l, 3),
                                  "speedup": round(plain_l / casc_l, 3)}
        del wl, outs_l
        torch.cuda.empty_cache()
        page_ops = config5_page_ops(prism_amd, w, dev)
        # the HBM roofline counts every key once (the shared prefix once for the batch): the
        # per-sequence re-reads of the prefix are served by the caches, so they are reported apart
        gbs_unique = unique_layer / (call_us * 1e-6) / 1e9
        traffic, traffic_src = profiled_traffic(args, w)
        cascade["traffic"], _ = profiled_traffic(args, w, "cascade_traffic_bytes_per_call")
        result = {
            "metric": "speculative verify attn GB/s of unique KV bytes (% of HBM peak) + MFMA %, "
                      "Qwen2.5-7B shape b=64 draft 5",
            "value": round(unique_layer * L / (step_ms * 1e-3) / 1e9, 2), "unit": "GB/s", **common,
            "config": cfg,
            "roofline": {
                "bound": "hbm", "achieved": round(gbs_unique, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs_unique / HBM_PEAK_GBS, 4), "traffic": traffic,
                **({"traffic_source": traffic_src} if traffic_src else {}),
                "mfma_tflops": round(tflops, 2), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                "kernel": "one pkv_decode_attn call (s_q=5, 35 query rows per KV head) = decode_lean_kernel<3> "
                          "(balanced tile ranges, 3 MFMA row tiles per wave) + combine_lean_kernel; bytes count "
                          "every key once, the shared prefix once for the batch; " + per_call,
                "bytes_per_call": unique_layer, "flops_per_call": flops_layer, "avg_call_us": round(call_us, 3),
                "per_sequence_bytes_per_call": bytes_layer, "gbs_per_sequence": round(gbs, 1),
            },
            "page_ops": page_ops,
            "cascade": cascade,
        }
        unit = "GB/s"
    if not args.no_cpu_baseline:
        n_cpu = min(args.cpu_layers if args.workload == "config3" else 1, L)
        print(f"[bench] cpu baseline on {n_cpu} layers", file=sys.stderr, flush=True)
        gpu_outs = {"out": outs}
        if args.workload == "config5":
            gpu_outs = {"verify": outs, "cascade": outs_cascade}
        result["cpu_baseline"], result["parity"] = cpu_baseline(w, n_cpu, unit, gpu_outs)
    print(json.dumps(result), flush=True)
    if result.get("parity") is not None and not result["parity"]["pass"]:
        print("[bench] PARITY FAILED: the GPU results differ from the CPU reference", file=sys.stderr, flush=True)
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())
