"""Benchmark: paged decode attention (append + attention) at the Qwen2.5-7B shape, batch 32.

Workload (the metric's configuration): 28 layers, 28 query / 4 KV heads,
head_dim 128, bf16, 256-token pages in a 2043-page (30 GB) pool fragmented by freeing a seeded 40%
of it, 32 sequences with context lengths lognormal(median 1500, sigma 1) clipped to [16, 32768].
One step = for each of the 28 layers, append one new K/V row per sequence and run paged decode
attention over it (prism_amd.flash_attn_with_kvcache, the drop-in for Prism's per-layer call at
engine/executor.py:260-261).  Inputs are resident in HBM before timing; every layer reads its own
cache, so a step streams the whole working set and the 256 MB Infinity Cache cannot serve it.

The step is captured once in a HIP graph and replayed (as Prism's executor runs decode); HIP events
on the replay stream bracket the K timed replays.  Prints one JSON line: value = algorithmic HBM
bytes per step / step time (GB/s), the per-call roofline (step time / 28 calls) and a CPU baseline
(the oracle's torch-CPU reference path on a bounded sample of the same workload, N=1 only).
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--split", type=int, default=0, help="split_tokens (0 = library choice)")
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--merge", choices=["auto", "two-pass", "fused"], default="auto",
                    help="split-K merge: library choice, second launch, or inside the attention launch")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=4, help="layers in the CPU baseline sample")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after timing, gather this many MiB of pages once (counter calibration)")
    return ap.parse_args()


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_config3_traffic.md"


def profiled_traffic(args, w):
    """HBM bytes per call from the committed FETCH_SIZE / WRITE_SIZE counter passes over this same
    workload (default seed, 28 layers, library-chosen kernel); None for any other configuration."""
    if args.seed != 0 or w.layers != 28 or args.split or args.merge != "auto" or not TRAFFIC_PROFILE.exists():
        return None, None
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_call:"):
            return int(line.split(":", 1)[1]), str(TRAFFIC_PROFILE.relative_to(ROOT))
    return None, None


def cpu_baseline(w, n_layers: int) -> dict:
    """The oracle's torch-CPU path (index_select page gather + fp32 SDPA) on n_layers of the workload."""
    import numpy as np
    import torch

    from oracle import paged_attention as pa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kv = w.kv
    bt = w.block_table.cpu()
    sl = w.cache_seqlens.cpu()
    # keep only the referenced pages on the host, with the block table remapped onto them
    used = sorted({int(p) for b in range(w.batch) for p in bt[b, : -(-(int(sl[b]) + 1) // kv.page_size)]})
    remap = torch.full((kv.max_pages,), 0, dtype=torch.int64)
    remap[torch.tensor(used)] = torch.arange(len(used))
    bt_host = remap[bt.long()].to(torch.int32)
    idx = torch.tensor(used, device=kv.k_pool.device)
    layers = []
    for l in range(n_layers):
        layers.append((kv.k_caches[l].index_select(0, idx).cpu(), kv.v_caches[l].index_select(0, idx).cpu(),
                       w.q[l].cpu(), w.k[l].cpu(), w.v[l].cpu()))

    def run():
        for kc, vc, q, k, v in layers:
            pa.flash_attn_cpu(q, kc, vc, k, v, cache_seqlens=sl, block_table=bt_host, causal=True)

    for _ in range(3):
        run()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    per_layer = med / n_layers
    bytes_layer = w.decode_bytes_per_layer()
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(bytes_layer / per_layer / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "us_per_step": round(per_layer * w.layers * 1e6, 1),
        "sample": f"{n_layers} of {w.layers} layers, all {w.batch} sequences, referenced pages only; "
                  f"3 warm-ups, median of 5; torch {torch.__version__} CPU, {model}",
    }


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs on a single MI355X and has no multi-GPU "
              "path (the paged KV hot path shards by KV head / sequence; see DESIGN.md). Use --gpus 1.",
              file=sys.stderr)
        return 2
    import torch

    import prism_amd
    from prism_amd import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"[bench] building config3 workload (layers={args.layers}, seed={args.seed})", file=sys.stderr, flush=True)
    w = workloads.config3(dev, seed=args.seed, layers=args.layers)
    L = w.layers
    outs = [torch.empty_like(q) for q in w.q]
    kv = w.kv

    def call(l):
        prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                          cache_seqlens=w.cache_seqlens, block_table=w.block_table,
                                          causal=True, out=outs[l], split_tokens=args.split,
                                          two_pass={"auto": None, "two-pass": True, "fused": False}[args.merge])

    def step():
        for l in range(L):
            call(l)

    # An eager step sizes the split-K workspace; the step is then captured in a HIP graph and
    # replayed, as Prism's executor runs decode (engine/executor.py:272-310, :358-360).
    step()
    torch.cuda.synchronize()
    cap = torch.cuda.Stream(device=dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            step()
    torch.cuda.current_stream(dev).wait_stream(cap)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} graph replays)", file=sys.stderr, flush=True)

    # HIP events on the replay stream bracket exactly the K timed steps.
    stream = torch.cuda.current_stream(dev)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    t_end.record(stream)
    torch.cuda.synchronize()
    step_ms = t_start.elapsed_time(t_end) / args.steps
    avg_call_us = step_ms * 1e3 / L
    status = prism_amd.read_status(dev)
    if status:
        print(f"[bench] WARNING: kernel status flags {status}", file=sys.stderr)

    bytes_layer = w.decode_bytes_per_layer()
    bytes_step = bytes_layer * L
    value = bytes_step / (step_ms * 1e-3) / 1e9
    achieved = bytes_layer / (avg_call_us * 1e-6) / 1e9
    print(f"[bench] step {step_ms * 1e3:.1f} us, call avg {avg_call_us:.2f} us, {achieved:.0f} GB/s",
          file=sys.stderr, flush=True)

    if args.copy_probe_mib:
        n_pages = max(1, args.copy_probe_mib * (1 << 20) // (kv.bytes_per_page * 2 * L))
        src = list(range(min(n_pages, kv.max_pages)))
        probe = prism_amd.FlashAttnKVCache(L, kv.num_kv_heads, kv.head_dim, len(src), kv.page_size, str(dev))
        prism_amd.copy_pages(kv, probe, src, list(range(len(src))), None)
        torch.cuda.synchronize()
        print(f"[bench] copy probe: {len(src) * kv.bytes_per_page * 2 * L} bytes read and written by "
              f"copy_pages_kernel", file=sys.stderr, flush=True)

    traffic, traffic_src = profiled_traffic(args, w)
    result = {
        "metric": "paged decode attn HBM GB/s (% of peak) + us/step, Qwen2.5-7B shape b=32",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "us_per_step": round(step_ms * 1e3, 1),
        "tokens_per_s": round(w.batch / (step_ms * 1e-3), 1),
        "pct_of_peak_hbm": round(100 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config3: Qwen2.5-7B paged decode (append + attention), 28 layers, b=32, "
                        "ctx lognormal(1500, 1) in [16, 32768], 2043-page 30 GB pool, 40% churn",
            "batch": w.batch, "layers": L, "n_heads": w.n_heads, "n_kv": kv.num_kv_heads,
            "head_dim": kv.head_dim, "page_size": kv.page_size, "pool_pages": kv.max_pages,
            "sum_ctx": int(w.ctx.sum()), "max_ctx": int(w.ctx.max()), "seed": args.seed,
            "split_tokens": args.split or "auto", "merge": args.merge,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": "one pkv_decode_attn call = decode_lean_kernel (append + balanced paged attention, "
                      "split-K partials) + combine_lean_kernel (merge); HIP events around K graph replays "
                      "of the 28-call step, per call = step / 28",
            "bytes_per_call": bytes_layer,
            "avg_call_us": round(avg_call_us, 3),
        },
    }
    if not args.no_cpu_baseline:
        print(f"[bench] cpu baseline on {args.cpu_layers} layers", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, min(args.cpu_layers, L))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
