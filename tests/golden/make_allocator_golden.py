"""Record golden traces of the reference allocator and prefix cache (run in the build container).

Imports engine/kv_cache.py and engine/prefix_cache.py from /root/reference by file path (their only
dependency is torch; the caches are built on the CPU with tiny shapes), drives them with seeded
random operation sequences, and writes every operation's arguments, result (or exception class) and
the resulting observable state to tests/golden/allocator_traces.json and prefix_traces.json.

These pin what only the reference's own code fixes exactly: the LIFO free-list order after
arbitrary interleavings of new/ensure/free/free_all (engine/kv_cache.py:49, :79-103, :121), the
block-table rows (:123-153), transfer_sequence's page pairing (:174-209), and PrefixCache's LRU,
refcount and eviction behaviour over long traces (engine/prefix_cache.py:30-127).

Nothing from the reference is copied into the repository; only the recorded vectors are.
Usage:  python tests/golden/make_allocator_golden.py [/root/reference]
"""
from __future__ import annotations

import importlib.util
import json
import random
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def _load(ref_root: Path, name: str):
    spec = importlib.util.spec_from_file_location(f"ref_{name}", ref_root / "engine" / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _state(kv) -> dict:
    return {
        "free_pages": list(kv.free_pages),
        "seq_pages": {str(k): list(v) for k, v in kv.seq_pages.items()},
        "seq_len": {str(k): v for k, v in kv.seq_len.items()},
        "seq_owner": {str(k): v for k, v in kv.seq_owner.items()},
        "pages_used": kv.pages_used,
        "pages_free": kv.pages_free,
    }


def allocator_trace(kv_mod, seed: int, n_ops: int, max_pages: int, page_size: int, share: bool) -> dict:
    """share=False never lists one page in two sequences (the product must match these exactly);
    share=True adds new_sequence(prefix_pages=...) on a live sequence's pages, where the reference
    frees pages still in use (only the oracle restatement is checked against those)."""
    import torch

    rng = random.Random(seed)
    kv = kv_mod.FlashAttnKVCache(1, 1, 8, max_pages, page_size, "cpu", torch.bfloat16)
    kv2 = kv_mod.FlashAttnKVCache(1, 1, 8, max_pages, page_size, "cpu", torch.bfloat16)
    owners = ["a", "b", "c"]
    next_id = 0
    ops = []
    for _ in range(n_ops):
        live = list(kv.seq_pages)
        kind = rng.choices(
            ["new", "new_prefix", "ensure", "update", "free", "free_model", "free_all", "table",
             "query", "transfer"],
            weights=[14, 4 if share else 0, 20, 10, 10, 3, 1, 8, 5, 3])[0]
        rec = {"op": kind}
        try:
            if kind == "new":
                sid = next_id
                next_id += 1
                owner = rng.choice(owners)
                rec["args"] = [sid, owner]
                kv.new_sequence(sid, owner)
            elif kind == "new_prefix" and live:
                src = rng.choice(live)
                npref = rng.randint(1, len(kv.seq_pages[src]))
                prefix = list(kv.seq_pages[src][:npref])
                sid = next_id
                next_id += 1
                owner = rng.choice(owners)
                plen = npref * page_size
                rec["args"] = [sid, owner, prefix, plen]
                kv.new_sequence(sid, owner, prefix_pages=prefix, prefix_len=plen)
            elif kind == "ensure" and live:
                sid = rng.choice(live)
                total = kv.seq_len[sid] + rng.randint(0, 3 * page_size)
                rec["args"] = [sid, total]
                kv._ensure_capacity(sid, total)
            elif kind == "update" and live:
                sids = rng.sample(live, rng.randint(1, min(3, len(live))))
                if rng.random() < 0.5:
                    n = rng.randint(0, 2 * page_size)
                else:
                    n = [rng.randint(0, 2 * page_size) for _ in sids]
                rec["args"] = [sids, n]
                kv.update_seqlens(sids, n)
            elif kind == "free" and live:
                sid = rng.choice(live + [10_000])
                rec["args"] = [sid]
                kv.free_sequence(sid)
            elif kind == "free_model":
                owner = rng.choice(owners)
                rec["args"] = [owner]
                kv.free_model_sequences(owner)
            elif kind == "free_all":
                rec["args"] = []
                kv.free_all()
            elif kind == "table" and live:
                sids = rng.sample(live, rng.randint(1, min(4, len(live))))
                bt, sl = kv.build_block_table(sids)
                rec["args"] = [sids]
                rec["result"] = {"rows": [bt[i, :len(kv.seq_pages[s])].tolist() for i, s in enumerate(sids)],
                                 "seqlens": sl.tolist(), "width": int(bt.shape[1])}
            elif kind == "query":
                owner = rng.choice(owners)
                n = rng.randint(0, 4)
                sid = rng.choice(live) if live else 10_000
                rec["args"] = [owner, n, sid]
                rec["result"] = {"sequences_for_model": kv.sequences_for_model(owner),
                                 "memory_used_by_model": kv.memory_used_by_model(owner),
                                 "has_capacity": kv.has_capacity(n),
                                 "get_seq_len": kv.get_seq_len(sid)}
            elif kind == "transfer" and live:
                sid = rng.choice(live)
                dst = 50_000 + next_id
                next_id += 1
                rec["args"] = [sid, dst]
                n = kv.transfer_sequence(sid, kv2, dst)
                rec["result"] = {"pages": n, "dst_pages": list(kv2.seq_pages.get(dst, [])),
                                 "dst_len": kv2.seq_len.get(dst), "target": _state(kv2)}
                kv2.free_sequence(dst)
            else:
                continue
        except Exception as exc:  # noqa: BLE001 - the exception class is part of the trace
            rec["raises"] = type(exc).__name__
        rec["state"] = _state(kv)
        ops.append(rec)
    return {"seed": seed, "max_pages": max_pages, "page_size": page_size, "share": share, "ops": ops}


def prefix_trace(pc_mod, seed: int, n_ops: int, page_size: int) -> dict:
    rng = random.Random(seed)
    pc = pc_mod.PrefixCache(None, page_size=page_size)
    vocab = 3
    prompts: list[list[int]] = []
    models = ["m0", "m1"]
    next_page = 0
    ops = []

    def prompt():
        if prompts and rng.random() < 0.6:
            base = rng.choice(prompts)
            cut = rng.randint(0, len(base))
            p = base[:cut] + [rng.randrange(vocab) for _ in range(rng.randint(0, 3 * page_size))]
        else:
            p = [rng.randrange(vocab) for _ in range(rng.randint(0, 4 * page_size))]
        prompts.append(p)
        return p

    for _ in range(n_ops):
        kind = rng.choices(["lookup", "store", "ref", "unref", "is_cached", "evict"],
                           weights=[30, 25, 10, 12, 10, 8])[0]
        rec = {"op": kind}
        if kind == "lookup":
            p = prompt()
            m = rng.choice(models)
            rec["args"] = [p, m]
            pages, n = pc.lookup(p, m)
            rec["result"] = [list(pages), n]
        elif kind == "store":
            p = prompt()
            m = rng.choice(models)
            npages = rng.randint(0, len(p) // page_size + 1)
            pages = list(range(next_page, next_page + npages))
            next_page += npages
            rec["args"] = [p, pages, m]
            pc.store(p, pages, m)
        elif kind == "ref":
            pages = [rng.randrange(max(1, next_page)) for _ in range(rng.randint(0, 4))]
            rec["args"] = [pages]
            pc.ref_pages(pages)
        elif kind == "unref":
            pages = [rng.randrange(max(1, next_page)) for _ in range(rng.randint(0, 4))]
            rec["args"] = [pages]
            rec["result"] = pc.unref_pages(pages)
        elif kind == "is_cached":
            page = rng.randrange(max(1, next_page))
            rec["args"] = [page]
            rec["result"] = pc.is_cached_page(page)
        elif kind == "evict":
            n = rng.randint(0, 3)
            rec["args"] = [n]
            rec["result"] = pc.evict_lru(n)
        rec["refs"] = {str(k): v for k, v in sorted(pc._page_refs.items())}
        rec["lru_pages"] = [e.page_id for e in pc._cache.values()]
        rec["num_cached_pages"] = pc.num_cached_pages
        ops.append(rec)
    return {"seed": seed, "page_size": page_size, "ops": ops}


def main(ref_root: str = "/root/reference") -> None:
    root = Path(ref_root)
    kv_mod = _load(root, "kv_cache")
    pc_mod = _load(root, "prefix_cache")
    alloc = [allocator_trace(kv_mod, seed, 300, mp, ps, share)
             for seed, mp, ps, share in [(1, 24, 16, False), (2, 12, 16, False), (3, 40, 8, False),
                                         (4, 6, 32, False), (5, 24, 16, True), (6, 10, 16, True)]]
    prefix = [prefix_trace(pc_mod, seed, 300, ps) for seed, ps in [(11, 4), (12, 8), (13, 2)]]
    (HERE / "allocator_traces.json").write_text(json.dumps({"traces": alloc}, separators=(",", ":")))
    (HERE / "prefix_traces.json").write_text(json.dumps({"traces": prefix}, separators=(",", ":")))
    print("wrote", HERE / "allocator_traces.json", HERE / "prefix_traces.json")


if __name__ == "__main__":
    main(*sys.argv[1:])
