"""Replays of operation traces recorded from the reference allocator and prefix cache.

tests/golden/allocator_traces.json holds seeded random sequences of new / new-with-prefix /
_ensure_capacity / update_seqlens / free / free_model_sequences / free_all / build_block_table /
queries / transfer_sequence on engine/kv_cache.py's FlashAttnKVCache, each op with its arguments,
its result or exception class, and the whole observable state after it (free list order,
seq_pages, seq_len, seq_owner, pages_used, pages_free).  prefix_traces.json does the same for
engine/prefix_cache.py's PrefixCache (results, per-page refcounts, LRU order).  Both were written by
tests/golden/make_allocator_golden.py.

The oracle restatements (oracle/kv_state.py) must reproduce every trace.  The product drop-ins must
reproduce every allocator trace in which no page is listed by two sequences (share=False) and every
prefix-cache trace: with shared pages the product deliberately keeps pages that are still in use
off the free list, where the reference returns them (engine/kv_cache.py:87-89); those semantics
are tested in test_host_state.py.
"""
import json
from pathlib import Path

import pytest

from oracle.kv_state import KVAllocatorRef, PrefixCacheRef

GOLDEN = Path(__file__).resolve().parent / "golden"
ALLOC = json.loads((GOLDEN / "allocator_traces.json").read_text())["traces"]
PREFIX = json.loads((GOLDEN / "prefix_traces.json").read_text())["traces"]


def _raises_like(exc: BaseException, name: str) -> bool:
    return any(c.__name__ == name for c in type(exc).__mro__)


def _state(kv) -> dict:
    return {
        "free_pages": list(kv.free_pages),
        "seq_pages": {str(k): list(v) for k, v in kv.seq_pages.items()},
        "seq_len": {str(k): v for k, v in kv.seq_len.items()},
        "seq_owner": {str(k): v for k, v in kv.seq_owner.items()},
        "pages_used": kv.pages_used,
        "pages_free": kv.pages_free,
    }


class _ProductAlloc:
    """prism_amd.kv_cache.FlashAttnKVCache on the CPU; page copies recorded instead of launched."""

    def __init__(self, max_pages, page_size, monkeypatch):
        import prism_amd.kv_cache as kvm

        self.copies = []

        def cpu_copy(src, dst, src_ids, dst_ids, fill, staged=None):
            self.copies.append((list(src_ids), list(dst_ids), fill))
            for s, d in zip(src_ids, dst_ids):
                dst.k_pool[:, d] = src.k_pool[:, s]
                dst.v_pool[:, d] = src.v_pool[:, s]

        monkeypatch.setattr(kvm, "copy_pages", cpu_copy)
        self.kv = kvm.FlashAttnKVCache(1, 1, 8, max_pages, page_size, "cpu")
        self.kv2 = kvm.FlashAttnKVCache(1, 1, 8, max_pages, page_size, "cpu")

    def table(self, sids):
        bt, sl = self.kv.build_block_table(sids)
        return ([bt[i, :len(self.kv.seq_pages[s])].tolist() for i, s in enumerate(sids)], sl.tolist(),
                int(bt.shape[1]))

    def transfer(self, sid, dst):
        n = self.kv.transfer_sequence(sid, self.kv2, dst)
        if n:
            src_ids, dst_ids, fill = self.copies[-1]
            assert fill is None
            assert src_ids == self.kv.seq_pages[sid][:n] and dst_ids == self.kv2.seq_pages[dst][:n]
        return n


class _OracleAlloc:
    def __init__(self, max_pages, page_size, monkeypatch=None):
        self.kv = KVAllocatorRef(max_pages, page_size)
        self.kv2 = KVAllocatorRef(max_pages, page_size)

    def table(self, sids):
        rows, sl = self.kv.block_table(sids)
        return rows, sl, max(1, max(len(r) for r in rows))

    def transfer(self, sid, dst):
        n, pairs = self.kv.transfer_sequence(sid, self.kv2, dst)
        assert pairs == list(zip(self.kv.seq_pages.get(sid, [])[:n], self.kv2.seq_pages.get(dst, [])[:n]))
        return n


def _replay_alloc(trace, impl):
    kv = impl.kv
    for i, rec in enumerate(trace["ops"]):
        op, args = rec["op"], rec.get("args", [])
        where = f"seed {trace['seed']} op {i} {op}{args}"
        try:
            result = None
            if op == "new":
                kv.new_sequence(args[0], args[1])
            elif op == "new_prefix":
                kv.new_sequence(args[0], args[1], prefix_pages=args[2], prefix_len=args[3])
            elif op == "ensure":
                kv._ensure_capacity(args[0], args[1])
            elif op == "update":
                kv.update_seqlens(args[0], args[1])
            elif op == "free":
                kv.free_sequence(args[0])
            elif op == "free_model":
                kv.free_model_sequences(args[0])
            elif op == "free_all":
                kv.free_all()
            elif op == "table":
                rows, sl, width = impl.table(args[0])
                result = {"rows": rows, "seqlens": sl, "width": width}
            elif op == "query":
                owner, n, sid = args
                result = {"sequences_for_model": kv.sequences_for_model(owner),
                          "memory_used_by_model": kv.memory_used_by_model(owner),
                          "has_capacity": kv.has_capacity(n), "get_seq_len": kv.get_seq_len(sid)}
            elif op == "transfer":
                sid, dst = args
                n = impl.transfer(sid, dst)
                result = {"pages": n, "dst_pages": list(impl.kv2.seq_pages.get(dst, [])),
                          "dst_len": impl.kv2.seq_len.get(dst), "target": _state(impl.kv2)}
                impl.kv2.free_sequence(dst)
            else:
                raise AssertionError(f"unknown op {op}")
        except Exception as exc:  # noqa: BLE001 - compared with the recorded exception class
            assert "raises" in rec, f"{where}: unexpected {type(exc).__name__}: {exc}"
            assert _raises_like(exc, rec["raises"]), f"{where}: raised {type(exc).__name__}, want {rec['raises']}"
        else:
            assert "raises" not in rec, f"{where}: expected {rec['raises']}"
            if "result" in rec:
                assert result == rec["result"], f"{where}: result {result} != {rec['result']}"
        assert _state(kv) == rec["state"], f"{where}: state differs"


@pytest.mark.parametrize("trace", ALLOC, ids=[f"seed{t['seed']}{'-share' if t['share'] else ''}" for t in ALLOC])
def test_oracle_allocator_reproduces_reference_trace(trace):
    _replay_alloc(trace, _OracleAlloc(trace["max_pages"], trace["page_size"]))


@pytest.mark.parametrize("trace", [t for t in ALLOC if not t["share"]],
                         ids=[f"seed{t['seed']}" for t in ALLOC if not t["share"]])
def test_product_allocator_reproduces_reference_trace(trace, monkeypatch):
    _replay_alloc(trace, _ProductAlloc(trace["max_pages"], trace["page_size"], monkeypatch))


def test_traces_cover_the_allocator_surface():
    ops = {o["op"] for t in ALLOC for o in t["ops"]}
    assert ops >= {"new", "new_prefix", "ensure", "update", "free", "free_model", "free_all", "table", "query",
                   "transfer"}
    raised = {o.get("raises") for t in ALLOC for o in t["ops"]}
    assert {"RuntimeError", "IndexError"} <= raised   # both out-of-pages paths are in the traces


def _replay_prefix(trace, pc, lru):
    for i, rec in enumerate(trace["ops"]):
        op, args = rec["op"], rec["args"]
        where = f"seed {trace['seed']} op {i} {op}"
        result = None
        if op == "lookup":
            pages, n = pc.lookup(args[0], args[1])
            result = [list(pages), n]
        elif op == "store":
            pc.store(args[0], args[1], args[2])
        elif op == "ref":
            pc.ref_pages(args[0])
        elif op == "unref":
            result = pc.unref_pages(args[0])
        elif op == "is_cached":
            result = pc.is_cached_page(args[0])
        elif op == "evict":
            result = pc.evict_lru(args[0])
        if "result" in rec:
            assert result == rec["result"], f"{where}: {result} != {rec['result']}"
        assert {str(k): v for k, v in sorted(pc._page_refs.items())} == rec["refs"], f"{where}: refcounts"
        assert lru() == rec["lru_pages"], f"{where}: LRU order"
        assert pc.num_cached_pages == rec["num_cached_pages"], where


@pytest.mark.parametrize("trace", PREFIX, ids=[f"seed{t['seed']}" for t in PREFIX])
def test_oracle_prefix_cache_reproduces_reference_trace(trace):
    pc = PrefixCacheRef(trace["page_size"])
    _replay_prefix(trace, pc, pc.lru_pages)


@pytest.mark.parametrize("trace", PREFIX, ids=[f"seed{t['seed']}" for t in PREFIX])
def test_product_prefix_cache_reproduces_reference_trace(trace):
    from prism_amd.prefix_cache import PrefixCache

    pc = PrefixCache(None, page_size=trace["page_size"])
    _replay_prefix(trace, pc, lambda: [e.page_id for e in pc._cache.values()])
