"""GPU parity at the long end of what Prism calls: decode past 8k keys and whole-prompt prefill.

* Config 3 draws contexts in [16, 32768] to exercise split-K across long contexts, and Prism's
  eager decode path serves sequences past its 32-page graph limit (engine/executor.py:343,
  :385-386).  A 32767-key sequence spans 1024 tiles of the balanced kernel: about 80 split-K parts
  in config 3's batch and 256 on its own, several 64-tile descriptor windows per range and
  several merge rounds per row.  Tested in config 3's ragged 7B batch (with a 12000-key sequence
  beside it) under both merges, and alone (the B = 1 graph) at the 7B and 14B shapes.
* executor.prefill passes the whole prompt at once, B = 1, up to the 4096-position rotary table
  (engine/executor.py:46, :97-120): a 4096-token prompt at the 7B shape and a 2000-token one at
  14B, no prefix.  The fp64 oracle checks a sample of query rows (page and tile edges, the first
  and last rows, and a seeded draw) of two KV heads; the append is checked bit-exact on every
  head and page, and every output row must be finite.

Every check is the one tests/test_gpu_workloads.py applies to the benchmark workloads
(pkv_testutil.LayerCheck): appended rows bit-exact, every other page of the pool unchanged,
attention within max-abs 1e-2 / mean-abs 1e-3 of the fp64 oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import prism_amd
from pkv_testutil import LayerCheck, free_cached
from prism_amd import workloads

pytestmark = pytest.mark.gpu


def _call(w, l, out, **kw):
    kv = w.kv
    return prism_amd.flash_attn_with_kvcache(w.q[l], kv.k_caches[l], kv.v_caches[l], k=w.k[l], v=w.v[l],
                                             cache_seqlens=w.cache_seqlens, block_table=w.block_table,
                                             causal=True, out=out, **kw)


def _check_layers(w, what, layers, kv_heads=None, rows=None, **kw):
    for l in layers:
        print(f"{what} layer {l}: B={w.batch} s_q={w.s_q} ctx max {int(w.ctx.max())} sum {int(w.ctx.sum())}",
              flush=True)
        chk = LayerCheck(w, l, kv_heads=kv_heads)
        out = torch.full_like(w.q[l], float("nan"))
        _call(w, l, out, **kw)
        chk.check(out, f"{what} layer {l}", rows=rows)
        assert torch.isfinite(out.float()).all(), f"{what}: an output row was not written"
        del chk
        free_cached()


@pytest.mark.parametrize("merge", [None, False, True])
def test_long_sequences_in_the_ragged_batch(gpu, merge):
    # config 3's seed-0 batch with sequence 0 at 32767 cached keys and sequence 1 at 12000
    w = workloads.long_decode(gpu, seed=0, layers=2)
    assert int(w.ctx[0]) == 32767 and int(w.ctx[1]) == 12000 and w.batch == 32
    _check_layers(w, f"long decode merge={merge}", [0, 1], two_pass=merge)
    del w
    free_cached()


@pytest.mark.parametrize("shape", ["7B", "14B"])
@pytest.mark.parametrize("merge", [None, True])
def test_one_sequence_at_32767_keys(gpu, shape, merge):
    # the B = 1 decode graph at the top of the range: 256 split-K parts of one sequence
    w = workloads.long_decode(gpu, seed=1, layers=1, shape=shape, batch=1)
    assert int(w.ctx[0]) == 32767
    _check_layers(w, f"B=1 32767 keys {shape} merge={merge}", [0], two_pass=merge)
    del w
    free_cached()


def _row_sample(s_q: int, seed: int) -> np.ndarray:
    edges = [0, 1, 31, 32, 33, 127, 128, 255, 256, 257, 511, 512, s_q // 2, s_q - 33, s_q - 32, s_q - 2, s_q - 1]
    draw = np.random.default_rng(seed).choice(s_q, size=96, replace=False)
    return np.unique(np.clip(np.concatenate([edges, draw]), 0, s_q - 1))


@pytest.mark.parametrize("shape,prompt,kv_heads", [("7B", 4096, [0, 3]), ("14B", 2000, [2, 7])])
def test_whole_prompt_prefill(gpu, shape, prompt, kv_heads):
    w = workloads.prompt_prefill(gpu, seed=2, layers=1, shape=shape, prompt=prompt)
    assert w.batch == 1 and w.s_q == prompt and int(w.ctx[0]) == 0
    _check_layers(w, f"prefill {shape} {prompt}", [0], kv_heads=kv_heads, rows=_row_sample(prompt, prompt))
    del w
    free_cached()
