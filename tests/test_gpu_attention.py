"""GPU parity of the append + attention kernels against the CPU oracle (through the C ABI).

Bit-exact for the appended cache rows (the whole pools are compared), and the north_star bf16
tolerance (max-abs <= 1e-2, mean-abs <= 1e-3 against the fp64 oracle rounded to bf16) for outputs.
"""
import numpy as np
import pytest
import torch

import prism_amd
from oracle import paged_attention as pa
from pkv_testutil import assert_attn_close, make_paged_case

pytestmark = pytest.mark.gpu


def _poison_stale_slots(cpu, dev, ctx):
    """NaN into every cache slot that holds no cached key: the slots past each sequence's keys
    (the appended rows included) and the pages no sequence lists.  Whole tiles are copied into
    LDS, so those bytes reach the kernels; none may reach an output."""
    kc, bt = cpu["k_cache"], cpu["block_table"].numpy()
    num_pages, P = kc.shape[:2]
    live = np.zeros((num_pages, P), dtype=bool)
    for b, c in enumerate(ctx):
        for t in range(int(c)):
            live[bt[b, t // P], t % P] = True
    stale = torch.from_numpy(~live)
    for name in ("k_cache", "v_cache"):
        cpu[name][stale] = float("nan")
        dev[name].copy_(cpu[name].to(dev[name].device))


def _run_and_check(gpu, *, batch, ctx, page_size, n_kv, n_heads, head_dim, s_q, causal=True, append=True,
                   split_tokens=0, seed=0, kernel="auto", extra_cols=0, two_pass=None, grid=0, what="",
                   poison=False):
    cpu, dev = make_paged_case(gpu, batch=batch, ctx=ctx, page_size=page_size, n_kv=n_kv, n_heads=n_heads,
                               head_dim=head_dim, s_q=s_q, seed=seed, extra_cols=extra_cols)
    if poison:
        _poison_stale_slots(cpu, dev, ctx)
    print(f"case {what} B={batch} ctx={list(ctx)[:6]} P={page_size} kv={n_kv} h={n_heads} hd={head_dim} "
          f"s_q={s_q} causal={causal} append={append} split={split_tokens} kernel={kernel} two_pass={two_pass} "
          f"grid={grid}",
          flush=True)
    kw = dict(cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"], causal=causal)
    k = dev["k"] if append else None
    v = dev["v"] if append else None
    # NaN-filled output: a row the kernels fail to write cannot pass on stale values of an
    # earlier call that the caching allocator hands back
    out = torch.full_like(dev["q"], float("nan"))
    if kernel == "prefill":
        out = prism_amd.prefill_attention(dev["q"], dev["k_cache"], dev["v_cache"], k, v, out=out, **kw)
    else:
        out = prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], k, v,
                                                split_tokens=split_tokens, two_pass=two_pass,
                                                kernel=kernel, grid=grid, out=out, **kw)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(
        cpu["q"], cpu["k_cache"], cpu["v_cache"], cpu["k"] if append else None, cpu["v"] if append else None,
        cache_seqlens=cpu["cache_seqlens"], block_table=cpu["block_table"], causal=causal)
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb), "K cache not bit-exact after append"
    assert np.array_equal(pa.bf16_bits(dev["v_cache"]), vb), "V cache not bit-exact after append"
    assert_attn_close(out, ref, what)
    return out


DECODE_CASES = [
    # (batch, ctx, page, n_kv, n_heads, hd, s_q)
    (4, [1, 300, 1023, 512], 256, 2, 14, 64, 1),          # config-1 shape
    (3, [0, 255, 256], 256, 4, 28, 128, 1),                # page boundaries, empty cache
    (5, [31, 32, 33, 63, 64], 16, 4, 28, 128, 1),           # 16-token pages
    (2, [700, 5], 32, 8, 40, 128, 1),                      # 14B shape
    (2, [100, 1000], 64, 4, 4, 128, 1),                    # g = 1
    (3, [517, 2, 90], 256, 4, 28, 128, 5),                 # verify, R = 35
    (2, [40, 300], 256, 2, 16, 64, 8),                     # R = 64
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 4, 28, 128, 1),  # ragged, multi-split
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[f"d{i}" for i in range(len(DECODE_CASES))])
def test_decode_append_attention(gpu, case):
    B, ctx, P, n_kv, nh, hd, s_q = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                   what=f"decode{case}")


STALE_NAN_CASES = [
    # (batch, ctx, page, n_kv, n_heads, hd, s_q, kernel): every sequence ends inside a tile
    (4, [1, 300, 1023, 517], 256, 4, 28, 128, 1, "auto"),     # 7B decode, balanced kernel
    (3, [517, 2, 90], 256, 4, 28, 128, 5, "auto"),            # verify rows
    (2, [700, 5], 32, 8, 40, 128, 1, "auto"),                 # 14B, two head groups
    (4, [1, 300, 1023, 517], 256, 2, 14, 64, 1, "auto"),      # head_dim 64
    (3, [517, 2, 90], 256, 4, 28, 128, 1, "heads"),           # per-head kernel
    (2, [100, 1000], 64, 4, 4, 128, 1, "auto"),               # g = 1
    (2, [200, 37], 256, 4, 28, 128, 64, "prefill"),           # prefill chunk
]


@pytest.mark.parametrize("case", STALE_NAN_CASES, ids=[f"n{i}" for i in range(len(STALE_NAN_CASES))])
def test_stale_nan_slots_never_reach_the_output(gpu, case):
    B, ctx, P, n_kv, nh, hd, s_q, kernel = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                   kernel=kernel, poison=True, what=f"stale-nan{case}")


FEWER_KEYS_CASES = [
    # (batch, ctx, page, n_kv, n_heads, hd, s_q, kernel): no append, causal, fewer cached keys than
    # queries, so the first rows see no key while later rows of the same wave see some
    (2, [21, 80], 32, 2, 10, 128, 256, "auto"),   # prefill, LDS kernel
    (2, [21, 80], 64, 2, 14, 64, 128, "auto"),    # prefill, head_dim 64 kernel
    (3, [2, 4, 0], 256, 4, 28, 128, 5, "auto"),   # verify rows, balanced kernel
    (3, [2, 4, 0], 256, 4, 28, 128, 5, "heads"),  # verify rows, per-head kernel
    (2, [3, 1], 256, 1, 7, 128, 2, "auto"),       # a one-head shard
]


@pytest.mark.parametrize("case", FEWER_KEYS_CASES, ids=[f"f{i}" for i in range(len(FEWER_KEYS_CASES))])
def test_rows_that_see_no_key_beside_rows_that_do(gpu, case):
    """Rows with no visible key get zeros although other rows of their wave see keys: such a row
    is part of the wave's decision to mask a tile (a negative limit), not left out of it like the
    padding rows past the real ones."""
    B, ctx, P, n_kv, nh, hd, s_q, kernel = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q, append=False,
                   kernel=kernel, what=f"fewer-keys{case}")


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("s_q", [3, 8])
def test_per_head_two_pass_merge_above_16_rows(gpu, hd, s_q):
    """The per-head kernel's second-launch merge at more than 16 query rows per KV head: its
    512 threads cover 32 rows at head_dim 64, of which a workgroup owns 16."""
    _run_and_check(gpu, batch=6, ctx=[0, 0, 2356, 1300, 0, 2014], page_size=128, n_kv=2, n_heads=14, head_dim=hd,
                   s_q=s_q, split_tokens=64, kernel="heads", two_pass=True, what=f"heads-two-pass hd={hd} s_q={s_q}")


@pytest.mark.parametrize("split", [32, 64, 256, 1 << 20])
def test_decode_split_invariance(gpu, split):
    _run_and_check(gpu, batch=3, ctx=[1500, 33, 700], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   split_tokens=split, what=f"split{split}")


def test_split_merge_rearms_across_calls_and_matches_two_pass(gpu):
    # consecutive calls of different shapes share one workspace: the in-kernel merge counters
    # must be back at zero after every call, and the two-pass merge must agree
    shapes = [(2, [5000, 40]), (6, [3000, 17, 4100, 800, 1, 2500]), (3, [9000, 600, 1]), (1, [33])]
    for i, (B, ctx) in enumerate(shapes * 2):
        for two_pass in (False, True):
            _run_and_check(gpu, batch=B, ctx=ctx, page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                           split_tokens=256, seed=i, two_pass=two_pass, what=f"rearm{i}")


# The balanced kernel (head_dim 128, 4 KV heads, pages >= 32, <= 64 query rows per KV head):
# grids from one workgroup (every tile in one range, several 64-tile descriptor windows) to more
# workgroups than tiles, ranges holding many short sequences, new rows straddling a tile edge;
# 1 to 4 MFMA row tiles per wave (R = 7 .. 63: decode and speculative verify).
LEAN_CASES = [
    # (batch, ctx, page, n_heads, s_q, grid, append)
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 28, 1, 0, True),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 28, 1, 1, True),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 28, 1, 7, True),
    (40, [(i * 37) % 300 for i in range(40)], 32, 28, 1, 5, True),
    (3, [31, 64, 0], 64, 28, 2, 3, True),
    (2, [61, 700], 256, 16, 4, 4, True),
    (4, [0, 5, 300, 33], 256, 28, 1, 2, False),
    (5, [10, 20, 30, 40, 50], 256, 28, 1, 64, True),
    (70, [(i * 53) % 900 for i in range(70)], 256, 28, 1, 0, True),
    (70, [(i * 53) % 900 for i in range(70)], 256, 28, 1, 9, True),
    (3, [517, 2, 90], 256, 28, 5, 0, True),                 # verify R = 35: 3 row tiles
    (3, [517, 2, 90], 256, 28, 5, 5, True),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 28, 4, 7, True),  # R = 28: 2 row tiles
    (4, [700, 33, 1, 2000], 256, 28, 9, 6, True),           # R = 63: 4 row tiles, appends straddle tiles
    (40, [(i * 37) % 300 for i in range(40)], 32, 28, 5, 5, True),
    (2, [61, 700], 256, 16, 8, 3, False),                   # g = 4, R = 32, no append
    (1, [0], 256, 28, 6, 1, True),                          # empty cache, R = 42
    (64, [2027 + (i * 97) % 1024 for i in range(64)], 256, 28, 5, 0, True),  # config-5 shape
]


@pytest.mark.parametrize("merge", ["two-pass", "in-launch"])
@pytest.mark.parametrize("case", LEAN_CASES, ids=[f"l{i}" for i in range(len(LEAN_CASES))])
def test_balanced_decode_kernel(gpu, case, merge):
    B, ctx, P, nh, s_q, grid, append = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=4, n_heads=nh, head_dim=128, s_q=s_q,
                   append=append, grid=grid, two_pass=merge == "two-pass", seed=len(ctx) + grid,
                   what=f"lean{case[:1] + case[2:]}-{merge}")


# The balanced kernel with KV heads in groups of four (8 and 12 KV heads: Qwen2.5-14B, and a
# larger GQA model), decode and verify row counts, both merges: a range may straddle two head groups.
GROUP_CASES = [
    # (batch, ctx, page, n_kv, n_heads, s_q, grid)
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 8, 40, 1, 0),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 8, 40, 1, 7),
    (3, [517, 2, 90], 256, 8, 40, 5, 0),                      # R = 25: two row tiles
    (40, [(i * 37) % 300 for i in range(40)], 32, 8, 40, 1, 5),
    (5, [10, 2000, 30, 40, 50], 64, 12, 48, 2, 3),           # three head groups, R = 8
    (1, [0], 256, 8, 64, 1, 1),                               # empty cache, g = 8
]


@pytest.mark.parametrize("merge", ["two-pass", "in-launch"])
@pytest.mark.parametrize("case", GROUP_CASES, ids=[f"g{i}" for i in range(len(GROUP_CASES))])
def test_balanced_kernel_head_groups(gpu, case, merge):
    B, ctx, P, n_kv, nh, s_q, grid = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=128, s_q=s_q,
                   grid=grid, two_pass=merge == "two-pass", seed=len(ctx) + grid, what=f"groups{case}-{merge}")


# The balanced kernel's narrower geometries: 2 or 1 KV heads of head_dim 128 per group (64- and
# 128-token tiles, 2 or 4 phase waves per head whose softmax states merge through LDS), head_dim 64
# in groups of 4 or 2 (two 32-key subtiles per wave; 64- and 128-token tiles): Qwen2.5-0.5B, 7B on
# 4 and 2 tensor-parallel ranks, 3 and 6 KV heads (several groups), verify row counts whose phase
# merge needs two rounds (R = 35 with 1 KV head, R = 64 with 2), pages exactly one tile long.
GEOM_CASES = [
    # (batch, ctx, page, n_kv, n_heads, hd, s_q, grid, append)
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 2, 14, 64, 1, 0, True),      # 0.5B
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 2, 14, 64, 1, 7, True),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 1, 7, 128, 1, 0, True),      # 7B, TP 4
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 1, 7, 128, 1, 5, True),
    (6, [3000, 17, 4100, 800, 1, 2500], 256, 2, 14, 128, 1, 9, True),     # 7B, TP 2
    (40, [(i * 37) % 300 for i in range(40)], 128, 1, 7, 128, 1, 5, True),
    (40, [(i * 37) % 300 for i in range(40)], 64, 2, 14, 128, 1, 3, True),
    (40, [(i * 37) % 300 for i in range(40)], 128, 2, 14, 64, 1, 11, True),
    (70, [(i * 53) % 900 for i in range(70)], 256, 8, 40, 128, 1, 0, True),  # 14B, over 64 sequences
    (5, [10, 2000, 130, 40, 250], 128, 3, 21, 128, 1, 3, True),           # 3 groups of 1
    (5, [10, 2000, 130, 40, 250], 64, 6, 24, 128, 2, 4, True),            # 3 groups of 2
    (5, [10, 2000, 130, 40, 250], 64, 4, 16, 64, 1, 2, True),             # hd 64, one group of 4
    (5, [10, 2000, 130, 40, 250], 128, 6, 18, 64, 3, 6, True),            # hd 64, 3 groups of 2
    (3, [517, 2, 90], 256, 1, 7, 128, 5, 0, True),                        # verify R = 35
    (3, [517, 2, 90], 256, 1, 7, 128, 5, 4, True),
    (4, [700, 33, 1, 2000], 256, 1, 7, 128, 9, 6, True),                  # R = 63, appends straddle tiles
    (2, [61, 700], 256, 2, 16, 128, 8, 3, True),                          # R = 64
    (2, [61, 700], 256, 2, 16, 64, 8, 3, False),                          # hd 64, R = 64, no append
    (4, [0, 5, 300, 33], 256, 1, 7, 128, 1, 2, False),
    (1, [0], 256, 2, 14, 64, 1, 1, True),                                 # empty cache
    (64, [2027 + (i * 97) % 1024 for i in range(64)], 256, 1, 7, 128, 5, 0, True),
]


@pytest.mark.parametrize("merge", ["two-pass", "in-launch"])
@pytest.mark.parametrize("case", GEOM_CASES, ids=[f"x{i}" for i in range(len(GEOM_CASES))])
def test_balanced_kernel_narrow_geometries(gpu, case, merge):
    B, ctx, P, n_kv, nh, hd, s_q, grid, append = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                   append=append, grid=grid, two_pass=merge == "two-pass", seed=len(ctx) + grid + n_kv,
                   what=f"geom{case[:1] + case[2:]}-{merge}")


# The sequence-aligned split (decode rows of 2-8 sequences at 4 KV heads per group, any batch with
# phase waves): per = ceil(T / grid) tiles per range, ceil(t_b / per) ranges per sequence when they
# fit the grid, else the plain split.  After a 1-row append the 7B cases hold t = [3, 2, 1, 4]
# tiles: grid 6 fits exactly (per 2: 2 + 1 + 1 + 2 ranges), grid 5 misses by one (plain split),
# grid 8 leaves two workgroups idle; eight 2048-key sequences fill all 256 ranges of two tiles
# (every sequence a whole number of ranges).
ALIGNED_CASES = [
    # (batch, ctx, n_kv, n_heads, hd, grid)
    (4, [95, 63, 30, 126], 4, 28, 128, 6),
    (4, [95, 63, 30, 126], 4, 28, 128, 5),
    (4, [95, 63, 30, 126], 4, 28, 128, 8),
    (8, [2047] * 8, 4, 28, 128, 0),
    (7, [3000, 17, 4100, 800, 1, 2500, 64], 4, 28, 128, 0),
    (5, [10, 2000, 130, 40, 250], 1, 7, 128, 0),               # 7B, TP 4 (4 phase waves)
    (12, [(i * 311) % 1500 for i in range(12)], 2, 14, 64, 0),  # 0.5B (2 phase waves)
    (3, [127, 128, 129], 2, 14, 128, 4),                        # 7B, TP 2
    (70, [(i * 53) % 900 for i in range(70)], 2, 14, 64, 0),   # 0.5B past 64 sequences (4-chunk scan)
    (70, [(i * 53) % 900 for i in range(70)], 1, 7, 128, 0),   # TP 4 past 64 sequences
]


@pytest.mark.parametrize("merge", ["two-pass", "in-launch"])
@pytest.mark.parametrize("case", ALIGNED_CASES, ids=[f"a{i}" for i in range(len(ALIGNED_CASES))])
def test_sequence_aligned_split(gpu, case, merge):
    B, ctx, n_kv, nh, hd, grid = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=256, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=1,
                   grid=grid, two_pass=merge == "two-pass", seed=B + grid + n_kv,
                   what=f"aligned{case}-{merge}")


def test_balanced_in_launch_merge_rearms_across_calls(gpu):
    # the balanced kernel's per-(sequence, head) arrival counters must be back at zero after every
    # call: consecutive calls of different shapes and grids share one workspace, with sequences
    # split into up to ~20 parts, and each result must match the oracle (and so the two-pass merge)
    shapes = [(6, [3000, 17, 4100, 800, 1, 2500], 7), (2, [5000, 40], 16), (1, [33], 3),
              (40, [(i * 37) % 300 for i in range(40)], 5), (3, [9000, 600, 1], 21)]
    for i, (B, ctx, grid) in enumerate(shapes * 2):
        for two_pass in (False, True):
            _run_and_check(gpu, batch=B, ctx=ctx, page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                           grid=grid, seed=i, two_pass=two_pass, what=f"lean-rearm{i}")


@pytest.mark.parametrize("case", [DECODE_CASES[1], DECODE_CASES[4], DECODE_CASES[5], DECODE_CASES[7]],
                         ids=["d1", "d4", "d5", "d7"])
def test_per_head_kernel_on_balanced_shapes(gpu, case):
    # the same shapes through the per-(sequence, head, split) kernel, both merges
    B, ctx, P, n_kv, nh, hd, s_q = case
    for two_pass in (False, True):
        _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                       kernel="heads", two_pass=two_pass, what=f"heads{case}")


@pytest.mark.parametrize("kernel", ["auto", "heads"])
@pytest.mark.parametrize("two_pass", [True, False])
def test_verify_part_holding_only_keys_a_row_cannot_see(gpu, kernel, two_pass):
    # speculative verify (s_q > 1) with a split-K part that starts past some query rows' last
    # visible key: those rows keep a -inf running max while the other rows of their wave rescale
    # (a part per 32-token tile on the balanced kernel's default grid, 512-token splits per head)
    for i, (ctx, s_q, append) in enumerate([([259], 4, False), ([513, 1027], 4, False), ([1025], 2, False),
                                            ([1023, 252], 4, True), ([509, 1019, 3], 5, True)]):
        _run_and_check(gpu, batch=len(ctx), ctx=ctx, page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=s_q,
                       append=append, kernel=kernel, two_pass=two_pass, seed=i, what=f"verify-edge{i}")


def test_batch_beyond_balanced_limit(gpu):
    # more than 256 sequences: the per-head kernel serves the call
    ctx = [(i * 29) % 200 for i in range(300)]
    _run_and_check(gpu, batch=300, ctx=ctx, page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   what="b300")


def test_decode_without_append_and_non_causal(gpu):
    _run_and_check(gpu, batch=3, ctx=[50, 1, 600], page_size=32, n_kv=2, n_heads=14, head_dim=64, s_q=1,
                   append=False, what="noappend")
    _run_and_check(gpu, batch=2, ctx=[77, 400], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=3,
                   causal=False, what="noncausal")
    _run_and_check(gpu, batch=3, ctx=[77, 400, 5], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=5,
                   causal=False, grid=4, what="noncausal-verify")


def test_decode_extra_block_table_columns(gpu):
    # a wider table than needed (stale columns are never read)
    _run_and_check(gpu, batch=2, ctx=[10, 300], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   extra_cols=5, what="widetable")


PREFILL_CASES = [
    (2, [0, 700], 256, 8, 40, 128, 128),
    (3, [0, 33, 290], 32, 4, 28, 128, 37),
    (2, [5, 1000], 256, 2, 14, 64, 100),
    (1, [0], 256, 4, 4, 128, 300),
    (3, [2100, 4000, 1], 256, 8, 40, 128, 64),  # 14B shape, long tile loops through the 4-stage pipeline
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[f"p{i}" for i in range(len(PREFILL_CASES))])
def test_prefill_append_attention(gpu, case):
    B, ctx, P, n_kv, nh, hd, s_q = case
    _run_and_check(gpu, batch=B, ctx=ctx, page_size=P, n_kv=n_kv, n_heads=nh, head_dim=hd, s_q=s_q,
                   what=f"prefill{case}")


def test_prefill_kernel_on_small_queries_matches(gpu):
    # the row-parallel kernel on a decode-sized problem (cross-checks both kernels' indexing)
    _run_and_check(gpu, batch=3, ctx=[900, 4, 256], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   kernel="prefill", what="prefill-s1")
    _run_and_check(gpu, batch=2, ctx=[90, 513], page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=5,
                   kernel="prefill", what="prefill-s5")


def test_strided_qkv_views_like_prism(gpu):
    # engine/executor.py:256-260 passes q/k/v as views into the fused QKV projection output
    torch.manual_seed(0)
    B, nh, n_kv, hd, P = 4, 28, 4, 128, 256
    qs, kvs = nh * hd, n_kv * hd
    cpu, dev = make_paged_case(gpu, batch=B, ctx=[10, 200, 256, 1000], page_size=P, n_kv=n_kv, n_heads=nh,
                               head_dim=hd, s_q=1)
    qkv = torch.randn(B, 1, qs + 2 * kvs, device=gpu).to(torch.bfloat16)
    q = qkv[:, :, :qs].view(B, 1, nh, hd)
    k = qkv[:, :, qs:qs + kvs].view(B, 1, n_kv, hd)
    v = qkv[:, :, qs + kvs:].view(B, 1, n_kv, hd)
    assert not k.is_contiguous()
    out = prism_amd.flash_attn_with_kvcache(q, dev["k_cache"], dev["v_cache"], k=k, v=v,
                                            cache_seqlens=dev["cache_seqlens"], block_table=dev["block_table"],
                                            causal=True)
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(q.cpu(), cpu["k_cache"], cpu["v_cache"], k.cpu(), v.cpu(),
                                                 cache_seqlens=cpu["cache_seqlens"],
                                                 block_table=cpu["block_table"], causal=True)
    assert np.array_equal(pa.bf16_bits(dev["k_cache"]), kb)
    assert_attn_close(out, ref, "strided")


def test_config1_workload_end_to_end(gpu):
    from prism_amd import workloads

    w = workloads.config1(gpu, seed=0)
    kv = w.kv
    k0, v0 = kv.k_caches[0].cpu(), kv.v_caches[0].cpu()
    out = prism_amd.flash_attn_with_kvcache(w.q[0], kv.k_caches[0], kv.v_caches[0], k=w.k[0], v=w.v[0],
                                            cache_seqlens=w.cache_seqlens, block_table=w.block_table, causal=True)
    torch.cuda.synchronize()
    ref, kb, vb = pa.flash_attn_with_kvcache_ref(w.q[0].cpu(), k0, v0, w.k[0].cpu(), w.v[0].cpu(),
                                                 cache_seqlens=w.cache_seqlens.cpu(),
                                                 block_table=w.block_table.cpu(), causal=True)
    assert np.array_equal(pa.bf16_bits(kv.k_caches[0]), kb)
    assert np.array_equal(pa.bf16_bits(kv.v_caches[0]), vb)
    assert_attn_close(out, ref, "config1")


def test_bad_page_id_is_flagged_not_faulted(gpu):
    # a block-table entry outside the pool is skipped and reported through the status word
    cpu, dev = make_paged_case(gpu, batch=2, ctx=[40, 300], page_size=256, n_kv=4, n_heads=28, head_dim=128,
                               s_q=1)
    bt = dev["block_table"].clone()
    bt[1, 0] = 10_000
    st = torch.zeros(1, dtype=torch.int32, device=gpu)
    prism_amd.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"], dev["k"], dev["v"],
                                      cache_seqlens=dev["cache_seqlens"], block_table=bt, causal=True, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) & 1


def test_balanced_kernel_at_its_batch_limit_and_on_empty_caches(gpu):
    # 256 sequences fill all four 64-sequence chunks of the balanced kernel's in-register scan;
    # a batch of empty caches makes every range a run of one-tile sequences (only the new row)
    rng = np.random.default_rng(3)
    ctx = [int(c) for c in rng.integers(0, 120, size=256)]
    _run_and_check(gpu, batch=256, ctx=ctx, page_size=32, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   what="balanced B=256")
    _run_and_check(gpu, batch=256, ctx=ctx, page_size=32, n_kv=4, n_heads=28, head_dim=128, s_q=2,
                   what="balanced B=256 verify")
    _run_and_check(gpu, batch=8, ctx=[0] * 8, page_size=256, n_kv=4, n_heads=28, head_dim=128, s_q=1,
                   what="all empty")


@pytest.mark.parametrize("batch,ctx,s_q", [
    (64, [(i * 37) % 300 for i in range(64)], 8),   # the largest batch ranked by length
    (6, [200, 200, 200, 35, 200, 0], 24),           # equal lengths: ties ranked by index
    (70, [(i * 53) % 260 for i in range(70)], 4),   # above 64 sequences: launch order
])
def test_prefill_launch_order_covers_every_item(gpu, batch, ctx, s_q):
    # the prefill grid is walked heaviest first; every (sequence, KV head, row block) item must
    # still be computed exactly once (the NaN-filled output catches a missed one)
    _run_and_check(gpu, batch=batch, ctx=ctx, page_size=32, n_kv=4, n_heads=28, head_dim=128, s_q=s_q,
                   kernel="prefill", what=f"prefill order B={batch}")
    _run_and_check(gpu, batch=batch, ctx=ctx, page_size=16, n_kv=2, n_heads=14, head_dim=64, s_q=s_q,
                   kernel="prefill", what=f"prefill order hd64 B={batch}")
