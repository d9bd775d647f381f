"""DecodeBatch host planning (CPU): the update packet, applied by a restatement of
pkv_table_update, must leave exactly the block table and lengths build_block_table would give,
and send only what changed.  Also pins the oracle's element-by-element restatement of the
reference's per-step graph refill (engine/kv_cache.py:147-151, engine/executor.py:345-356)."""
import random

import numpy as np
import torch

from oracle.kv_state import KVAllocatorRef, graph_staging_elementwise
from prism_amd import DecodeBatch, FlashAttnKVCache


def _apply(packet, n_len, n_ent, bt, sl, num_pages):
    """pkv_table_update restated: lengths, then (row, column, page) entries; bad ones skipped."""
    flagged = False
    for k in range(n_len):
        row, length = packet[2 * k], packet[2 * k + 1]
        if 0 <= row < sl.shape[0] and length >= 0:
            sl[row] = length
        else:
            flagged = True
    e = packet[2 * n_len:].reshape(-1, 3)
    assert e.shape[0] == n_ent
    for row, col, page in e:
        if 0 <= row < bt.shape[0] and 0 <= col < bt.shape[1] and 0 <= page < num_pages:
            bt[row, col] = page
        else:
            flagged = True
    return flagged


def _check_rows(db, kv, bt, sl, seq_ids, gb):
    for i, sid in enumerate(seq_ids):
        pages = kv.seq_pages[sid]
        assert list(bt[i, :len(pages)]) == pages, f"row {i} (sequence {sid})"
        assert sl[i] == kv.seq_len[sid]
    for i in range(len(seq_ids), gb):
        assert bt[i, 0] == db.null_page and sl[i] == 0, f"padded row {i}"


def test_plan_rebuilds_tables_and_sends_only_changes():
    rng = random.Random(7)
    kv = FlashAttnKVCache(1, 1, 8, 300, 16, "cpu")
    db = DecodeBatch(kv, max_batch=12, max_blocks=64)
    assert db.null_page not in kv.free_pages
    bt = np.full((12, 64), db.null_page, dtype=np.int32)
    sl = np.zeros(12, dtype=np.int32)
    live: list[int] = []
    next_id = 0
    for _ in range(300):
        # batch churn: finish some sequences, start others, shuffle the rows now and then
        if live and rng.random() < 0.15:
            sid = live.pop(rng.randrange(len(live)))
            kv.free_sequence(sid)
        while len(live) < rng.randint(1, 10) and kv.pages_free > 20:
            kv.new_sequence(next_id)
            kv.seq_len[next_id] = 0
            kv._ensure_capacity(next_id, rng.randint(0, 200))
            kv.seq_len[next_id] = len(kv.seq_pages[next_id]) * 16 - rng.randint(0, 15)
            live.append(next_id)
            next_id += 1
        if rng.random() < 0.1:
            rng.shuffle(live)
        gb = rng.randint(len(live), 12)
        n_new = rng.choice([1, 1, 1, 5])
        for sid in live:
            kv._ensure_capacity(sid, kv.seq_len[sid] + n_new)
        packet, n_len, n_ent = db.plan(list(live), gb)
        assert not _apply(packet, n_len, n_ent, bt, sl, kv.max_pages)
        _check_rows(db, kv, bt, sl, live, gb)
        sent_pages = {sid: list(kv.seq_pages[sid]) for sid in live}
        kv.update_seqlens(list(live), n_new)
        # steady state: growing the same batch sends exactly the new pages and the lengths
        for sid in live:
            kv._ensure_capacity(sid, kv.seq_len[sid] + 1)
        new_pages = sum(len(kv.seq_pages[s]) - len(sent_pages[s]) for s in live)
        packet, n_len, n_ent = db.plan(list(live), gb)
        assert n_ent == new_pages, (n_ent, new_pages)
        assert n_len == len(live)  # every length moved by n_new
        assert not _apply(packet, n_len, n_ent, bt, sl, kv.max_pages)
        _check_rows(db, kv, bt, sl, live, gb)


def test_null_page_survives_free_all_and_is_stable():
    kv = FlashAttnKVCache(1, 1, 8, 10, 16, "cpu")
    p = kv.reserve_null_page()
    assert p == 0 and kv.reserve_null_page() == p  # LIFO: the first page handed out
    kv.new_sequence(1)
    kv.free_all()
    assert p not in kv.free_pages and len(kv.free_pages) == 9
    for s in range(9):
        kv.new_sequence(s)
    assert all(p not in pages for pages in kv.seq_pages.values())


def test_plan_rejects_bad_batches():
    kv = FlashAttnKVCache(1, 1, 8, 40, 16, "cpu")
    db = DecodeBatch(kv, max_batch=4, max_blocks=3)
    kv.new_sequence(1)
    kv.seq_len[1] = 0
    import pytest
    with pytest.raises(ValueError):
        db.plan([1, 1], 4)
    with pytest.raises(ValueError):
        db.plan([1], 5)
    kv._ensure_capacity(1, 16 * 4)
    with pytest.raises(RuntimeError):
        db.plan([1], 2)


def test_elementwise_staging_restatement_matches_block_table():
    rng = random.Random(3)
    ref = KVAllocatorRef(200, 16)
    ids = []
    for s in range(6):
        ref.new_sequence(s)
        ref._ensure_capacity(s, rng.randint(1, 300))
        ref.seq_len[s] = rng.randint(0, len(ref.seq_pages[s]) * 16 - 1)
        ids.append(s)
    rows, lens = ref.block_table(ids)
    bt = torch.zeros(8, 32, dtype=torch.int32)
    sl = torch.zeros(8, dtype=torch.int32)
    gbt = torch.full((8, 32), -5, dtype=torch.int32)
    gsl = torch.full((8,), -5, dtype=torch.int32)
    cos = torch.arange(400 * 4, dtype=torch.float32).reshape(400, 4)
    sin = -cos
    gcos = torch.zeros(8, 1, 4)
    gsin = torch.zeros(8, 1, 4)
    graph_staging_elementwise(bt, sl, gbt, gsl, ref.seq_pages, ref.seq_len, ids, cos, sin, gcos, gsin)
    for i, r in enumerate(rows):
        assert gbt[i, :len(r)].tolist() == r and int(gsl[i]) == lens[i]
        assert torch.equal(gcos[i, 0], cos[lens[i]]) and torch.equal(gsin[i, 0], sin[lens[i]])
    assert int(gbt[6:].abs().sum()) == 0 and int(gsl[6:].abs().sum()) == 0  # rows past B zeroed
