"""Pins of the row layout the node's store reads (oracle.staged_step, derive, store_commit,
written_ranges), on the CPU.

The store stays the reference's (store/src/storage.rs); what must hold is that the staging bytes
this build writes land in the store's tables where the store puts them. Pinned by:

* the store's own literal case (store/tests/service.rs:26-68,176-262): two tables staged in one
  file, then an overwrite, a padding row and a new slot; written ranges and row bytes as the
  Rust test asserts them;
* end to end on the mirror's layout: a cache gathered into [L, H, cap, 2, d] (the oracle's
  gather, which the HIP kernel equals byte for byte), described as the mirror describes it
  (core/everserve/state/mirror.py:778-800), committed table by table, restored from the written
  ranges into another cache at other head slots (core/everserve/state/mirror.py:916-937):
  every restored row equals its source row;
* a run-by-run copy against a row-by-row copy (the store copies runs of consecutive slots,
  storage.rs:916-943), and the incremental restore's since_step filter (storage.rs:430-451).
"""

import numpy as np
import torch

import oracle
from tests.cases import bits, caches, strides_of

ROW = 16  # shape [2, 4] of bfloat16


def stage_fill(slots, fills):
    return np.concatenate([np.full(ROW, f, dtype=np.uint8) for f in fills])


def test_the_stores_own_case():
    tables, written = {}, {}
    # stage_two: tables 0 and 1 (layers 0 and 1, one head, table stride 1), slots [3, 9]
    two = np.concatenate([stage_fill([3, 9], [1, 1]), stage_fill([3, 9], [2, 2])])
    step10 = {"stage": "s0", "base_offset": 0, "layer_stride": 2 * ROW, "head_stride": 0,
              "layers": [0, 1], "heads": [0], "table_stride": 1, "slots": [3, 9],
              "dtype": "bfloat16", "shape": [2, 4]}
    oracle.store_commit(two, step10, tables, 64, written, 10)
    # stage: layer 0 only, slots [9, -1, 12] filled [1, 7, 1]: an overwrite, padding, a new slot
    step11 = {"stage": "s2", "base_offset": 0, "layer_stride": 0, "head_stride": 0,
              "layers": [0], "heads": [0], "table_stride": 1, "slots": [9, -1, 12],
              "dtype": "bfloat16", "shape": [2, 4]}
    oracle.store_commit(stage_fill([9, -1, 12], [1, 7, 1]), step11, tables, 64, written, 11)

    assert sorted(tables) == [0, 1]
    assert oracle.written_ranges(written[0]) == [(3, 1), (9, 1), (12, 1)]
    assert oracle.written_ranges(written[1]) == [(3, 1), (9, 1)]
    t0 = tables[0].reshape(64, ROW)
    assert len(tables[0]) == 64 * ROW
    assert (t0[[3, 9, 12]] == 1).all()
    assert (t0[[0, 4]] == 0).all()
    assert (tables[1].reshape(64, ROW)[3] == 2).all()
    # restore rows total: 3 + 2 written slots
    assert sum(c for _, c in oracle.written_ranges(written[0]) + oracle.written_ranges(written[1])) == 5
    # since step 10, only the slots the step-11 commit wrote
    assert oracle.written_ranges(written[0], since_step=10) == [(9, 1), (12, 1)]
    assert oracle.written_ranges(written[1], since_step=10) == []


def test_derive_names_tables_by_layer_and_head_slot():
    step = oracle.staged_step("st", [0, 2], [5, 1], capacity=8, head_dim=4, elem=2,
                              slots=[1, 2], dtype="bfloat16")
    row = 2 * 4 * 2
    assert step["layer_stride"] == 2 * 8 * row and step["head_stride"] == 8 * row
    assert oracle.derive(step) == [
        (5, 0), (1, 8 * row),                              # layer 0: head slots 5 then 1
        (2005, 2 * 2 * 8 * row), (2001, 2 * 2 * 8 * row + 8 * row),  # layer 2
    ]


def test_staged_rows_land_in_the_store_and_restore_at_other_head_slots():
    src = caches("kv_first", 8, torch.bfloat16, n_layers=3, nb=7, seed=13)
    _, _, bs, d = oracle.recognise(src[0].shape)
    slots = [5, -1, 17, 0, 27, 26, 25, 3]
    held = [0, 2]
    cap = 16
    staged = oracle.gather_rows(src, slots, held, cap, d, bs, strides_of(src[0]), 2)
    step = oracle.staged_step("stage-1-1.rows", [0, 1, 2], held, cap, d, 2, slots, "bfloat16")
    tables, written = {}, {}
    num_slots = 7 * bs
    oracle.store_commit(staged.view(np.uint8).reshape(-1), step, tables, num_slots, written, 1)
    assert sorted(tables) == [0, 2, 1000, 1002, 2000, 2002]

    # the restore: per table, the written rows by range, into head slot moves[theirs]
    moves = {0: 1, 2: 0}
    dst = [torch.zeros_like(t) for t in src]
    for table, rows in tables.items():
        layer, head = divmod(table, oracle.HEAD_STRIDE)
        idx = np.concatenate([np.arange(s, s + c) for s, c in oracle.written_ranges(written[table])])
        table_rows = rows.view(np.uint16).reshape(num_slots, 2, d)[idx]  # [n, 2, d]
        one = np.zeros((1, 1, len(idx), 2, d), dtype=np.uint16)
        one[0, 0] = table_rows
        oracle.scatter_rows([dst[layer]], idx, [moves[head]], one, len(idx), d, bs,
                            strides_of(dst[layer]), 2)
    live = sorted({s for s in slots if s >= 0})
    want = oracle.gather_rows(src, live, held, len(live), d, bs, strides_of(src[0]), 2)
    got = oracle.gather_rows(dst, live, [moves[h] for h in held], len(live), d, bs,
                             strides_of(dst[0]), 2)
    assert np.array_equal(got, want)
    # the padding row was skipped: slot 0 holds slot 0's own row, once
    assert oracle.written_ranges(written[0]) == [(0, 1), (3, 1), (5, 1), (17, 1), (25, 3)]


def test_the_run_copy_equals_a_row_by_row_copy():
    rng = np.random.default_rng(3)
    slots = [4, 5, 6, -1, 9, 10, 2, 3, -1, 30]
    stage = rng.integers(0, 255, size=len(slots) * ROW, dtype=np.uint8)
    step = {"stage": "s", "base_offset": 0, "layer_stride": 0, "head_stride": 0, "layers": [0],
            "heads": [0], "table_stride": 1, "slots": slots, "dtype": "bfloat16", "shape": [2, 4]}
    tables, written = {}, {}
    oracle.store_commit(stage, step, tables, 32, written, 7)
    want = np.zeros(32 * ROW, dtype=np.uint8)
    for i, s in enumerate(slots):
        if s >= 0:
            want[s * ROW:(s + 1) * ROW] = stage[i * ROW:(i + 1) * ROW]
    assert np.array_equal(tables[0], want)
    assert oracle.written_ranges(written[0]) == [(2, 5), (9, 2), (30, 1)]


def test_a_slot_outside_the_store_is_refused():
    step = {"stage": "s", "base_offset": 0, "layer_stride": 0, "head_stride": 0, "layers": [0],
            "heads": [0], "table_stride": 1, "slots": [64], "dtype": "bfloat16", "shape": [2, 4]}
    try:
        oracle.store_commit(np.zeros(ROW, np.uint8), step, {}, 64, {}, 1)
    except ValueError as e:
        assert "outside" in str(e)
    else:
        raise AssertionError("slot 64 of 64 accepted")


def test_gathered_bytes_are_the_cache_bytes():
    # the staging bytes for (layer, head index, t) are the cache row of that slot, K then V
    src = caches("blocks_first", 8, torch.float16, n_layers=2, seed=4)
    _, _, bs, d = oracle.recognise(src[0].shape)
    staged = oracle.gather_rows(src, [9], [1], 1, d, bs, strides_of(src[0]), 2)
    b, o = divmod(9, bs)
    for layer in range(2):
        k = bits(src[layer][b, 0, o, 1])
        v = bits(src[layer][b, 1, o, 1])
        assert np.array_equal(staged[layer, 0, 0], np.stack([k, v]))
