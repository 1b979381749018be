"""The restore path end to end on the GPU: a rank's caches gathered into staging rows, committed
into the store's tables (the store's own commit, restated in the oracle), then restored into
another rank's caches at other head slots by everserve_amd.state.restore.Restorer, chunk by chunk.

Checked byte for byte: every written slot's rows in the new head slot equal the source rows, the
other head slots are untouched (core/tests/test_kvcopy.py:162-189 states the same round trip for
the torch path).
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state.restore import Restorer, Table
from tests.cases import bits, caches, strides_of

pytestmark = pytest.mark.gpu


def commit(src, slots, held, cap, steps=1):
    """The store's tables after committing `slots` of every layer and held head of `src`."""
    _, nb, bs, d = oracle.recognise(src[0].shape)
    e = src[0].element_size()
    staged = oracle.gather_rows(src, slots, held, cap, d, bs, strides_of(src[0]), e)
    step = oracle.staged_step("s", list(range(len(src))), held, cap, d, e, slots,
                              "bfloat16" if e == 2 else "uint8")
    tables, written = {}, {}
    oracle.store_commit(staged.view(np.uint8).reshape(-1), step, tables, nb * bs, written, steps)
    return tables, written


@pytest.mark.parametrize("layout", ["kv_first", "blocks_first", "combined"])
@pytest.mark.parametrize("chunk_bytes", [64, 1 << 20])
def test_restored_rows_land_in_the_new_head_slots(ext, layout, chunk_bytes):
    nb, bs, h, d = 40, 4, 3, 8
    src = caches(layout, d, torch.bfloat16, n_layers=3, nb=nb, bs=bs, h=h, seed=31)
    slots = [5, -1, 17, 0, 27, 26, 25, 3, 100, 101, 102, 159, 50]
    held = [0, 2]
    tables, written = commit(src, slots, held, cap=16)
    moves = {0: 1, 2: 0}  # the unit in their head slot 0 goes to our 1, theirs 2 to our 0
    dst = [torch.zeros_like(t).cuda() for t in src]
    r = Restorer(ext, dst, chunk_bytes=chunk_bytes, threads=4)
    rows = r.restore([Table(t, rows, oracle.written_ranges(written[t])) for t, rows in tables.items()],
                     moves)
    live = sorted({s for s in slots if s >= 0})
    assert rows == len(live) * len(src) * len(held)
    want = oracle.gather_rows(src, live, held, len(live), d, bs, strides_of(src[0]), 2)
    cpu = [t.cpu() for t in dst]
    got = oracle.gather_rows(cpu, live, [moves[x] for x in held], len(live), d, bs,
                             strides_of(cpu[0]), 2)
    assert np.array_equal(got, want)
    # head slot 2 of ours was never a target: still zero
    untouched = oracle.gather_rows(cpu, list(range(nb * bs)), [2], nb * bs, d, bs,
                                   strides_of(cpu[0]), 2)
    assert not untouched.any()


def test_an_incremental_restore_copies_only_the_later_slots(ext):
    src = caches("kv_first", 8, torch.bfloat16, n_layers=2, nb=16, bs=4, h=2, seed=41)
    tables, written = {}, {}
    _, _, bs, d = oracle.recognise(src[0].shape)
    for step, slots in ((1, [0, 1, 2, 3]), (2, [9, 10])):
        staged = oracle.gather_rows(src, slots, [0, 1], 8, d, bs, strides_of(src[0]), 2)
        desc = oracle.staged_step("s", [0, 1], [0, 1], 8, d, 2, slots, "bfloat16")
        oracle.store_commit(staged.view(np.uint8).reshape(-1), desc, tables, 64, written, step)
    dst = [torch.zeros_like(t).cuda() for t in src]
    Restorer(ext, dst).restore(
        [Table(t, rows, oracle.written_ranges(written[t], since_step=1)) for t, rows in tables.items()],
        {0: 0, 1: 1})
    cpu = [t.cpu() for t in dst]
    assert np.array_equal(
        oracle.gather_rows(cpu, [9, 10], [0, 1], 2, d, bs, strides_of(cpu[0]), 2),
        oracle.gather_rows(src, [9, 10], [0, 1], 2, d, bs, strides_of(src[0]), 2))
    assert not oracle.gather_rows(cpu, [0, 1, 2, 3], [0, 1], 4, d, bs, strides_of(cpu[0]), 2).any()


def test_tables_opened_from_files_and_heads_not_mapped_are_skipped(ext, tmp_path):
    nb, bs, h, d = 24, 4, 3, 8
    src = caches("combined", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=51)
    slots = [7, 8, 9, 40, 41, 95]
    tables, written = commit(src, slots, [0, 1, 2], cap=8)
    opened = []
    for t, rows in tables.items():
        path = tmp_path / f"table{t}.rows"
        rows.tofile(path)
        opened.append(Table.open(t, str(path), oracle.written_ranges(written[t])))
    dst = [torch.zeros_like(t).cuda() for t in src]
    moves = {0: 2, 2: 1}  # head slot 1's tables are not this rank's: skipped
    got_rows = Restorer(ext, dst, chunk_bytes=3 * 32).restore(opened, moves)
    assert got_rows == len(slots) * len(src) * len(moves)
    cpu = [t.cpu() for t in dst]
    for theirs, ours in moves.items():
        assert np.array_equal(
            oracle.gather_rows(cpu, slots, [ours], 8, d, bs, strides_of(cpu[0]), 2),
            oracle.gather_rows(src, slots, [theirs], 8, d, bs, strides_of(src[0]), 2))
    assert not oracle.gather_rows(cpu, list(range(nb * bs)), [0], nb * bs, d, bs,
                                  strides_of(cpu[0]), 2).any()


def test_ranges_outside_a_table_and_partial_rows_are_refused(ext):
    src = caches("kv_first", 8, torch.bfloat16, n_layers=1, nb=8, bs=4, h=2, seed=61)
    dst = [torch.zeros_like(t).cuda() for t in src]
    r = Restorer(ext, dst)
    rows = np.zeros(32 * 32, dtype=np.uint8)  # 32 slots of 32-byte rows
    with pytest.raises(ValueError, match="outside"):
        r.restore([Table(0, rows, [(30, 3)])], {0: 0})
    with pytest.raises(ValueError, match="outside"):
        r.restore([Table(1, rows, [(-1, 2)])], {1: 1})
    with pytest.raises(ValueError, match="whole number"):
        r.restore([Table(0, rows[:-5], [(0, 1)])], {0: 0})
    assert not dst[0].any()


@pytest.mark.parametrize("piece_rows", [16, 5, 1])
def test_many_chunks_on_a_side_stream_twice_with_the_same_buffers(ext, piece_rows):
    """Chunks inside one slot range (slot ids made on the device) and across several (slot ids
    copied), each reaching the device in pieces (a chunk whole, pieces that do not divide it,
    one row at a time), the copies on the Restorer's stream and the scatters on the caller's
    side stream, and a second restore that reuses the buffers and events of the first."""
    nb, bs, h, d = 64, 4, 2, 64
    src = caches("kv_first", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=71)
    rng = np.random.default_rng(71)
    slots = sorted(rng.choice(nb * bs, size=150, replace=False).tolist() + list(range(40, 90)))
    slots = sorted(set(slots))
    tables, written = commit(src, slots, [0, 1], cap=len(slots))
    ranges = {t: oracle.written_ranges(written[t]) for t in tables}
    assert any(c > 40 for _, c in ranges[0])  # a range longer than a chunk
    dst = [torch.zeros_like(t).cuda() for t in src]
    row_bytes = 2 * d * 2
    # 16 rows of each of the group's 2 tables a chunk
    r = Restorer(ext, dst, chunk_bytes=2 * 16 * row_bytes, threads=2,
                 piece_bytes=2 * piece_rows * row_bytes)
    side = torch.cuda.Stream()
    want = oracle.gather_rows(src, slots, [0, 1], len(slots), d, bs, strides_of(src[0]), 2)
    for _ in range(2):
        for t in dst:
            t.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            rows = r.restore([Table(t, tb, ranges[t]) for t, tb in tables.items()], {0: 1, 1: 0})
        assert rows == len(slots) * len(src) * 2
        cpu = [t.cpu() for t in dst]
        got = oracle.gather_rows(cpu, slots, [1, 0], len(slots), d, bs, strides_of(cpu[0]), 2)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("chunk_bytes", [1, 32, 3 * 32])
def test_a_chunk_smaller_than_a_row_of_every_table_still_holds_one(ext, chunk_bytes):
    """A chunk carries at least one row of each of a group's tables: with a chunk of one row or
    less and 4 head tables a group, the buffers hold 4 rows, and the restore equals the
    oracle's rows."""
    nb, bs, h, d = 8, 4, 4, 8
    src = caches("kv_first", d, torch.bfloat16, n_layers=1, nb=nb, bs=bs, h=h, seed=83)
    slots = [0, 1, 2, 5, 9, 10, 30]
    tables, written = commit(src, slots, [0, 1, 2, 3], cap=8)
    dst = [torch.zeros_like(t).cuda() for t in src]
    r = Restorer(ext, dst, chunk_bytes=chunk_bytes, piece_bytes=1)
    moves = {0: 2, 1: 3, 2: 0, 3: 1}
    rows = r.restore([Table(t, tb, oracle.written_ranges(written[t])) for t, tb in tables.items()],
                     moves)
    assert rows == len(slots) * 4
    assert r.timing["launches"] == len(slots)  # a chunk of one row of each of the 4 tables
    cpu = dst[0].cpu()
    got = oracle.gather_rows([cpu], slots, [2, 3, 0, 1], 8, d, bs, strides_of(cpu), 2)
    want = oracle.gather_rows([src[0]], slots, [0, 1, 2, 3], 8, d, bs, strides_of(src[0]), 2)
    assert np.array_equal(got, want)


def test_two_threads_restoring_through_one_restorer(ext):
    """Two threads restore through one Restorer at once (different tables, different head slots,
    small chunks so each restore runs many): the restores take turns on its buffers, and both
    land."""
    import threading

    nb, bs, h, d = 64, 4, 4, 16
    src = caches("kv_first", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=87)
    slots = list(range(0, 200, 3))
    tables, written = commit(src, slots, [0, 1, 2, 3], cap=128)
    dst = [torch.zeros_like(t).cuda() for t in src]
    r = Restorer(ext, dst, chunk_bytes=4 * 8 * 2 * d * 2, piece_bytes=2 * 8 * 2 * d * 2)
    mine = {0: [t for t in tables if t % 1000 in (0, 1)], 1: [t for t in tables if t % 1000 in (2, 3)]}
    moves = {0: 3, 1: 2, 2: 1, 3: 0}
    errors = []

    def run(k):
        try:
            for _ in range(3):
                r.restore([Table(t, tables[t], oracle.written_ranges(written[t])) for t in mine[k]],
                          moves)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(k,)) for k in (0, 1)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for li in range(2):
        cpu = dst[li].cpu()
        got = oracle.gather_rows([cpu], slots, [3, 2, 1, 0], 128, d, bs, strides_of(cpu), 2)
        want = oracle.gather_rows([src[li]], slots, [0, 1, 2, 3], 128, d, bs,
                                  strides_of(src[li]), 2)
        assert np.array_equal(got, want), li


def test_empty_written_ranges_are_passed_over(ext):
    """A table's list of written ranges may hold empty ones: they write nothing and the rest
    lands; a table whose ranges are all empty is skipped, as one with none is."""
    nb, bs, h, d = 8, 4, 2, 8
    src = caches("kv_first", d, torch.bfloat16, n_layers=1, nb=nb, bs=bs, h=h, seed=85)
    slots = [0, 1, 2, 9, 10]
    tables, written = commit(src, slots, [0, 1], cap=8)
    dst = [torch.zeros_like(t).cuda() for t in src]
    with_empty = [(0, 3), (5, 0), (9, 2), (20, 0)]
    rows = Restorer(ext, dst).restore([Table(0, tables[0], with_empty),
                                       Table(1, tables[1], [(4, 0)])], {0: 1, 1: 0})
    assert rows == len(slots)
    cpu = dst[0].cpu()
    got = oracle.gather_rows([cpu], slots, [1], 8, d, bs, strides_of(cpu), 2)
    want = oracle.gather_rows([src[0]], slots, [0], 8, d, bs, strides_of(src[0]), 2)
    assert np.array_equal(got, want)
    assert not cpu[:, :, :, 0].any()  # head slot 0 (table 1's) stays untouched


def test_tables_that_do_not_fit_this_ranks_cache_are_refused_before_anything_is_written(ext):
    """A table of a layer this rank lacks, a head slot past the layer's heads, a written range
    past the cache's slots (a table of a larger cache), rows of another size, or two tables into
    one head slot: each refuses the whole restore, and nothing of the good tables is written."""
    src = caches("kv_first", 8, torch.bfloat16, n_layers=2, nb=8, bs=4, h=2, seed=62)
    tables, written = commit(src, [0, 1, 5, 9], [0, 1], cap=8)
    good = [Table(t, rows, oracle.written_ranges(written[t])) for t, rows in tables.items()]
    dst = [torch.zeros_like(t).cuda() for t in src]
    r = Restorer(ext, dst)
    big = np.zeros(64 * 32, dtype=np.uint8)  # a table of 64 slots; this cache has 32
    cases = [
        (good + [Table(2000, tables[0], [(0, 2)])], {0: 0, 1: 1}, "layer 2"),
        (good, {0: 0, 1: 2}, "head slot 2 outside"),
        (good[:1] + [Table(1, big, [(30, 3)])], {0: 0, 1: 1}, "past this cache"),
        (good[:1] + [Table(1, tables[0][:-8], [(0, 1)])], {0: 0, 1: 1}, "whole number"),
        (good[:1] + [Table(1, tables[0].reshape(-1, 16), [(0, 1)])], {0: 0, 1: 1},
         "whole number"),
        (good + [Table(1, tables[0], [(0, 1)])], {0: 1, 1: 1}, "already restored"),
    ]
    for extra, moves, match in cases:
        with pytest.raises(ValueError, match=match):
            r.restore(extra, moves)
        torch.cuda.synchronize()
        assert not any(t.any() for t in dst), match


def test_each_layer_keeps_its_own_strides(ext):
    """Layer 1 is a view with other strides than layer 0 (the same shape, stored in another
    dimension order): the restore addresses each layer with its own five strides."""
    nb, bs, h, d = 16, 4, 2, 8
    src = caches("kv_first", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=63)
    slots = [3, 4, 5, 17, 40, 63]
    tables, written = commit(src, slots, [0, 1], cap=8)
    dst0 = torch.zeros_like(src[0]).cuda()
    order = [4, 3, 2, 1, 0]
    dst1 = torch.zeros_like(src[1]).cuda().permute(order).contiguous().permute(order)
    assert dst1.stride() != dst0.stride()
    Restorer(ext, [dst0, dst1]).restore(
        [Table(t, rows, oracle.written_ranges(written[t])) for t, rows in tables.items()],
        {0: 1, 1: 0})
    for li, dst in enumerate((dst0, dst1)):
        cpu = dst.cpu()
        assert np.array_equal(
            oracle.gather_rows([cpu], slots, [1, 0], 8, d, bs, strides_of(cpu), 2),
            oracle.gather_rows([src[li]], slots, [0, 1], 8, d, bs, strides_of(src[li]), 2)), li


def test_a_layers_heads_are_scattered_in_one_launch_per_chunk(ext):
    """Tables of one layer with the same written ranges form one group: the chunks carry all the
    group's heads, so the launch count is the chunk count of one table, not of each, and the
    pieces a chunk is copied in add no launch."""
    nb, bs, h, d = 32, 4, 4, 8
    src = caches("blocks_first", d, torch.bfloat16, n_layers=3, nb=nb, bs=bs, h=h, seed=64)
    slots = list(range(0, 100))
    tables, written = commit(src, slots, [0, 1, 2, 3], cap=128)
    dst = [torch.zeros_like(t).cuda() for t in src]
    per_chunk_rows = 10
    r = Restorer(ext, dst, chunk_bytes=4 * per_chunk_rows * 2 * d * 2,
                 piece_bytes=4 * 3 * 2 * d * 2)
    moves = {0: 3, 1: 2, 2: 1, 3: 0}
    rows = r.restore([Table(t, tb, oracle.written_ranges(written[t])) for t, tb in tables.items()],
                     moves)
    assert rows == 100 * 3 * 4
    assert r.timing["launches"] == 3 * 10
    cpu = [t.cpu() for t in dst]
    assert np.array_equal(
        oracle.gather_rows(cpu, slots, [3, 2, 1, 0], 128, d, bs, strides_of(cpu[0]), 2),
        oracle.gather_rows(src, slots, [0, 1, 2, 3], 128, d, bs, strides_of(src[0]), 2))


@pytest.mark.parametrize("seed", range(12))
def test_random_restores_equal_the_oracle(ext, seed):
    """Seeded random restores: layout, head count, block size, layers, written slots committed
    over several steps (so some tables of a layer differ in their ranges and fall into separate
    groups), a random head map onto a cache with more head slots, random chunk and piece sizes. Every
    restored head slot equals the source's rows at every written slot, and every other slot of
    the cache is untouched."""
    rng = np.random.default_rng(1000 + seed)
    layout = ["kv_first", "blocks_first", "combined"][seed % 3]
    nb, bs = int(rng.integers(8, 40)), int(rng.choice([1, 2, 4, 5, 16]))
    h_src, d = int(rng.integers(1, 5)), int(rng.choice([8, 6, 64]))
    n_layers = int(rng.integers(1, 4))
    src = caches(layout, d, torch.bfloat16, n_layers=n_layers, nb=nb, bs=bs, h=h_src,
                 seed=seed + 7)
    _, _, _, dd = oracle.recognise(src[0].shape)
    e = 2
    held = sorted(rng.choice(h_src, size=int(rng.integers(1, h_src + 1)), replace=False).tolist())
    tables, written = {}, {}
    num_slots = nb * bs
    for step in (1, 2, 3):
        slots = sorted(rng.choice(num_slots, size=int(rng.integers(1, num_slots // 2 + 2)),
                                  replace=False).tolist())
        cap = 1 << max(3, (len(slots) - 1).bit_length())
        # later steps commit some layers and maybe one head only: a layer's tables then differ
        # in their written ranges
        heads = held if step == 1 or rng.random() < 0.5 else held[:1]
        layers = (list(range(n_layers)) if step == 1 else
                  sorted(rng.choice(n_layers, size=int(rng.integers(1, n_layers + 1)),
                                    replace=False).tolist()))
        rows = oracle.gather_rows(src, slots, heads, cap, dd, bs, strides_of(src[0]), e)
        desc = oracle.staged_step("s", layers, heads, cap, dd, e, slots, "bfloat16")
        oracle.store_commit(rows.view(np.uint8).reshape(-1), desc, tables, num_slots, written,
                            step)
    h_dst = h_src + int(rng.integers(0, 3))
    targets = rng.permutation(h_dst)[:len(held)].tolist()
    moves = dict(zip(held, targets))
    dst_shape = {"kv_first": (2, nb, bs, h_dst, d), "blocks_first": (nb, 2, bs, h_dst, d),
                 "combined": (nb, h_dst, bs, 2 * d)}[layout]
    dst = [torch.zeros(dst_shape, dtype=torch.bfloat16, device="cuda") for _ in range(n_layers)]
    row_bytes = 2 * d * e
    chunk = int(rng.integers(1, 64)) * row_bytes
    piece = int(rng.integers(1, 64)) * row_bytes  # pieces past the chunk are a chunk
    r = Restorer(ext, dst, chunk_bytes=chunk, threads=int(rng.integers(1, 5)), piece_bytes=piece)
    tabs = [Table(t, rows, oracle.written_ranges(written[t])) for t, rows in tables.items()]
    got_rows = r.restore(tabs, moves)
    assert got_rows == sum(int(written[t].astype(bool).sum()) for t in tables)
    cpu = [t.cpu() for t in dst]
    all_slots = list(range(num_slots))
    for layer in range(n_layers):
        back = oracle.gather_rows(cpu[layer:layer + 1], all_slots, list(range(h_dst)), num_slots,
                                  d, bs, strides_of(cpu[0]), e)[0]  # [h_dst, slots, 2, d]
        want = np.zeros_like(back)
        for theirs, ours in moves.items():
            t = layer * 1000 + theirs
            live = np.flatnonzero(written[t])
            src_rows = oracle.gather_rows(src[layer:layer + 1], live.tolist(), [theirs],
                                          max(1, live.size), d, bs, strides_of(src[0]), e)[0, 0]
            want[ours, live] = src_rows[:live.size]
        assert np.array_equal(back, want), (layer, moves)


def test_layers_with_the_same_ranges_share_a_launch_unless_heads_or_layout_differ(ext):
    """A catch-up's tables: every layer written at the same few slots. Layers with the same head
    slots and layout are scattered together in one launch; a layer missing a head's table, or
    laid out differently, keeps a launch of its own; a chunk too small for two layers keeps every
    layer apart. Bytes as the oracle's, every other head slot untouched."""
    nb, bs, h, d = 32, 4, 2, 8
    kv = caches("kv_first", d, torch.bfloat16, n_layers=4, nb=nb, bs=bs, h=h, seed=91)
    bf = caches("blocks_first", d, torch.bfloat16, n_layers=1, nb=nb, bs=bs, h=h, seed=92)
    src = kv[:3] + bf + kv[3:]  # layer 3 is blocks_first
    slots = [9, 10, 11, 40, 41, 77, 3]
    t_kv, w_kv = commit(kv, slots, [0, 1], cap=8)
    t_bf, w_bf = commit(bf, slots, [0, 1], cap=8)
    tables = {}
    for t, rows in t_kv.items():  # kv's layers 0, 1, 2, 3 are ours 0, 1, 2, 4
        layer = t // 1000
        tables[(layer if layer < 3 else 4) * 1000 + t % 1000] = (rows, w_kv[t])
    for t, rows in t_bf.items():
        tables[3000 + t % 1000] = (rows, w_bf[t])
    del tables[1001]  # layer 1 has head 0's table only
    moves = {0: 1, 1: 0}
    for chunk_bytes, launches in ((1 << 20, 3), (len(slots) * 2 * 2 * d * 2, 5)):
        dst = [torch.zeros_like(t).cuda() for t in src]
        r = Restorer(ext, dst, chunk_bytes=chunk_bytes)
        rows = r.restore([Table(t, tb, oracle.written_ranges(w)) for t, (tb, w) in tables.items()],
                         moves)
        assert rows == len(slots) * len(tables)
        # layers 0, 2, 4 together (kv_first, both heads); layer 1 (one head); layer 3 (blocks_first)
        assert r.timing["launches"] == launches
        for layer, t in enumerate(dst):
            cpu = t.cpu()
            theirs = [x for x in (0, 1) if layer * 1000 + x in tables]
            got = oracle.gather_rows([cpu], slots, [moves[x] for x in theirs], 8, d, bs,
                                     strides_of(cpu), 2)
            want = oracle.gather_rows([src[layer]], slots, theirs, 8, d, bs,
                                      strides_of(src[layer]), 2)
            assert np.array_equal(got, want), layer
            if len(theirs) == 1:  # layer 1's head slot 0 (theirs 1) is not written
                rest = oracle.gather_rows([cpu], list(range(nb * bs)), [0], nb * bs, d, bs,
                                          strides_of(cpu), 2)
                assert not rest.any()


def test_a_catch_up_sized_group_in_16_mib_pieces(ext):
    """8 tables of 16 MiB whose written ranges are 630 runs of 24-48 rows (about 90 MiB over the
    group): the Restorer cuts the group into pieces of 16 MiB, ranges cut at the pieces' edges,
    one launch for the chunk. Every row lands where torch's indexing puts it (the tables' rows at
    their slots, head by head), and nothing else is written."""
    nb, bs, h, d = 2048, 16, 8, 128
    n = nb * bs
    rng = np.random.default_rng(7)
    starts = np.arange(630) * 52 + rng.integers(0, 4, size=630)
    counts = rng.integers(24, 49, size=630)
    written = [(int(s), int(c)) for s, c in zip(starts, counts)]
    assert 5 * (16 << 20) < int(counts.sum()) * h * 512 < 7 * (16 << 20)
    tables = {}
    for head in range(h):
        rows = rng.integers(0, 1 << 16, size=(n, 2 * d), dtype=np.uint16) & 0xBFFF
        tables[head] = rows.view(np.uint8)
    dst = torch.zeros((2, nb, bs, h, d), dtype=torch.bfloat16, device="cuda")
    r = Restorer(ext, [dst])
    moves = {x: (x + 3) % h for x in range(h)}
    got = r.restore([Table(x, tables[x], written) for x in range(h)], moves)
    slots = np.concatenate([np.arange(s, s + c) for s, c in written])
    assert got == slots.size * h
    assert r.timing["launches"] == 1
    want = torch.zeros_like(dst)
    s = torch.from_numpy(slots).cuda()
    for x in range(h):
        rows = torch.from_numpy(tables[x].view(np.int16).reshape(n, 2, d)).cuda()
        want[:, s // bs, s % bs, moves[x]] = rows[s].transpose(0, 1).contiguous().view(
            torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(dst.view(torch.int16), want.view(torch.int16))


def test_the_heap_is_frozen_when_built_unless_asked_not_to(ext):
    """freeze_heap (default on) collects and freezes the Python heap when the Restorer is built;
    freeze_heap=False leaves the collector as it is. Either way the collector is on afterwards."""
    import gc

    dst = [torch.zeros((2, 8, 4, 2, 8), dtype=torch.bfloat16, device="cuda")]
    gc.unfreeze()
    Restorer(ext, dst, freeze_heap=False)
    assert gc.get_freeze_count() == 0 and gc.isenabled()
    Restorer(ext, dst)
    assert gc.get_freeze_count() > 0 and gc.isenabled()
    gc.unfreeze()
