"""The host side of the ordered restore: ``destination_order`` on the CPU.

The pairs it returns must name every non-padding staged row exactly once, in increasing slot
order; the whole-block fast path must return what the generic sort returns.
"""

import numpy as np
import pytest

from everserve_amd.state.restore import destination_order


def check(slots, got_slots, rows_of):
    slots = np.asarray(slots, dtype=np.int64)
    keep = np.flatnonzero(slots >= 0)
    assert sorted(rows_of.tolist()) == keep.tolist()
    assert np.array_equal(got_slots, slots[rows_of])
    assert (np.diff(got_slots) >= 0).all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_any_slot_list_comes_back_sorted_without_padding(seed):
    rng = np.random.default_rng(seed)
    slots = rng.choice(10_000, size=777, replace=False).astype(np.int64)
    slots[rng.random(777) < 0.1] = -1
    check(slots, *destination_order(slots))
    check(slots, *destination_order(slots, block_size=16))


@pytest.mark.parametrize("bs", [1, 4, 16])
def test_whole_blocks_order_the_blocks_and_match_the_generic_sort(bs):
    blocks = np.random.default_rng(4).permutation(512)
    slots = (blocks[:, None] * bs + np.arange(bs)).reshape(-1)
    fast = destination_order(slots, block_size=bs)
    generic = destination_order(slots)
    assert np.array_equal(fast[0], generic[0]) and np.array_equal(fast[1], generic[1])
    assert np.array_equal(fast[0], np.arange(512 * bs))


def test_runs_that_are_not_whole_blocks_take_the_generic_path():
    slots = np.array([5, 6, 7, 8, 0, 1, 2, 3], dtype=np.int64)  # the first run starts mid-block
    got, rows_of = destination_order(slots, block_size=4)
    check(slots, got, rows_of)
    assert got.tolist() == [0, 1, 2, 3, 5, 6, 7, 8]


def test_empty_and_all_padding():
    for slots in ([], [-1, -1, -1, -1]):
        got, rows_of = destination_order(slots, block_size=4)
        assert got.size == 0 and rows_of.size == 0


def test_release_later_drops_the_tables_off_the_calling_thread(tmp_path):
    import gc
    import threading
    import weakref

    from everserve_amd.state.restore import Table, release_later

    path = tmp_path / "table.rows"
    np.zeros(4096, dtype=np.uint8).tofile(path)
    tables = [Table.open(7, str(path), [(0, 8)]) for _ in range(3)]
    maps = [weakref.ref(t.rows) for t in tables]
    th = release_later(tables)
    assert tables == [] and isinstance(th, threading.Thread)
    th.join()
    gc.collect()
    assert all(m() is None for m in maps)


def test_written_ranges_are_summarised_once_as_the_plan_reads_them():
    """The plan's view of a written list: empty ranges dropped, any negative start or count
    flagged, the largest end over every range (empty ones included)."""
    from everserve_amd.state.restore import _Written

    w = _Written.of([(4, 3), (9, 0), (12, 5), (40, 0)])
    assert w.starts.tolist() == [4, 12] and w.counts.tolist() == [3, 5]
    assert not w.negative and w.end == 40
    assert w.key == _Written.of([(4, 3), (12, 5)]).key
    assert w.key != _Written.of([(4, 3), (12, 6)]).key
    assert _Written.of([(-1, 2)]).negative and _Written.of([(3, -1)]).negative
    assert _Written.of([(0, 0)]).starts.size == 0
    assert _Written.of([]).end == 0 and not _Written.of([]).negative


def test_reserving_descriptors_grows_the_table_and_leaves_none_open():
    """reserve_descriptors holds its duplicates only while it runs; the descriptor table then
    has room for that many more."""
    import os

    from everserve_amd.state.restore import reserve_descriptors

    def fdsize() -> int:
        with open("/proc/self/status") as f:
            return next(int(line.split()[1]) for line in f if line.startswith("FDSize"))

    before = sorted(os.listdir("/proc/self/fd"))
    reserve_descriptors(600)
    reserve_descriptors(0)
    assert sorted(os.listdir("/proc/self/fd")) == before
    assert fdsize() >= len(before) + 600


def test_reserving_past_the_descriptor_limit_stops_there_quietly():
    """At the process's descriptor limit the reservation stops without an error and closes
    what it held."""
    import os
    import resource

    from everserve_amd.state.restore import reserve_descriptors

    soft, hard = resource.getrlimit(resource.RLIMIT_NOFILE)
    before = sorted(os.listdir("/proc/self/fd"))
    resource.setrlimit(resource.RLIMIT_NOFILE, (len(before) + 40, hard))
    try:
        reserve_descriptors(500)
    finally:
        resource.setrlimit(resource.RLIMIT_NOFILE, (soft, hard))
    assert sorted(os.listdir("/proc/self/fd")) == before


def test_gc_paused_restores_the_collector_as_it_found_it(tmp_path):
    """Collection is off inside the block and as before after it, also when the block raises;
    open_tables opens every table inside such a block."""
    import gc

    from everserve_amd.state.restore import gc_paused, open_tables

    assert gc.isenabled()
    with gc_paused():
        assert not gc.isenabled()
    assert gc.isenabled()
    with pytest.raises(RuntimeError):
        with gc_paused():
            raise RuntimeError("inside")
    assert gc.isenabled()
    gc.disable()
    try:
        with gc_paused():
            pass
        assert not gc.isenabled()
    finally:
        gc.enable()
    path = tmp_path / "t.rows"
    path.write_bytes(bytes(range(64)) * 4)
    tables = open_tables([(3, str(path), [(0, 2)]), (1004, str(path), [(1, 1)])])
    assert [t.table for t in tables] == [3, 1004] and tables[1].head == 4
    assert tables[0].rows.nbytes == 256 and bytes(tables[0].rows[:4]) == bytes(range(4))
