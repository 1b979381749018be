"""The restore's host gather (evs_host_gather_ranges), on the CPU: it is host code only.

Against numpy's concatenation of the same row ranges, for one range, many small ones, empty ones,
sizes that take one thread and sizes that take several, and bad ranges refused.
"""

import numpy as np
import pytest

from everserve_amd import kernels


@pytest.fixture(scope="module")
def ext():
    path = kernels.library_path()
    return kernels.Kernels(kernels.open_library(path), path)


def concat(table, row_bytes, starts, counts):
    rows = table.reshape(-1, row_bytes)
    parts = [rows[s:s + c] for s, c in zip(starts, counts)]
    return np.concatenate(parts).reshape(-1) if parts else np.zeros(0, np.uint8)


@pytest.mark.parametrize("num_slots,row_bytes,ranges", [
    (64, 16, [(3, 1), (9, 1), (12, 1)]),                 # the store test's written slots
    (4096, 512, [(0, 4096)]),                             # every slot
    (4096, 512, [(5, 0), (7, 3), (100, 0), (200, 50)]),  # empty ranges among others
    (70000, 512, [(i * 7, 3) for i in range(9000)]),     # many short ranges, several threads
    (100000, 256, [(0, 40000), (50000, 50000)]),          # large, several threads
])
def test_the_rows_of_the_ranges_in_order(ext, num_slots, row_bytes, ranges):
    rng = np.random.default_rng(num_slots)
    table = rng.integers(0, 255, size=num_slots * row_bytes, dtype=np.uint8)
    starts = np.array([s for s, _ in ranges], dtype=np.int64)
    counts = np.array([c for _, c in ranges], dtype=np.int64)
    want = concat(table, row_bytes, starts, counts)
    dst = np.full(max(1, want.size), 0xEE, dtype=np.uint8)
    rows = ext.host_gather_ranges(table.ctypes.data, num_slots, row_bytes, starts, counts,
                                  dst.ctypes.data, dst.size // row_bytes, 8)
    assert rows == counts.sum()
    assert np.array_equal(dst[:want.size], want)


def test_bad_ranges_are_refused(ext):
    table = np.zeros(64, np.uint8)  # 4 rows of 16 bytes
    dst = np.full(64, 7, np.uint8)  # room for 4 rows
    with pytest.raises(kernels.KernelError, match="negative range"):
        ext.host_gather_ranges(table.ctypes.data, 4, 16, np.array([-1]), np.array([1]),
                               dst.ctypes.data, 4)
    with pytest.raises(kernels.KernelError, match="row_bytes"):
        ext.host_gather_ranges(table.ctypes.data, 4, 0, np.array([0]), np.array([1]),
                               dst.ctypes.data, 4)
    # past the table's end, by the start or by the count, and the largest count that overflows
    for start, count in ((4, 1), (3, 2), (1, 2**62)):
        with pytest.raises(kernels.KernelError, match="outside the table"):
            ext.host_gather_ranges(table.ctypes.data, 4, 16, np.array([0, start]),
                                   np.array([1, count]), dst.ctypes.data, 4)
    # more rows than dst holds: refused before the first range is copied
    with pytest.raises(kernels.KernelError, match="more rows than dst"):
        ext.host_gather_ranges(table.ctypes.data, 4, 16, np.array([0, 1]), np.array([3, 2]),
                               dst.ctypes.data, 4)
    assert (dst == 7).all()
    # the whole table into exactly enough room is fine
    assert ext.host_gather_ranges(table.ctypes.data, 4, 16, np.array([0]), np.array([4]),
                                  dst.ctypes.data, 4) == 4


@pytest.mark.parametrize("tables,num_slots,row_bytes,ranges", [
    (1, 64, 16, [(3, 1), (9, 1), (12, 1)]),
    (8, 4096, 512, [(0, 4096)]),                            # a layer's heads, every slot
    (8, 4096, 512, [(5, 0), (7, 3), (100, 0), (200, 50)]),
    (3, 70000, 512, [(i * 7, 3) for i in range(9000)]),    # several threads cut across tables
    (5, 9000, 256, [(17, 4000), (5000, 3999)]),
])
def test_several_tables_with_the_same_ranges_land_in_their_own_blocks(ext, tables, num_slots,
                                                                       row_bytes, ranges):
    rng = np.random.default_rng(tables * num_slots)
    srcs = [rng.integers(0, 255, size=num_slots * row_bytes, dtype=np.uint8)
            for _ in range(tables)]
    starts = np.array([s for s, _ in ranges], dtype=np.int64)
    counts = np.array([c for _, c in ranges], dtype=np.int64)
    rows = int(counts.sum())
    room = rows + 3  # a pitch larger than the rows: the gaps stay untouched
    dst = np.full((tables, room * row_bytes), 0xEE, dtype=np.uint8)
    got = ext.host_gather_tables([t.ctypes.data for t in srcs], num_slots, row_bytes, starts,
                                 counts, dst.ctypes.data, room, 8)
    assert got == rows
    for j, t in enumerate(srcs):
        assert np.array_equal(dst[j, :rows * row_bytes], concat(t, row_bytes, starts, counts)), j
        assert (dst[j, rows * row_bytes:] == 0xEE).all()


def test_a_multi_table_gather_refuses_before_copying(ext):
    a, b = np.zeros(64, np.uint8), np.zeros(64, np.uint8)
    dst = np.full(128, 7, np.uint8)
    with pytest.raises(kernels.KernelError, match="outside the table"):
        ext.host_gather_tables([a.ctypes.data, b.ctypes.data], 4, 16, np.array([0, 3]),
                               np.array([1, 2]), dst.ctypes.data, 4)
    with pytest.raises(kernels.KernelError, match="table 1 is null"):
        ext.host_gather_tables([a.ctypes.data, 0], 4, 16, np.array([0]), np.array([1]),
                               dst.ctypes.data, 4)
    assert (dst == 7).all()
    assert ext.host_gather_tables([], 4, 16, np.array([0]), np.array([1]), 0, 4) == 1
