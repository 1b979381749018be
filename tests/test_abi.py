"""The C-ABI library, without a GPU: it loads, exports every entry point include/*.h declares,
and refuses bad arguments before touching the device. No kernel is launched here."""

import ctypes
import re
from pathlib import Path

import pytest

from everserve_amd import build, kernels

ROOT = Path(__file__).resolve().parents[1]


def declared() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(evs_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    return kernels.open_library(kernels.library_path())


def test_every_declared_entry_point_is_exported_and_bound(lib):
    names = declared()
    assert len(names) >= 18, names
    for name in sorted(names):
        assert hasattr(lib, name), f"{name} is declared but not exported"
    assert names == set(kernels.ENTRY_POINTS), names ^ set(kernels.ENTRY_POINTS)


def test_the_region_layout_is_the_reference_modules(lib):
    # core/csrc/kernels.h:18-22 and core/everserve/comm/slotkernel.py:55,73-80
    words = (ctypes.c_int64 * 5)()
    assert lib.evs_layout_constants(words, 5) == 0
    assert list(words) == [8, 16, 1, 11, 12]
    assert lib.evs_layout_constants(words, 4) == 1


def test_slot_blocks_is_the_reference_formula(lib):
    out = ctypes.c_int64()
    for maxn, words in ((65536, 1), (65536, 16), (2, 1), (3000, 4), (0, 1)):
        assert lib.evs_slot_blocks(maxn, words, ctypes.byref(out)) == 0
        per_block = 256 * words
        assert out.value == (maxn // 2 + per_block - 1) // per_block
    assert lib.evs_slot_blocks(10, 0, ctypes.byref(out)) == 1


def test_bad_arguments_are_refused_with_a_message(lib):
    strides = (ctypes.c_int64 * 5)(96, 24, 8, 672, 1)
    # an element size the kernels do not take: refused before any device call
    rc = lib.evs_gather_rows(None, 1, None, 5, None, 2, None, 8, 8, 4, strides, 3, None)
    assert rc == 1
    assert b"element size" in lib.evs_last_error()
    rc = lib.evs_gather_rows(None, 1, None, 9, None, 2, None, 8, 8, 4, strides, 2, None)
    assert rc == 1 and b"capacity" in lib.evs_last_error()
    rc = lib.evs_scatter_rows(None, 1, None, 5, None, 2, None, 8, 8, 4, None, 2, None)
    assert rc == 1 and b"five strides" in lib.evs_last_error()
    # nothing to move: success without a launch
    assert lib.evs_gather_rows(None, 0, None, 5, None, 2, None, 8, 8, 4, strides, 2, None) == 0
    assert lib.evs_last_error() == b""
    rc = lib.evs_local_reduce(None, None, None, None, 4, 1, 0, None, None, None)
    assert rc == 1 and b"null" in lib.evs_last_error()
    rc = lib.evs_copy_rows_async(None, None, 2, 16, 8, None)
    assert rc == 1 and b"pitch" in lib.evs_last_error()
    # the range scatter: a negative range count, rows but no range, more rows than the staging
    # holds, no range arrays; nothing to move is a success
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: each call stops at its checks
    rc = lib.evs_scatter_ranges(fake, 1, fake, fake, -1, 4, fake, 2, fake, 8, 8, 4, strides, 2,
                                None)
    assert rc == 1 and b"negative range" in lib.evs_last_error()
    rc = lib.evs_scatter_ranges(fake, 1, fake, fake, 0, 4, fake, 2, fake, 8, 8, 4, strides, 2,
                                None)
    assert rc == 1 and b"no range" in lib.evs_last_error()
    rc = lib.evs_scatter_ranges(fake, 1, fake, fake, 1, 9, fake, 2, fake, 8, 8, 4, strides, 2,
                                None)
    assert rc == 1 and b"capacity" in lib.evs_last_error()
    rc = lib.evs_scatter_ranges(fake, 1, None, fake, 1, 4, fake, 2, fake, 8, 8, 4, strides, 2,
                                None)
    assert rc == 1 and b"null index" in lib.evs_last_error()
    assert lib.evs_scatter_ranges(fake, 1, None, None, 0, 0, fake, 2, fake, 8, 8, 4, strides, 2,
                                  None) == 0


def test_the_build_is_stamped_with_this_trees_sources():
    stamp = kernels._check_stamp(kernels._PACKAGE)
    assert stamp.name == kernels.LIBRARY
    assert build.stamp()["sources"] == kernels.stamp()["sources"]


def test_the_reduce_state_size_is_the_headers():
    from everserve_amd import kernels

    header = (Path(__file__).resolve().parents[1] / "include" / "everserve_mi355x.h").read_text()
    m = re.search(r"#define EVS_REDUCE_STATE_WORDS (\d+)", header)
    assert m is not None and int(m.group(1)) == kernels.REDUCE_STATE_WORDS


def test_a_launch_past_the_work_item_limit_is_refused_before_launch(lib):
    """HIP takes at most 2^32 - 1 work-items along x. C2's shape at 1,048,576 slots over 32 layers
    is 2^24 gather workgroups of 256 threads, exactly 2^32 work-items: refused with a message,
    before any device call (this runs without a GPU). 8 slots fewer would be 2^24 - 128
    workgroups, within the limit."""
    strides = (ctypes.c_int64 * 5)(16384, 1024, 128, 134217728, 1)
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the call stops at its checks
    n = 1 << 20
    rc = lib.evs_gather_rows(fake, 32, fake, n, fake, 8, ctypes.c_void_p(1 << 21), n, 128, 16,
                             strides, 2, None)
    assert rc == 1 and b"work-items" in lib.evs_last_error()
    rc = lib.evs_scatter_rows(fake, 32, fake, 2 * n, fake, 8, ctypes.c_void_p(1 << 21), 2 * n,
                              128, 16, strides, 2, None)
    assert rc == 1 and b"work-items" in lib.evs_last_error()
    rc = lib.evs_scatter_ranges(fake, 32, fake, fake, 1, 2 * n, fake, 8, ctypes.c_void_p(1 << 21),
                                2 * n, 128, 16, strides, 2, None)
    assert rc == 1 and b"work-items" in lib.evs_last_error()


def test_failed_parity_flags_fail_the_bench(tmp_path):
    import bench

    good = {"extra": {"a": {"rows_equal_x": True, "sum_exact": True}, "flag": False}}
    assert bench.failed_checks(good) == []
    bad = {"extra": {"c4": {"round_trip_equal_first_4_layers": False},
                     "s": {"k": {"sum_exact": False}}, "spot_check": False, "rows_check": True}}
    assert bench.failed_checks(bad) == ["extra.c4.round_trip_equal_first_4_layers",
                                        "extra.s.k.sum_exact", "extra.spot_check"]

def test_scatter_rows_sorts_first_from_two_to_the_18_slots_and_8_gib():
    sf = kernels.sort_first
    c4 = dict(layers=32, heads=8, d=128, elem=2)  # 32 GiB of rows at 262,144 slots
    assert sf(1 << 18, capturing=False, **c4)
    assert not sf((1 << 18) - 1, capturing=False, **c4)  # too few slots
    assert not sf(1 << 18, capturing=True, **c4)  # the sort's memset stays out of graphs
    assert not sf(1 << 31, capturing=False, **c4)  # past the sort's limit
    # 8 layers of the cache (8 GiB) sort, 4 layers (4 GiB) do not
    assert sf(1 << 18, layers=8, heads=8, d=128, elem=2, capturing=False)
    assert not sf(1 << 18, layers=4, heads=8, d=128, elem=2, capturing=False)
    assert kernels.ORDER_MIN_SLOTS == 1 << 18 and kernels.ORDER_MIN_BYTES == 8 << 30
    # told the cache's slot count, it sorts only a call that writes seven eighths of it or more
    assert sf(1 << 18, capturing=False, num_slots=1 << 18, **c4)
    assert sf(7 << 17, capturing=False, num_slots=1 << 20, **c4)
    assert not sf((7 << 17) - 1, capturing=False, num_slots=1 << 20, **c4)
