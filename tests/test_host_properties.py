"""Property tests of the library's host copies, on the CPU (host code only), over drawn inputs.

hypothesis draws the cases; each is checked against a plain numpy restatement here or the oracle:

* evs_host_gather_tables: T tables of the same written ranges gathered side by side, table j's
  rows at dst + j * dst_rows rows, any row size (odd ones included, so the nontemporal copy's
  unaligned head and tail run), empty ranges, 1 to 16 threads; the bytes past each table's rows
  keep their fill.
* evs_store_commit: a step of slots with padding, repeats (the last write wins), runs and gaps,
  into tables that already hold rows, on 1 to 16 threads, at sizes on both sides of the
  commit's switch to nontemporal stores; rows, written steps and CRC32C equal the oracle's
  restatement of the store's commit (store/src/storage.rs:864-957).
"""

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle
from everserve_amd import kernels
from everserve_amd.state import staging
from everserve_amd.state.store import derive, row_bytes_of

# the same draws on every run (reproducible in CI), and no example database written to the tree
SETTINGS = settings(max_examples=60, deadline=None, derandomize=True, database=None,
                    suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])


@pytest.fixture(scope="module")
def ext():
    path = kernels.library_path()
    return kernels.Kernels(kernels.open_library(path), path)


@st.composite
def gather_cases(draw):
    row_bytes = draw(st.sampled_from([1, 3, 16, 24, 250, 256, 512, 1000]))
    num_slots = draw(st.integers(1, 3000))
    tables = draw(st.integers(1, 9))
    n_ranges = draw(st.integers(0, 12))
    ranges = []
    for _ in range(n_ranges):
        start = draw(st.integers(0, num_slots))
        count = draw(st.integers(0, num_slots - start))
        ranges.append((start, count))
    extra = draw(st.integers(0, 5))
    threads = draw(st.integers(1, 16))
    seed = draw(st.integers(0, 2**31 - 1))
    return row_bytes, num_slots, tables, ranges, extra, threads, seed


@SETTINGS
@given(case=gather_cases())
def test_gather_tables_is_the_concatenation_of_each_tables_ranges(ext, case):
    row_bytes, num_slots, tables, ranges, extra, threads, seed = case
    rng = np.random.default_rng(seed)
    srcs = [rng.integers(0, 256, size=num_slots * row_bytes, dtype=np.uint8) for _ in range(tables)]
    starts = np.array([s for s, _ in ranges], dtype=np.int64)
    counts = np.array([c for _, c in ranges], dtype=np.int64)
    total = int(counts.sum())
    dst_rows = total + extra
    dst = np.full(max(1, tables * dst_rows * row_bytes), 0xA5, dtype=np.uint8)
    got = ext.host_gather_tables([t.ctypes.data for t in srcs], num_slots, row_bytes, starts,
                                 counts, dst.ctypes.data, dst_rows, threads)
    assert got == total
    for j, t in enumerate(srcs):
        rows = t.reshape(num_slots, row_bytes)
        want = (np.concatenate([rows[s:s + c] for s, c in ranges]).reshape(-1) if ranges
                else np.zeros(0, np.uint8))
        base = j * dst_rows * row_bytes
        assert np.array_equal(dst[base:base + total * row_bytes], want), j
        assert (dst[base + total * row_bytes:base + dst_rows * row_bytes] == 0xA5).all(), j


@st.composite
def commit_cases(draw):
    d = draw(st.sampled_from([8, 64, 128]))
    num_slots = draw(st.integers(16, 4096))
    n = draw(st.sampled_from([1, 7, 64, 300, 2048]))
    layers = sorted(draw(st.sets(st.integers(0, 3), min_size=1, max_size=3)))
    heads = sorted(draw(st.sets(st.integers(0, 7), min_size=1, max_size=4)))
    threads = draw(st.integers(1, 16))
    seed = draw(st.integers(0, 2**31 - 1))
    return d, num_slots, n, layers, heads, threads, seed


@SETTINGS
@given(case=commit_cases())
def test_the_commit_is_the_stores_over_drawn_steps(ext, case):
    d, num_slots, n, layers, heads, threads, seed = case
    rng = np.random.default_rng(seed)
    ours = {"rows": {}, "steps": {}, "crc": {}}
    theirs = {"rows": {}, "steps": {}, "crc": {}}
    for step in (1, 2):
        slots = rng.integers(0, num_slots, size=n)
        if n > 4:  # runs of consecutive slots, padding and a repeat
            a = int(rng.integers(0, num_slots - 4))
            slots[:4] = np.arange(a, a + 4)
            slots[rng.random(n) < 0.1] = -1
            slots[-1] = slots[0]
        cap = staging.capacity_for(n)
        e = 2
        size = (max(layers) + 1) * len(heads) * cap * 2 * d * e
        stage = rng.integers(0, 256, size=size, dtype=np.uint8)
        desc = staging.describe("s", layers, heads, cap, d, e, slots.tolist(), "bfloat16")
        rb = row_bytes_of(desc)
        tabs = derive(desc)
        for t, _ in tabs:
            if t not in ours["rows"]:
                ours["rows"][t] = np.zeros(num_slots * rb, dtype=np.uint8)
                ours["steps"][t] = np.zeros(num_slots, dtype=np.uint64)
                ours["crc"][t] = np.zeros(num_slots, dtype=np.uint32)
        ext.store_commit(stage, [o for _, o in tabs], [ours["rows"][t] for t, _ in tabs],
                         [ours["steps"][t] for t, _ in tabs], [ours["crc"][t] for t, _ in tabs],
                         num_slots, rb, desc["slots"], step, threads)
        oracle.store_commit(stage, desc, theirs["rows"], num_slots, theirs["steps"], step,
                            theirs["crc"])
    for t in theirs["rows"]:
        assert np.array_equal(ours["rows"][t], theirs["rows"][t]), t
        assert np.array_equal(ours["steps"][t], theirs["steps"][t]), t
        assert np.array_equal(ours["crc"][t], theirs["crc"][t]), t
