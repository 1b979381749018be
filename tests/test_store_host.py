"""The store's commit copy and its checksums (evs_store_commit, evs_crc32c), on the CPU: host code.

* **CRC32C pins.** Both the library's and the oracle's CRC32C must give the published check
  value of "123456789" (0xE3069283) and the RFC 3720 B.4 vectors. They must also satisfy the
  CRC's affine law on random data of every length, crc(a) ^ crc(b) ^ crc(c) == crc(a ^ b ^ c)
  for equal lengths, and agree with each other row by row. The store computes them with the
  crc32c crate 0.6.8 (store/Cargo.toml:25), which is absent here.
* **The commit.** The library's commit is checked against the oracle's restatement of
  ``Storage::commit`` (store/src/storage.rs:864-957), which the store's own byte case pins
  (tests/test_oracle_store.py). It must match byte for byte: the tables, the written steps and
  the checksums, over random multi-table steps with padding, runs, repeated slots and
  overwrites, on one thread and several.
* **Refusals** happen before anything is written.
* :class:`everserve_amd.state.store.StoreTables` is checked against the oracle, in memory and
  file-backed, with its written ranges.
"""

import numpy as np
import pytest

import oracle
from everserve_amd import kernels
from everserve_amd.state import staging
from everserve_amd.state.store import StoreTables, derive, row_bytes_of

VECTORS = [
    (b"123456789", 0xE3069283),
    (bytes(32), 0x8A9136AA),
    (b"\xff" * 32, 0x62A8AB43),
    (bytes(range(32)), 0x46DD794E),
    (bytes(range(31, -1, -1)), 0x113FDB5C),
]


@pytest.fixture(scope="module")
def ext():
    path = kernels.library_path()
    return kernels.Kernels(kernels.open_library(path), path)


@pytest.mark.parametrize("data,want", VECTORS)
def test_crc32c_gives_the_published_values(ext, data, want):
    assert oracle.crc32c(data) == want
    assert ext.crc32c(data) == want


@pytest.mark.parametrize("n", [0, 1, 3, 7, 8, 9, 31, 64, 511, 512, 4099])
def test_crc32c_is_affine_and_both_agree(ext, n):
    rng = np.random.default_rng(n)
    a, b, c = (rng.integers(0, 256, size=n, dtype=np.uint8) for _ in range(3))
    for f in (oracle.crc32c, ext.crc32c):
        assert f(a.tobytes()) ^ f(b.tobytes()) ^ f(c.tobytes()) == f((a ^ b ^ c).tobytes())
    assert ext.crc32c(a) == oracle.crc32c(a.tobytes())


@pytest.mark.parametrize("row_bytes", [1, 7, 8, 32, 512])
@pytest.mark.parametrize("rows", [1, 3, 4, 5, 13, 300])
def test_crc32c_of_rows_is_the_crc_of_each_row(ext, row_bytes, rows):
    data = np.random.default_rng(rows * row_bytes).integers(0, 256, size=(rows, row_bytes),
                                                           dtype=np.uint8)
    want = oracle.crc32c_rows(data)
    assert np.array_equal(ext.crc32c_rows(data, row_bytes), want)
    assert [oracle.crc32c(r.tobytes()) for r in data] == want.tolist()


def staged(layers, heads, cap, d, elem, slots, seed):
    rb = 2 * d * elem
    # rows are placed by layer id (layer * layer_stride): the bytes span up to the highest id
    size = (max(layers) + 1) * len(heads) * cap * rb
    stage = np.random.default_rng(seed).integers(0, 256, size=size, dtype=np.uint8)
    desc = staging.describe("s", layers, heads, cap, d, elem, slots,
                            {1: "uint8", 2: "bfloat16", 4: "float32"}[elem])
    return stage, desc


def commit_both(ext, stage, desc, num_slots, step, threads, state):
    """The library's commit into `state`'s arrays, and the oracle's into its own."""
    ours, theirs = state
    rb = row_bytes_of(desc)
    tabs = derive(desc)
    for t, _ in tabs:
        if t not in ours["rows"]:
            ours["rows"][t] = np.zeros(num_slots * rb, dtype=np.uint8)
            ours["steps"][t] = np.zeros(num_slots, dtype=np.uint64)
            ours["crc"][t] = np.zeros(num_slots, dtype=np.uint32)
    fresh = ext.store_commit(stage, [o for _, o in tabs], [ours["rows"][t] for t, _ in tabs],
                             [ours["steps"][t] for t, _ in tabs], [ours["crc"][t] for t, _ in tabs],
                             num_slots, rb, desc["slots"], step, threads)
    oracle.store_commit(stage, desc, theirs["rows"], num_slots, theirs["steps"], step,
                        theirs["crc"])
    return fresh


@pytest.mark.parametrize("threads", [1, 4])
def test_the_commit_is_the_stores(ext, threads):
    num_slots, d, elem = 96, 8, 2
    ours = {"rows": {}, "steps": {}, "crc": {}}
    theirs = {"rows": {}, "steps": {}, "crc": {}}
    steps = [
        ([0, 1, 2], [0, 2], 16, [5, 6, 7, 8, -1, 40, 41, 90, 3], 1),      # runs, padding
        ([1, 2], [0, 2], 8, [40, 41, 42, 10, 10, -1], 2),                  # overwrite, a repeat
        ([0, 1, 2, 3], [2], 8, list(range(88, 96)), 0),                    # a new table, step 0
    ]
    seen: set[tuple[int, int]] = set()
    for layers, heads, cap, slots, step in steps:
        stage, desc = staged(layers, heads, cap, d, elem, slots, seed=step + 7)
        fresh = commit_both(ext, stage, desc, num_slots, step, threads, (ours, theirs))
        new = {(t, s) for t, _ in derive(desc) for s in slots if s >= 0} - seen
        seen |= new
        assert fresh == len(new)
    assert sorted(ours["rows"]) == sorted(theirs["rows"])
    for t in theirs["rows"]:
        assert np.array_equal(ours["rows"][t], theirs["rows"][t]), t
        assert np.array_equal(ours["steps"][t], theirs["steps"][t]), t
        assert np.array_equal(ours["crc"][t], theirs["crc"][t]), t
    assert ours["steps"][3002][88] == 1  # step 0 counts as written: recorded as 1


@pytest.mark.parametrize("threads", [1, 16])
def test_a_large_step_written_with_streaming_stores_is_the_stores(ext, threads):
    """A step of 4 MiB or more takes the commit's other copy (nontemporal stores): 4 tables of
    2,048 rows of 512 B, ascending runs, padding and a repeated slot, then a small step into the
    same tables."""
    num_slots, d, elem = 4096, 128, 2
    ours = {"rows": {}, "steps": {}, "crc": {}}
    theirs = {"rows": {}, "steps": {}, "crc": {}}
    rng = np.random.default_rng(11)
    slots = rng.permutation(num_slots)[:2048].tolist()
    slots[5], slots[99] = -1, slots[98]
    stage, desc = staged([0, 1], [0, 1], 2048, d, elem, slots, seed=12)
    assert stage.nbytes >= 4 << 20
    commit_both(ext, stage, desc, num_slots, 4, threads, (ours, theirs))
    stage, desc = staged([0, 1], [0, 1], 8, d, elem, [7, 8, 9, slots[0]], seed=13)
    commit_both(ext, stage, desc, num_slots, 5, threads, (ours, theirs))
    for t in theirs["rows"]:
        assert np.array_equal(ours["rows"][t], theirs["rows"][t]), t
        assert np.array_equal(ours["steps"][t], theirs["steps"][t]), t
        assert np.array_equal(ours["crc"][t], theirs["crc"][t]), t


def test_store_tables_reuse_a_table_sets_commit_arguments(ext):
    """Steps that name a table set, another one with a new table, and the first again (its
    arguments built before are used): every table equals the oracle's after each step."""
    num_slots, d = 64, 8
    store = StoreTables(ext, num_slots, threads=2)
    tables, written, crcs = {}, {}, {}
    for step, (layers, heads, slots) in enumerate((([0, 1], [0], [1, 2, 3]),
                                                   ([1, 2], [0, 1], [4, 5, -1]),
                                                   ([0, 1], [0], [6, 1]),
                                                   ([1, 2], [0, 1], [7])), start=1):
        stage, desc = staged(layers, heads, 8, d, 2, slots, seed=20 + step)
        store.commit(stage, desc, step)
        oracle.store_commit(stage, desc, tables, num_slots, written, step, crcs)
        assert sorted(store.tables) == sorted(tables)
        for t, want in tables.items():
            assert np.array_equal(np.asarray(store.tables[t].rows), want), (step, t)
            assert np.array_equal(store.tables[t].crc, crcs[t]), (step, t)
    assert len(store._plans) == 2


def test_store_tables_commits_from_two_threads_and_a_reader(ext):
    """Two threads commit steps of different layers while a third reads the table set as a
    restore does: the commits take turns, no read sees the set change under it, and every table
    ends equal to the oracle's."""
    import threading

    num_slots, d = 256, 8
    store = StoreTables(ext, num_slots, threads=4)
    steps = {k: [staged([k], [0, 1], 16, d, 2, list(range(i * 8 + k, i * 8 + k + 8)), seed=i + 50)
                 for i in range(12)] for k in (0, 1)}
    errors, done = [], threading.Event()

    def commit(k):
        try:
            for i, (stage, desc) in enumerate(steps[k]):
                store.commit(stage, desc, i + 1)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    def read():
        try:
            while not done.is_set():
                for t in store.restore_tables():
                    assert t.written and t.rows.size == num_slots * 2 * d * 2
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    reader = threading.Thread(target=read)
    reader.start()
    writers = [threading.Thread(target=commit, args=(k,)) for k in (0, 1)]
    for t in writers:
        t.start()
    for t in writers:
        t.join()
    done.set()
    reader.join()
    assert not errors, errors
    tables, written, crcs = {}, {}, {}
    for k in (0, 1):
        for i, (stage, desc) in enumerate(steps[k]):
            oracle.store_commit(stage, desc, tables, num_slots, written, i + 1, crcs)
    assert sorted(store.tables) == sorted(tables)
    for t, want in tables.items():
        assert np.array_equal(np.asarray(store.tables[t].rows), want), t
        assert np.array_equal(store.tables[t].crc, crcs[t]), t


def test_a_bad_step_is_refused_before_anything_is_written(ext):
    num_slots, d = 32, 8
    stage, desc = staged([0], [0, 1], 8, d, 2, [3, 4, 40], seed=1)
    rows = [np.zeros(num_slots * 32, dtype=np.uint8) for _ in range(2)]
    steps = [np.zeros(num_slots, dtype=np.uint64) for _ in range(2)]
    crcs = [np.zeros(num_slots, dtype=np.uint32) for _ in range(2)]
    offs = [o for _, o in derive(desc)]
    with pytest.raises(kernels.KernelError, match="outside"):
        ext.store_commit(stage, offs, rows, steps, crcs, num_slots, 32, desc["slots"], 3)
    with pytest.raises(kernels.KernelError, match="outside the staging"):
        ext.store_commit(stage[:100], offs, rows, steps, crcs, num_slots, 32, [3, 4], 3)
    assert not any(r.any() for r in rows) and not any(s.any() for s in steps)


@pytest.mark.parametrize("file_backed", [False, True])
def test_store_tables_commit_and_written_ranges(ext, tmp_path, file_backed):
    num_slots, d = 64, 6
    store = StoreTables(ext, num_slots, tmp_path / "rank0" if file_backed else None, threads=3)
    tables, written, crcs = {}, {}, {}
    for step, slots in ((1, [0, 1, 2, 3, 9, -1, 10]), (2, [20, 21, 2]), (3, [63, 62, 61])):
        stage, desc = staged([0, 1], [1, 2], 8, d, 2, slots, seed=step)
        store.commit(stage, desc, step)
        oracle.store_commit(stage, desc, tables, num_slots, written, step, crcs)
    store.flush()
    assert sorted(store.tables) == sorted(tables)
    for t, want in tables.items():
        assert np.array_equal(np.asarray(store.tables[t].rows), want)
        assert np.array_equal(store.tables[t].crc, crcs[t])
        for since in (0, 1, 2):
            assert store.written_ranges(t, since) == oracle.written_ranges(written[t], since)
    assert [tb.table for tb in store.restore_tables(2)] == sorted(tables)
    if file_backed:
        t = sorted(tables)[0]
        on_disk = np.fromfile(tmp_path / "rank0" / f"table{t}.rows", dtype=np.uint8)
        assert np.array_equal(on_disk, tables[t])


def test_store_tables_refuse_a_slot_outside_and_a_changed_row_size(ext):
    store = StoreTables(ext, 16)
    stage, desc = staged([0], [0], 8, 8, 2, [1, 2], seed=3)
    store.commit(stage, desc, 1)
    stage2, desc2 = staged([0], [0], 8, 8, 2, [1, 17], seed=4)
    with pytest.raises(ValueError, match="outside"):
        store.commit(stage2, desc2, 2)
    stage3, desc3 = staged([0], [0], 8, 4, 2, [1], seed=5)
    with pytest.raises(ValueError, match="bytes"):
        store.commit(stage3, desc3, 2)


def test_a_forked_child_commits_while_the_parent_is_busy(ext):
    """The library's host worker set belongs to the process that started it. A child forked
    while the parent's threads are in commits (so the set may be mid-call, its lock held by a
    thread the child does not have) commits on threads of its own and gets the store's bytes."""
    import os
    import threading
    import time

    num_slots, d, elem = 4096, 64, 2
    stage, desc = staged([0, 1, 2, 3], [0, 1], 1024, d, elem, list(range(1024)), seed=11)
    stop = threading.Event()

    def busy():
        state = ({"rows": {}, "steps": {}, "crc": {}}, {"rows": {}, "steps": {}, "crc": {}})
        step = 1
        while not stop.is_set():
            commit_both(ext, stage, desc, num_slots, step, 8, state)
            step += 1

    commit_both(ext, stage, desc, num_slots, 1, 8, ({"rows": {}, "steps": {}, "crc": {}},
                                                    {"rows": {}, "steps": {}, "crc": {}}))
    worker = threading.Thread(target=busy)
    worker.start()
    children = []
    try:
        for _ in range(4):
            time.sleep(0.02)
            pid = os.fork()
            if pid == 0:  # the child: one commit on 4 threads, checked against the oracle
                code = 1
                try:
                    ours = {"rows": {}, "steps": {}, "crc": {}}
                    theirs = {"rows": {}, "steps": {}, "crc": {}}
                    commit_both(ext, stage, desc, num_slots, 3, 4, (ours, theirs))
                    same = all(np.array_equal(ours[k][t], theirs[k][t])
                               for k in ours for t in theirs[k])
                    code = 0 if same else 2
                finally:
                    os._exit(code)
            children.append(pid)
    finally:
        stop.set()
        worker.join()
    deadline = time.monotonic() + 60
    codes = {}
    while len(codes) < len(children) and time.monotonic() < deadline:
        for pid in children:
            if pid not in codes:
                got, status = os.waitpid(pid, os.WNOHANG)
                if got == pid:
                    codes[pid] = os.waitstatus_to_exitcode(status)
        time.sleep(0.01)
    for pid in children:
        if pid not in codes:  # a child that hung: end it, and fail
            os.kill(pid, 9)
            os.waitpid(pid, 0)
    assert len(codes) == len(children), "a forked child did not finish its commit"
    assert all(c == 0 for c in codes.values()), codes
