"""The restore's copy into this rank's cache: a lost rank's store tables to the paged cache.

The reference's loop (core/everserve/state/mirror.py:916-939) takes each table the store names,
maps it from shared memory as ``[num_slots, 2, d]``, gathers the written rows on the host with
``torch.index_select`` into pinned memory, copies them to the device and scatters them with
``PagedKV.write_rows`` into the head slot the rank assigned. Published at 2.1-2.6 GB/s
(bench/runs/2026-10-05-shm-commit-4gpu/RESULT.md:36,45-46): the host gather bounds it.

:class:`Restorer` first checks every table against this rank's cache (its layers, head slots,
row size and slot count), so a bad table refuses the restore before anything is written. It then
groups the tables of a layer that share their written ranges (a store commit writes every held
head of a layer at the same slots) and restores each group in chunks, one scatter launch a chunk
(``evs_scatter_ranges`` with the group's head slots, the layer's own strides) writing all of the
group's heads: each cache block's rows are covered whole, in increasing slot order. A chunk
reaches the device in pieces, which keeps three things busy at once: host threads gathering
piece i+1's rows of all the group's tables side by side into a pinned buffer
(``evs_host_gather_tables``), the copy engine moving piece i to the device
(``evs_copy_rows_async``), and the scatter of the chunk before. Each piece is gathered and copied
straight into its place in the chunk's ``[tables, rows, 2, d]`` layout, so that the copies can be
small (the pipeline fills and drains sooner) while the scatters are large (a launch's ramp and
tail weigh less). The copies run on a stream of their own, so the copy engine goes from one piece
to the next without waiting for a scatter; events order each scatter after its chunk's copies
and each chunk's copies after the scatter that last read its device buffer. The scatter takes the
chunk's slots as the store's (start, count) ranges (``evs_scatter_ranges``), copied with the
chunk: no slot ids are built or copied. Rows land byte for byte where ``write_rows`` puts them.
"""

from __future__ import annotations

import contextlib
import gc
import mmap
import os
import threading
import time
from dataclasses import dataclass
from typing import Iterable, Mapping, Sequence

import numpy as np
import torch

from everserve_amd.state.paged import PagedKV

HEAD_STRIDE = 1_000
"""A table id is layer * 1000 + head slot (core/everserve/state/mirror.py:59)."""


def destination_order(slots, block_size: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """A restore's (slot, staged row) pairs by increasing slot: ``(slots_sorted, rows_of)``.

    ``slots[t]`` is the cache slot staged row t goes to; a negative slot is padding and is dropped.
    Handed to ``scatter_pairs``, the pairs write each layer's cache front to back, which on MI355X
    is faster than writing in staged order when the staged order is a permutation of the cache's
    (a spare's fresh cache under a new block table). When the slots are whole blocks, block-size
    runs ``b * block_size + [0, block_size)``, only the blocks are ordered.
    """
    s = np.asarray(slots, dtype=np.int64).reshape(-1)
    if block_size and block_size > 1 and s.size and s.size % block_size == 0:
        runs = s.reshape(-1, block_size)
        first = runs[:, 0]
        if ((first >= 0).all() and not (first % block_size).any()
                and (runs == first[:, None] + np.arange(block_size, dtype=np.int64)).all()):
            blocks = np.argsort(first, kind="stable")
            rows_of = (blocks[:, None] * block_size
                       + np.arange(block_size, dtype=np.int64)).reshape(-1)
            return s[rows_of], rows_of
    keep = np.flatnonzero(s >= 0)
    rows_of = keep[np.argsort(s[keep], kind="stable")]
    return s[rows_of], rows_of


@dataclass
class Table:
    """One store table of the lost rank: its rows and the slots written in it.

    ``rows`` is the table's bytes, ``[num_slots, row_bytes]`` (a numpy array: in memory, as
    ``StoreTables`` holds them, or a read-only mapping of the table file); ``written`` the
    ``(start, count)`` slot ranges the store names (proto/everserve/proto/mirror.proto:102-117).
    The mapping lives as long as the Table. On the hosts measured, unmapping 128 MiB of shared
    memory costs 0.7-3.4 ms, as much as gathering it: drop the tables after the restore with
    :func:`release_later`, or map them ahead of a failure and keep them mapped.
    """

    table: int
    rows: np.ndarray
    written: Sequence[tuple[int, int]]

    @property
    def layer(self) -> int:
        return self.table // HEAD_STRIDE

    @property
    def head(self) -> int:
        return self.table % HEAD_STRIDE

    @classmethod
    def open(cls, table: int, path: str, written: Sequence[tuple[int, int]]) -> "Table":
        """The table file at ``path`` mapped read-only (its pages are read when gathered).

        The mapping is marked for sequential reading (``MADV_SEQUENTIAL``): a restore reads each
        table once, front to back. Linux then leaves the pages' LRU state alone on this mapping's
        faults and unmap; otherwise the first restore of freshly written tables moves their pages
        to the active list, page by page under the LRU lock, which made the first unmap of
        4 GiB of tables take 97-111 ms against 23-28 ms for later ones."""
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size == 0:
                return cls(table, np.empty(0, dtype=np.uint8), written)
            mapping = mmap.mmap(f.fileno(), size, flags=mmap.MAP_SHARED, prot=mmap.PROT_READ)
        try:
            mapping.madvise(mmap.MADV_SEQUENTIAL)
        except (OSError, AttributeError):
            pass  # an advice only: the copy is the same without it
        return cls(table, np.frombuffer(mapping, dtype=np.uint8), written)


@contextlib.contextmanager
def gc_paused():
    """Python's automatic garbage collection off for the block, back on after if it was on: a
    collection the block's allocations would set off runs after it instead. The switch is
    process-wide: a thread that turns collection off meanwhile finds it on again when the block
    ends."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def open_tables(tables: Iterable[tuple[int, str, Sequence[tuple[int, int]]]]) -> list["Table"]:
    """:meth:`Table.open` of each ``(table, path, written)``, with garbage collection paused."""
    with gc_paused():
        return [Table.open(t, path, written) for t, path, written in tables]


def reserve_descriptors(count: int) -> None:
    """Grow this process's file-descriptor table to hold ``count`` more descriptors than are open
    now: hold that many duplicates of one descriptor at once, then close them (Linux never shrinks
    the table). It stops early, without an error, at the process's descriptor limit: the growth
    only saves time."""
    if count <= 0:
        return
    fd = os.open(os.devnull, os.O_RDONLY)
    held: list[int] = []
    try:
        for _ in range(count):
            try:
                held.append(os.dup(fd))
            except OSError:
                break
    finally:
        for d in held:
            os.close(d)
        os.close(fd)


def release_later(tables: list) -> threading.Thread:
    """Drop the restored ``tables`` (the list is emptied) on a daemon thread, so that unmapping
    their files, which costs about as much as restoring them, does not hold up the rank that
    resumes. The mappings go when the thread drops the last references to them; CPython unmaps
    with the GIL released. Returns the thread, to join where the release must be complete."""
    held = list(tables)
    tables.clear()

    def drop() -> None:
        held.clear()

    th = threading.Thread(target=drop, daemon=True, name="everserve-restore-release")
    th.start()
    return th


@dataclass
class _Written:
    """A written list's ranges as the plan uses them: the non-empty ranges' starts and counts
    (an empty range writes nothing), whether any start or count is negative, the largest end
    over every range, and the non-empty ranges as bytes, for grouping."""

    source: Sequence[tuple[int, int]]
    starts: np.ndarray
    counts: np.ndarray
    negative: bool
    end: int
    key: bytes

    @classmethod
    def of(cls, written: Sequence[tuple[int, int]]) -> "_Written":
        w = np.asarray(written, dtype=np.int64).reshape(-1, 2)
        starts, counts = w[:, 0], w[:, 1]
        live = counts > 0
        s, c = starts[live].copy(), counts[live].copy()
        return cls(written, s, c, bool((starts < 0).any() or (counts < 0).any()),
                   int((starts + counts).max()) if len(w) else 0, s.tobytes() + c.tobytes())


@dataclass
class _Group:
    """Tables with the same written ranges, scattered together, one launch a chunk: the tables
    of ``layers`` (one layer, or several that fit one chunk together), layer after layer, each
    layer's in the order of ``heads``."""

    layers: list[int]
    starts: np.ndarray
    counts: np.ndarray
    tables: list[Table]
    heads: list[int]
    """The head slot each of a layer's tables is written into; the same for every layer."""


class Restorer:
    """Writes restored tables into ``layers`` (this rank's caches, in layer order).

    ``chunk_bytes`` is the rows one scatter launch writes over all of a group's tables, and
    ``piece_bytes`` the most rows one host gather and one copy to the device carry (a piece is
    an eighth of its group, but 16 MiB at least); two pinned and two device buffers of
    ``chunk_bytes`` are allocated, and the pinned ones touched, once, here: a spare builds its
    Restorer when it starts, before any failure. On MI355X, inside a restore from ``/dev/shm``, a
    scatter of 64 MiB ran at 4.9 TB/s, of 128 MiB at 5.4 and of 256 MiB at 5.7 (a launch's ramp
    and tail weigh on the shorter ones), while the restore as a whole, bound by the PCIe copies,
    ran 0.5-1 % slower with 256 MiB copies than with 64 MiB ones, which fill and drain the
    pipeline sooner: hence large chunks of small pieces. A catch-up's groups are small (128 MiB
    for every table after 16 decode steps): there 16 MiB pieces took 6.4-6.8 ms against 6.9-7.1
    with 64 MiB ones, and the first catch-up after 256 steps 45 ms against 48-49.

    ``scales`` (optional): this rank's per-layer fp32 scale array on the device, ``[L]`` or
    ``[L, k]``, for an fp8 cache; :meth:`restore` writes the scales that travelled beside the rows
    into it. The rows themselves move as raw bytes and are never rescaled.

    ``freeze_heap`` (default on): when built, the Restorer runs a full garbage collection and then
    freezes every object left (``gc.freeze``), so that a later full collection walks only the
    objects made since. A full collection walks every object the process holds, 40-70 ms on
    MI355X hosts with torch loaded, and opening a restore's 256 tables allocates enough to set one
    off: the first catch-up restore measured 40-63 ms of it in some runs and none in others. After
    the freeze one takes well under a millisecond. Frozen objects are still freed when their last
    reference goes, but a reference cycle among them is never collected: pass ``False`` to leave
    the collector as it is.
    """

    def __init__(self, ext, layers: Sequence[torch.Tensor], chunk_bytes: int = 256 << 20,
                 threads: int | None = None, scales: torch.Tensor | None = None,
                 piece_bytes: int = 64 << 20, freeze_heap: bool = True) -> None:
        first = layers[0]
        self._ext = ext
        self.layers = list(layers)
        self.device = first.device
        self._geometry = [PagedKV.of(t) for t in layers]
        self.paged = self._geometry[0]
        for t, g in zip(layers, self._geometry):
            if t.dtype != first.dtype or t.device != first.device:
                raise ValueError("every layer's cache must have one dtype and one device")
            if g.block_size != self.paged.block_size or g.head_dim != self.paged.head_dim:
                raise ValueError("every layer's cache must have one block size and head size")
        self._ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long,
                                  device=self.device)
        self._strides = [list(g.layout_strides(t)) for t, g in zip(layers, self._geometry)]
        self._elem = first.element_size()
        self._row_bytes = 2 * self.paged.head_dim * self._elem
        # a chunk carries at least one row of each of a group's tables, and a group has at most
        # one table per head slot
        most_heads = max(g.num_heads for g in self._geometry)
        self._chunk_bytes = max(most_heads * self._row_bytes,
                                chunk_bytes // self._row_bytes * self._row_bytes)
        self._piece_bytes = min(self._chunk_bytes, max(self._row_bytes, int(piece_bytes)))
        self._launches = 0
        self._gather_s = self._wait_s = 0.0
        self._threads = threads or min(16, len(os.sched_getaffinity(0)))
        self.scales = scales
        if scales is not None and (scales.device != self.device or scales.dtype != torch.float32
                                   or scales.shape[0] != len(layers)):
            raise ValueError("scales: a float32 device tensor with one entry per layer")
        nb, rows = self._chunk_bytes, self._chunk_bytes // self._row_bytes
        self._host = [torch.empty(nb, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        # a chunk's ranges: its starts, then its first rows (one more); a range holds a row or
        # more, so a chunk of n rows has at most n ranges
        self._host_ranges = [torch.empty(2 * rows + 1, dtype=torch.long, pin_memory=True)
                             for _ in range(2)]
        # The pinned buffers are touched here, every page, so that the first restore does not
        # pay for it: the pinned allocator torch uses on ROCm backs its pages on first touch,
        # which on MI355X hosts costs about 15 ms per 256 MiB (a later fill takes 3 ms).
        for t in (*self._host, *self._host_ranges):
            t.zero_()
        self._dev = [torch.empty(nb, dtype=torch.uint8, device=self.device) for _ in range(2)]
        self._dev_ranges = [torch.empty(2 * rows + 1, dtype=torch.long, device=self.device)
                            for _ in range(2)]
        self._heads: dict[tuple[int, ...], torch.Tensor] = {}
        self._layer_ptrs: dict[tuple[int, ...], torch.Tensor] = {}
        self._copy_stream = torch.cuda.Stream(device=self.device)
        # The first pitched copy to the device in a process, and the first on a new stream, set up
        # the copy engine's queue: about 6 and 3 ms on MI355X. One of a few bytes here keeps that
        # out of the first restore.
        w = min(64, nb // 3)
        if w > 0:
            with torch.cuda.stream(self._copy_stream):
                self._ext.copy_rows_async(self._dev[0].data_ptr(), self._host[0].data_ptr(), 2, w,
                                          2 * w, self.device)
            self._copy_stream.synchronize()
        # per buffer: its last copy to the device (the pinned buffer is free after it) and its last
        # scatter (the device buffer is free after it)
        self._copied: list[torch.cuda.Event | None] = [None, None]
        self._scattered: list[torch.cuda.Event | None] = [None, None]
        self.timing: dict[str, float] = {}
        self._lock = threading.Lock()  # one restore at a time owns the buffers and events
        # A restore maps one table per (layer, head slot), and each mapping keeps a descriptor of
        # its file open. Linux grows a process's descriptor table by doubling it, and in a process
        # of more than one thread each growth waits for an RCU grace period: 15-40 ms a doubling
        # on the hosts measured, so the first restore to hold 256 tables paid 50-90 ms in its
        # opens. The table is grown now, at the spare's start (a few spare descriptors past one
        # per table).
        reserve_descriptors(len(layers) * most_heads + 16)
        if freeze_heap:
            gc.collect()
            gc.freeze()

    def _head_list(self, heads: Sequence[int]) -> torch.Tensor:
        key = tuple(heads)
        if key not in self._heads:
            self._heads[key] = torch.tensor(key, dtype=torch.long, device=self.device)
        return self._heads[key]

    def _layer_list(self, layers: Sequence[int]) -> torch.Tensor:
        key = tuple(layers)
        if key not in self._layer_ptrs:
            self._layer_ptrs[key] = torch.tensor([self.layers[i].data_ptr() for i in key],
                                                 dtype=torch.long, device=self.device)
        return self._layer_ptrs[key]

    def plan(self, tables: Iterable[Table], head_map: Mapping[int, int]) -> list[_Group]:
        """Check every table against this rank's cache and group them; nothing is enqueued.

        A table whose head slot ``head_map`` does not name, or with nothing written, is skipped,
        as the reference skips it (core/everserve/state/mirror.py:922-925). The rest must fit:

        Raises:
            ValueError: a table of a layer this rank does not have; a head slot outside the
                layer's heads; a table that is not whole rows of this cache's row size; a written
                range outside the table or past the cache's last slot; two tables written into
                one (layer, head slot).
        """
        rb = self._row_bytes
        groups: dict[tuple, _Group] = {}
        taken: set[tuple[int, int]] = set()
        # What a written list yields, worked out once per list (a store commit hands every table
        # of a step the same one): the catch-up after 16 decode steps checks 256 tables of 125
        # ranges each, which took 3.8 ms table by table and takes 0.8 ms with the list's work
        # done once (one x86 host).
        ranges: dict[int, _Written] = {}  # by the written list's identity
        for table in tables:
            if table.head not in head_map or not table.written:
                continue
            name = f"table {table.table}"
            layer = table.layer
            if not 0 <= layer < len(self.layers):
                raise ValueError(f"{name}: layer {layer}, but this rank has "
                                 f"{len(self.layers)} layers")
            geo = self._geometry[layer]
            head = int(head_map[table.head])
            if not 0 <= head < geo.num_heads:
                raise ValueError(f"{name}: head slot {head} outside the layer's "
                                 f"{geo.num_heads} heads")
            if (layer, head) in taken:
                raise ValueError(f"{name}: another table is already restored into layer "
                                 f"{layer}, head slot {head}")
            taken.add((layer, head))
            rows = table.rows
            if rows.nbytes % rb or (rows.ndim == 2 and rows.shape[1] * rows.itemsize != rb):
                raise ValueError(f"{name}: not a whole number of this cache's {rb}-byte rows")
            w = ranges.get(id(table.written))
            if w is None or w.source is not table.written:
                w = ranges[id(table.written)] = _Written.of(table.written)
            if w.negative or w.end > rows.nbytes // rb:
                raise ValueError(f"{name}: a written range lies outside the table")
            if w.end > geo.num_slots:
                raise ValueError(f"{name}: a written range ends at slot {w.end}, past "
                                 f"this cache's {geo.num_slots} slots")
            if not len(w.starts):
                continue
            key = (layer, w.key, rows.nbytes)
            g = groups.get(key)
            if g is None:
                g = groups[key] = _Group([layer], w.starts, w.counts, [], [])
            g.tables.append(table)
            g.heads.append(head)
        return self._merge(list(groups.values()))

    def _merge(self, groups: list[_Group]) -> list[_Group]:
        """Join groups of different layers that have the same ranges, head slots and layout
        strides into one group while their rows fit one chunk together: one launch then writes
        them all. A catch-up after a few decode steps has a few MiB per layer, which one layer a
        launch would spend on per-launch costs; a full restore's layers fill chunks by
        themselves and stay apart."""
        rb = self._row_bytes
        by_key: dict[tuple, list[_Group]] = {}
        for g in groups:
            order = np.argsort(g.heads, kind="stable")
            g.heads = [g.heads[i] for i in order]
            g.tables = [g.tables[i] for i in order]
            key = (g.starts.tobytes(), g.counts.tobytes(), g.tables[0].rows.nbytes,
                   tuple(g.heads), tuple(self._strides[g.layers[0]]))
            by_key.setdefault(key, []).append(g)
        out: list[_Group] = []
        for same in by_key.values():
            rows = int(same[0].counts.sum())
            one = rows * len(same[0].heads) * rb  # a layer's bytes
            per = max(1, self._chunk_bytes // one) if one else 1
            for i in range(0, len(same), per):
                part = same[i:i + per]
                out.append(_Group([layer for g in part for layer in g.layers], part[0].starts,
                                  part[0].counts, [t for g in part for t in g.tables],
                                  list(part[0].heads)))
        out.sort(key=lambda g: g.layers[0])
        return out

    def restore(self, tables: Iterable[Table], head_map: Mapping[int, int],
                scales: Mapping[int, Sequence[float]] | None = None) -> int:
        """Write every table whose head slot ``head_map`` names into its new head slot, and the
        per-layer ``scales`` (layer -> values) into this rank's scale array.

        Every table is checked first (:meth:`plan`); a refused restore writes nothing. Returns the
        rows written, over every table. Synchronises the device at the end, as the reference's
        restore does (core/everserve/state/mirror.py:938-939). Restores through one Restorer from
        several threads run one after another: they share its buffers. Python's automatic garbage
        collection is paused while it runs (:func:`gc_paused`).
        """
        with self._lock, gc_paused():
            return self._restore(tables, head_map, scales)

    def _restore(self, tables: Iterable[Table], head_map: Mapping[int, int],
                 scales: Mapping[int, Sequence[float]] | None) -> int:
        t0 = time.perf_counter()
        groups = self.plan(tables, head_map)
        side = None
        if scales:
            if self.scales is None:
                raise ValueError("scales given, but this Restorer has no scale array")
            side = {int(k): np.asarray(v, dtype=np.float32).reshape(self.scales.shape[1:])
                    for k, v in scales.items()}
            if any(not 0 <= k < len(self.layers) for k in side):
                raise ValueError("scales name a layer this rank does not have")
        stream = torch.cuda.current_stream(self.device)
        total = 0
        buf = 0
        self._launches = 0
        self._gather_s = self._wait_s = 0.0
        for g in groups:
            rows, buf = self._restore_group(g, stream, buf)
            total += rows * len(g.tables)
        if side:
            with torch.inference_mode():
                for layer, v in side.items():
                    self.scales[layer].copy_(torch.from_numpy(v), non_blocking=False)
        t1 = time.perf_counter()
        torch.cuda.synchronize(self.device)
        t2 = time.perf_counter()
        rb = self._row_bytes
        self.timing = {"copy_s": t2 - t0, "rows": total, "bytes": total * rb,
                       "launches": self._launches, "host_gather_s": self._gather_s,
                       "buffer_wait_s": self._wait_s, "final_sync_s": t2 - t1}
        return total

    @staticmethod
    def _ranges(g: _Group, first_row: np.ndarray, r0: int, r1: int) -> tuple[np.ndarray,
                                                                             np.ndarray]:
        """The group's ranges trimmed to its rows [r0, r1) (``first_row``: each range's first
        row in the group's order): (starts, counts)."""
        k0 = int(np.searchsorted(first_row, r0, side="right")) - 1
        k1 = int(np.searchsorted(first_row, r1, side="left"))
        st = g.starts[k0:k1].copy()
        ct = g.counts[k0:k1].copy()
        skip = r0 - first_row[k0]
        st[0] += skip
        ct[0] -= skip
        ct[-1] -= first_row[k1] - r1
        return st, ct

    def _restore_group(self, g: _Group, stream, buf: int) -> tuple[int, int]:
        """Enqueue one group's chunks, the first into buffer ``buf``: every table's rows of a
        slot range gathered on the host side by side and copied to the device, a piece at a time,
        then scattered into all of the group's head slots in one launch. Returns the rows
        enqueued per table and the buffer the next chunk takes."""
        rb, k = self._row_bytes, len(g.tables)
        first_row = np.concatenate([[0], np.cumsum(g.counts)])
        rows = int(first_row[-1])
        layer = g.layers[0]
        layer_ptrs = self._layer_list(g.layers)
        heads = self._head_list(g.heads)
        srcs = [t.rows.ctypes.data for t in g.tables]
        table_rows = g.tables[0].rows.nbytes // rb
        per_chunk = max(1, self._chunk_bytes // (k * rb))
        # pieces of an eighth of the group, but 16 MiB at least and piece_bytes at most: the
        # pipeline's fill (the first piece's gather) and drain (the last piece's copy) are then a
        # small part of a small group too
        piece = min(self._piece_bytes, max(16 << 20, rows * k * rb // 8))
        per_piece = max(1, piece // (k * rb))
        if k * per_chunk * rb > self._chunk_bytes:
            raise RuntimeError(f"layer {layer}: a chunk of {k} tables x {per_chunk} rows does "
                               f"not fit the {self._chunk_bytes}-byte buffers")
        for c0 in range(0, rows, per_chunk):
            c1 = min(rows, c0 + per_chunk)
            n = c1 - c0
            if self._copied[buf] is not None:
                w0 = time.perf_counter()
                self._copied[buf].synchronize()  # the copies out of this pinned buffer are done
                self._wait_s += time.perf_counter() - w0
            host, dev = self._host[buf].data_ptr(), self._dev[buf].data_ptr()
            # the chunk is [k, n, 2, d]: staged rows of k head slots at capacity n; a piece is
            # rows [p0, p1) of every table, k runs n rows apart
            for p0 in range(c0, c1, per_piece):
                p1 = min(c1, p0 + per_piece)
                st, ct = self._ranges(g, first_row, p0, p1)
                off = (p0 - c0) * rb
                g0 = time.perf_counter()
                got = self._ext.host_gather_tables(srcs, table_rows, rb, st, ct, host + off, n,
                                                   self._threads)
                self._gather_s += time.perf_counter() - g0
                if got != p1 - p0:
                    raise RuntimeError(f"layer {layer}: gathered {got} rows of [{p0}, {p1})")
                with torch.cuda.stream(self._copy_stream):
                    if p0 == c0 and self._scattered[buf] is not None:
                        self._copy_stream.wait_event(self._scattered[buf])
                    self._ext.copy_rows_async(dev + off, host + off, k, (p1 - p0) * rb, n * rb,
                                              self.device)
            st, ct = self._ranges(g, first_row, c0, c1)
            r = len(st)
            ranges = self._host_ranges[buf].numpy()
            ranges[:r] = st
            ranges[r] = 0
            np.cumsum(ct, out=ranges[r + 1:2 * r + 1])
            with torch.cuda.stream(self._copy_stream):
                self._ext.copy_rows_async(self._dev_ranges[buf].data_ptr(),
                                          self._host_ranges[buf].data_ptr(), 1, (2 * r + 1) * 8,
                                          (2 * r + 1) * 8, self.device)
                self._copied[buf] = self._copy_stream.record_event()
            stream.wait_event(self._copied[buf])
            dr = self._dev_ranges[buf]
            self._ext.scatter_ranges(layer_ptrs, dr[:r], dr[r:2 * r + 1], n, heads, dev, n,
                                     self.paged.head_dim, self.paged.block_size,
                                     self._strides[layer], self._elem)
            self._scattered[buf] = stream.record_event()
            self._launches += 1
            buf ^= 1
        return rows, buf
