"""The restore's copy into this rank's cache: a lost rank's store tables to the paged cache.

The reference's loop (core/everserve/state/mirror.py:916-939) takes each table the store names,
maps it from shared memory as ``[num_slots, 2, d]``, gathers the written rows on the host with
``torch.index_select`` into pinned memory, copies them to the device and scatters them with
``PagedKV.write_rows`` into the head slot the rank assigned. Published at 2.1-2.6 GB/s
(bench/runs/2026-10-05-shm-commit-4gpu/RESULT.md:36,45-46): the host gather bounds it.

:class:`Restorer` does the same table by table, in chunks, and keeps three things busy at once:
host threads gathering chunk i+1's rows into one pinned buffer (``evs_host_gather_ranges``), the
copy engine moving chunk i from the other pinned buffer to the device (``evs_copy_rows_async``),
and the scatter kernel writing chunk i-1 into the cache (``evs_scatter_rows``). The copies run on
a stream of their own, so the copy engine goes from one chunk to the next without waiting for
the scatter of the previous one; events order each scatter after its copy and each copy after
the scatter that last read its device buffer. A chunk of one slot range gets its slot ids from
``torch.arange`` on the device instead of a second copy. Rows land byte for byte where
``write_rows`` puts them.
"""

from __future__ import annotations

import os
import threading
import time
from dataclasses import dataclass
from typing import Iterable, Mapping, Sequence

import numpy as np
import torch

from everserve_amd.state.kvcopy import PagedKV

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
    memory costs 0.8-3.4 ms, as much as gathering it: drop the tables after the restore with
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
        """The table file at ``path`` mapped read-only (its pages are read when gathered)."""
        return cls(table, np.memmap(path, dtype=np.uint8, mode="r"), written)


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


class Restorer:
    """Writes restored tables into ``layers`` (this rank's caches, in layer order)."""

    def __init__(self, ext, layers: Sequence[torch.Tensor], chunk_bytes: int = 64 << 20,
                 threads: int | None = None) -> None:
        first = layers[0]
        self._ext = ext
        self.layers = list(layers)
        self.paged = PagedKV.of(first)
        self.device = first.device
        self._ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long,
                                  device=self.device)
        self._strides = list(self.paged.layout_strides(first))
        self._elem = first.element_size()
        self._row_bytes = 2 * self.paged.head_dim * self._elem
        self._chunk_rows = max(1, chunk_bytes // self._row_bytes)
        self._threads = threads or min(16, len(os.sched_getaffinity(0)))
        n, rb = self._chunk_rows, self._row_bytes
        self._host = [torch.empty(n * rb, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self._host_slots = [torch.empty(n, dtype=torch.long, pin_memory=True) for _ in range(2)]
        self._dev = [torch.empty(n * rb, dtype=torch.uint8, device=self.device) for _ in range(2)]
        self._dev_slots = [torch.empty(n, dtype=torch.long, device=self.device) for _ in range(2)]
        self._heads: dict[int, torch.Tensor] = {}
        self._copy_stream = torch.cuda.Stream(device=self.device)
        # per buffer: its last copy to the device (the pinned buffer is free after it) and its last
        # scatter (the device buffer is free after it)
        self._copied: list[torch.cuda.Event | None] = [None, None]
        self._scattered: list[torch.cuda.Event | None] = [None, None]
        self.timing: dict[str, float] = {}

    def _head(self, h: int) -> torch.Tensor:
        if h not in self._heads:
            self._heads[h] = torch.tensor([h], dtype=torch.long, device=self.device)
        return self._heads[h]

    def restore(self, tables: Iterable[Table], head_map: Mapping[int, int]) -> int:
        """Write every table whose head slot ``head_map`` names into its new head slot.

        Returns the rows written, over every table. Synchronises the device at the end, as the
        reference's restore does (core/everserve/state/mirror.py:938-939).
        """
        t0 = time.perf_counter()
        stream = torch.cuda.current_stream(self.device)
        rb = self._row_bytes
        total = 0
        buf = 0
        for table in tables:
            if table.head not in head_map or not table.written:
                continue
            nbytes = table.rows.nbytes
            if nbytes % rb:
                raise ValueError(f"table {table.table}: {nbytes} bytes is not a whole "
                                 f"number of {rb}-byte rows")
            starts = np.array([s for s, _ in table.written], dtype=np.int64)
            counts = np.array([c for _, c in table.written], dtype=np.int64)
            if (starts < 0).any() or (counts < 0).any() or \
                    (starts + counts).max() * rb > nbytes:
                raise ValueError(f"table {table.table}: a written range lies outside the table")
            rows, buf = self._restore_table(table, starts, counts, head_map[table.head], stream,
                                            buf)
            total += rows
        torch.cuda.synchronize(self.device)
        self.timing = {"copy_s": time.perf_counter() - t0, "rows": total,
                       "bytes": total * rb}
        return total

    def _restore_table(self, table: Table, starts: np.ndarray, counts: np.ndarray,
                       new_head: int, stream, buf: int) -> tuple[int, int]:
        """Enqueue one table's chunks, the first into buffer ``buf``: gathered from its rows,
        copied to the device, scattered at head slot ``new_head``. Returns the rows enqueued and
        the buffer the next chunk takes."""
        rb, n_chunk = self._row_bytes, self._chunk_rows
        first_row = np.concatenate([[0], np.cumsum(counts)])
        rows = int(first_row[-1])
        layer_ptr = self._ptrs[table.layer:table.layer + 1]
        head = self._head(new_head)
        for c0 in range(0, rows, n_chunk):
            c1 = min(rows, c0 + n_chunk)
            n = c1 - c0
            # the ranges, trimmed to output rows [c0, c1)
            k0 = int(np.searchsorted(first_row, c0, side="right")) - 1
            k1 = int(np.searchsorted(first_row, c1, side="left"))
            st = starts[k0:k1].copy()
            ct = counts[k0:k1].copy()
            skip = c0 - first_row[k0]
            st[0] += skip
            ct[0] -= skip
            ct[-1] -= first_row[k1] - c1 if k1 <= len(counts) else 0
            if self._copied[buf] is not None:
                self._copied[buf].synchronize()  # the copy out of this pinned buffer is done
            got = self._ext.host_gather_ranges(table.rows.ctypes.data, table.rows.nbytes // rb,
                                               rb, st, ct, self._host[buf].data_ptr(), n_chunk,
                                               self._threads)
            if got != n:
                raise RuntimeError(f"table {table.table}: gathered {got} rows of chunk "
                                   f"[{c0}, {c1})")
            one_range = len(st) == 1
            if not one_range:
                slots = self._host_slots[buf].numpy()
                at = 0
                for s, c in zip(st.tolist(), ct.tolist()):
                    slots[at:at + c] = np.arange(s, s + c, dtype=np.int64)
                    at += c
            with torch.cuda.stream(self._copy_stream):
                if self._scattered[buf] is not None:
                    self._copy_stream.wait_event(self._scattered[buf])
                self._ext.copy_rows_async(self._dev[buf].data_ptr(), self._host[buf].data_ptr(),
                                          1, n * rb, n * rb, self.device)
                if not one_range:
                    self._dev_slots[buf][:n].copy_(self._host_slots[buf][:n], non_blocking=True)
                self._copied[buf] = self._copy_stream.record_event()
            if one_range:
                torch.arange(int(st[0]), int(st[0]) + n, dtype=torch.long, device=self.device,
                             out=self._dev_slots[buf][:n])
            stream.wait_event(self._copied[buf])
            self._ext.scatter_rows(layer_ptr, self._dev_slots[buf][:n], head,
                                   self._dev[buf].data_ptr(), n, self.paged.head_dim,
                                   self.paged.block_size, self._strides, self._elem)
            self._scattered[buf] = stream.record_event()
            buf ^= 1
        return rows, buf
