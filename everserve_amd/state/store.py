"""The node store's tables for one rank, in this process: the commit copy and what a restore reads.

The store is the reference's Rust service (store/src/storage.rs). This module is its data path for
one rank, over the library's host commit (``evs_store_commit``), for a store that runs in this
process or links this library:

* :meth:`StoreTables.commit` takes one ``StagedStep`` and its staged bytes (what
  :class:`everserve_amd.state.staging.StepStager` hands its sink). It copies every table's rows,
  runs of consecutive slots as one copy, and records each written slot's step and the CRC32C of
  its row (``Storage::commit``, storage.rs:864-957; ``Layer::mark_written``, :494-504). The
  tables are committed on host threads.
* :meth:`StoreTables.written_ranges` and :meth:`StoreTables.restore_tables` are what a restore
  reads back: ``Layer::written_ranges`` (:430-451), as :class:`everserve_amd.state.restore.Table`
  objects.
* An fp8 cache's per-layer scales are not in the rows. When a staged step carries them
  (``job.scales``), the tables keep the latest beside the rows (:meth:`StoreTables.restore_scales`),
  for the restore to write into the new cache's scale array.

Tables are created on first use: ``num_slots * row_bytes`` bytes, zeroed, with every page touched
at creation so that the first commit into them pays no page faults (``Layer::create``,
:379-415). They are ``table<id>.rows`` files in ``directory`` when one is given, else anonymous
memory.
"""

from __future__ import annotations

import os
import threading
from dataclasses import dataclass, field
from pathlib import Path
from typing import Mapping

import numpy as np

from everserve_amd.state.restore import Table

DTYPE_BYTES = {
    "float8_e4m3fn": 1, "float8_e5m2": 1, "int8": 1, "uint8": 1,
    "float16": 2, "bfloat16": 2, "int16": 2, "float32": 4, "int32": 4, "float64": 8, "int64": 8,
}
"""Element bytes per dtype name (store/src/storage.rs:542-551)."""


def derive(step: Mapping) -> list[tuple[int, int]]:
    """(table id, byte offset of its first row) for every (layer, head) a descriptor names.

    store/src/storage.rs:521-540: the table id is ``layer * table_stride + head slot``; the rows
    of head index h of layer ``l`` start at ``base_offset + l * layer_stride + h * head_stride``.
    """
    out = []
    for layer in step["layers"]:
        for h, head in enumerate(step["heads"]):
            out.append((int(layer) * int(step["table_stride"]) + int(head),
                        int(step["base_offset"]) + int(layer) * int(step["layer_stride"])
                        + h * int(step["head_stride"])))
    return out


def row_bytes_of(step: Mapping) -> int:
    """Bytes of one row a descriptor names: the product of its shape times the element size."""
    n = 1
    for x in step["shape"]:
        n *= int(x)
    if step["dtype"] not in DTYPE_BYTES:
        raise ValueError(f"unknown dtype {step['dtype']!r}")
    return n * DTYPE_BYTES[step["dtype"]]


@dataclass
class StoreTable:
    """One table: its rows, and per slot the step of the last write (0: never) and its CRC32C."""

    table: int
    row_bytes: int
    rows: np.ndarray
    written_step: np.ndarray
    crc: np.ndarray
    path: Path | None = field(default=None)

    def holds_rows(self) -> bool:
        """Whether any slot has been written (``Layer::holds_rows``, storage.rs:418-421)."""
        return bool(self.written_step.any())


class StoreTables:
    """The tables of one rank, created on first use; ``num_slots`` per table."""

    def __init__(self, ext, num_slots: int, directory: str | os.PathLike | None = None,
                 threads: int | None = None) -> None:
        if num_slots <= 0:
            raise ValueError(f"num_slots must be positive, got {num_slots}")
        self._ext = ext
        self.num_slots = int(num_slots)
        self.directory = Path(directory) if directory is not None else None
        if self.directory is not None:
            self.directory.mkdir(parents=True, exist_ok=True)
        self.threads = threads or min(16, len(os.sched_getaffinity(0)))
        self.tables: dict[int, StoreTable] = {}
        self.step = 0
        self.scales: np.ndarray | None = None
        """The per-layer scales of the latest step that carried them."""
        self._plans: dict[tuple, object] = {}
        """Per table set a descriptor names, the commit's arguments built once (tables are
        never replaced once created)."""
        self._lock = threading.RLock()
        """Commits (the stager's copy thread) and reads (a restore, another thread) take turns
        on the table set; the rows a restore reads are the store's to keep still, as they are
        for the Rust store (no commit reaches a lost rank's tables)."""

    def _create(self, table: int, row_bytes: int) -> StoreTable:
        nbytes = self.num_slots * row_bytes
        path = None
        if self.directory is not None:
            path = self.directory / f"table{table}.rows"
            rows = np.memmap(path, dtype=np.uint8, mode="w+", shape=(nbytes,))
        else:
            rows = np.zeros(nbytes, dtype=np.uint8)
        rows[::4096] = 0  # touch every page now, not at the first commit
        t = StoreTable(table, row_bytes, rows, np.zeros(self.num_slots, dtype=np.uint64),
                       np.zeros(self.num_slots, dtype=np.uint32), path)
        self.tables[table] = t
        return t

    def commit(self, stage: np.ndarray, step: Mapping, step_no: int) -> int:
        """Copy one staged step's rows into its tables; the slots written for the first time.

        ``stage`` is the staged bytes (uint8), ``step`` the ``StagedStep`` descriptor. Every slot
        id and table must fit before anything is written, as the store checks a descriptor first.
        """
        with self._lock:
            return self._commit(stage, step, step_no)

    def _commit(self, stage: np.ndarray, step: Mapping, step_no: int) -> int:
        stage = np.ascontiguousarray(stage).view(np.uint8).reshape(-1)
        rb = row_bytes_of(step)
        key = (tuple(step["layers"]), tuple(step["heads"]), int(step["table_stride"]),
               int(step["base_offset"]), int(step["layer_stride"]), int(step["head_stride"]), rb)
        plan = self._plans.get(key)
        if plan is None:
            tables = derive(step)
            for table, _ in tables:
                have = self.tables.get(table)
                if have is not None and have.row_bytes != rb:
                    raise ValueError(f"table {table} holds rows of {have.row_bytes} bytes, the "
                                     f"step names {rb}")
        slots = np.asarray(step["slots"], dtype=np.int64)
        if slots.size and int(slots.max()) >= self.num_slots:
            raise ValueError(f"slot {int(slots.max())} outside 0..{self.num_slots}")
        if plan is None:
            made = [self.tables.get(t) or self._create(t, rb) for t, _ in tables]
            plan = self._plans[key] = self._ext.store_commit_plan(
                [off for _, off in tables], [t.rows for t in made],
                [t.written_step for t in made], [t.crc for t in made], self.num_slots, rb)
        fresh = self._ext.store_commit_with(plan, stage, slots, step_no, self.threads)
        self.step = max(self.step, int(step_no))
        return fresh

    def written_ranges(self, table: int, since_step: int = 0) -> list[tuple[int, int]]:
        """(start, count) runs of the slots written after ``since_step`` (storage.rs:430-451)."""
        with self._lock:
            hit = self.tables[table].written_step > since_step
        if not hit.any():
            return []
        edges = np.flatnonzero(np.diff(np.concatenate(([0], hit.view(np.int8), [0]))))
        return [(int(a), int(b - a)) for a, b in zip(edges[0::2], edges[1::2])]

    def restore_tables(self, since_step: int = 0) -> list[Table]:
        """Every table that holds rows written after ``since_step``, as a restore reads them."""
        out = []
        with self._lock:
            for tid in sorted(self.tables):
                ranges = self.written_ranges(tid, since_step)
                if ranges:
                    out.append(Table(tid, self.tables[tid].rows, ranges))
        return out

    def crc(self, table: int, slot: int) -> int:
        """The CRC32C recorded for one row when it was written; 0 for a slot never written."""
        return int(self.tables[table].crc[slot])

    def flush(self) -> None:
        """Write file-backed tables through to their files."""
        with self._lock:
            for t in self.tables.values():
                if isinstance(t.rows, np.memmap):
                    t.rows.flush()

    def restore_scales(self) -> dict[int, np.ndarray]:
        """Layer -> its scales as last committed; empty when no step carried any."""
        with self._lock:
            if self.scales is None:
                return {}
            return {layer: v.copy() for layer, v in enumerate(self.scales)}

    def sink(self, job) -> None:
        """A :class:`everserve_amd.state.staging.StepStager` sink: commit each staged step."""
        if job.descriptor is not None:
            self.commit(job.stage_bytes, job.descriptor, job.step)
        if getattr(job, "scales", None) is not None:
            with self._lock:
                self.scales = np.array(job.scales, dtype=np.float32, copy=True)
