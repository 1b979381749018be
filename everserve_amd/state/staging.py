"""The per-step snapshot: a step's committed rows, every layer and held head, into a staging file.

The reference's step path is ``MirrorCommittedKV.save`` / ``commit`` / ``_gather_step`` /
``_staging`` / ``_describe`` (core/everserve/state/mirror.py:536-800) over ``_GatherKernel``
(mirror.py:311-370). There, layers are marked as the forward runs. ``commit`` orders a side
stream after the forward with an event and launches one ``gather_rows`` that writes the rows
straight into a host-mapped staging file, ``<rank_dir>/<prefix><k>.rows`` in shared memory, over
PCIe. A sender thread waits for the side stream and sends the step's ``StagedStep`` descriptor to
the node's store, which maps the file by the descriptor's ``stage`` name (store/src/shm.rs:39-45)
and copies the named rows into its tables (store/src/storage.rs:864-957).

:class:`StepStager` keeps that interface, the staging files and the descriptor, and moves the data
differently:

* **The gather runs on the producing stream**, right behind the forward's last write, into a
  staging buffer in HBM (``evs_gather_rows``, one launch for every layer). At decode sizes it
  is a few microseconds of HBM time.
* **A fence-less event** (``evs_event_create(0)``) is recorded behind it. This costs the step
  thread a few microseconds and the device nothing.
* **A copy thread** waits for that event on the host. Only then does it deliver the step's rows
  into the stage's file (``evs_deliver_rows``): the copy engine moves them in batches into two
  pinned bounce buffers in turn, on the thread's own stream, while host threads copy the previous
  batch into the file with nontemporal stores. The file is mapped shared, so the bytes are the
  store's to read as soon as the call returns. Then the thread calls the caller's ``sink`` with
  the step's descriptor, whose ``stage`` names the file.

Registering the file for the device would let the copy engine write it directly, but this GPU
pool refuses ``hipHostRegister`` of existing memory, so the file is filled through pinned bounce
buffers instead.

Why no stream waits on another: on MI355X, a stream that waits on a pending event from another
stream (``hipStreamWaitEvent``) slowed the Llama-3-8B-shaped decode step it followed by about
260 us. That held with or without the event's system-scope fence. An already-completed event
costs about nothing to wait on. Here no device queue ever waits on another.

Staging files are pooled as in the reference (mirror.py:588-642): capacities are
``max(8, next_pow2(n))``, at most ``depth + 1`` files are kept and the rest are deleted. A file
returns to the pool only after its sink has returned, so a gather never overwrites rows the store
has not taken.

fp8 caches carry per-layer scales that are not part of the rows: the rows move as raw bytes.
Given ``scales`` (a float32 array on the device, one entry or one row per layer), the stager
snapshots them with each step's gather and writes them into the staging file after the rows,
where the descriptor (and so the store) does not look; the sink gets them as ``job.scales``.
"""

from __future__ import annotations

import mmap
import os
import queue
import tempfile
import threading
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Mapping, Sequence

import numpy as np
import torch

from everserve_amd.state.paged import HeadSlot, PagedKV, layer_index

HEAD_STRIDE = 1_000
"""Table id = layer * 1000 + head slot (core/everserve/state/mirror.py:59)."""

DTYPE_NAMES = {
    torch.bfloat16: "bfloat16",
    torch.float16: "float16",
    torch.float32: "float32",
    torch.float8_e4m3fn: "float8_e4m3fn",
    torch.float8_e5m2: "float8_e5m2",
    torch.int8: "int8",
    torch.uint8: "uint8",
}
"""The dtype names the store knows (core/everserve/state/mirror.py:49-58)."""


class StagingError(Exception):
    """A staged step failed on the copy thread; raised on the step thread at the next call."""


def capacity_for(n: int) -> int:
    """Rows a staging buffer holds for a step of ``n`` slots (core/everserve/state/mirror.py:596)."""
    if n < 1:
        raise ValueError(f"a step stages at least one slot, got {n}")
    return max(8, 1 << (n - 1).bit_length())


def describe(stage: str, layers: Sequence[int], heads: Sequence[HeadSlot], capacity: int,
             head_dim: int, elem: int, slots: Sequence[int], dtype: str) -> dict:
    """The ``StagedStep`` descriptor of rows staged as ``[L, H, capacity, 2, d]``.

    Field for field core/everserve/state/mirror.py:778-800 (proto/everserve/proto/mirror.proto:
    32-54). Row t of (layer ``l``, head index ``h``) is at ``l * layer_stride + h * head_stride +
    t * row_bytes``. Negative slot ids are padding, which the store skips.
    """
    row_bytes = 2 * head_dim * elem
    return {
        "stage": stage,
        "base_offset": 0,
        "layer_stride": len(heads) * capacity * row_bytes,
        "head_stride": capacity * row_bytes,
        "layers": sorted(int(x) for x in layers),
        "heads": [int(h) for h in heads],
        "table_stride": HEAD_STRIDE,
        "slots": (slots.astype(np.int64, copy=False).tolist() if isinstance(slots, np.ndarray)
                  else [int(s) for s in slots]),
        "dtype": dtype,
        "shape": [2, head_dim],
    }


class GatherKernel:
    """A step's gather as launches of ``gather_rows``, for the caches of one rank.

    Same role as the reference's ``_GatherKernel`` (core/everserve/state/mirror.py:311-370). It
    holds the layers' base addresses on the device and each layer's five strides. When every
    layer shares one shape, stride and dtype (the normal case), a step of every layer is one
    launch. Otherwise each layer is its own launch with its own strides, still the same kernel:
    the reference's torch path per layer has no counterpart here.
    """

    def __init__(self, ext, layers: Sequence[torch.Tensor], paged: PagedKV) -> None:
        first = layers[0]
        if any(t.dtype != first.dtype for t in layers):
            raise ValueError("every layer's cache must have one dtype")
        if any(t.device != first.device for t in layers):
            raise ValueError("every layer's cache must be on one device")
        self._ext = ext
        self.paged = paged
        self.device = first.device
        self._ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long,
                                  device=first.device)
        self._strides = [tuple(PagedKV.of(t).layout_strides(t)) for t in layers]
        for t in layers:
            p = PagedKV.of(t)
            if p.block_size != paged.block_size or p.head_dim != paged.head_dim:
                raise ValueError("every layer's cache must have one block size and head size")
        self.uniform = all(s == self._strides[0] for s in self._strides)
        self.elem = first.element_size()
        self.num_layers = len(layers)

    def gather(self, slots: torch.Tensor, heads: torch.Tensor, out_ptr: int, capacity: int,
               layers: Sequence[int] | None = None) -> None:
        """Write rows ``[0, n)`` of every listed layer (all by default) into ``[L, H, capacity, 2, d]``
        at ``out_ptr``, on the current stream."""
        d, bs = self.paged.head_dim, self.paged.block_size
        every = layers is None or len(layers) == self.num_layers
        if every and self.uniform:
            self._ext.gather_rows(self._ptrs, slots, heads, out_ptr, capacity, d, bs,
                                  self._strides[0], self.elem)
            return
        layer_bytes = heads.numel() * capacity * 2 * d * self.elem
        for layer in (range(self.num_layers) if layers is None else sorted(layers)):
            self._ext.gather_rows(self._ptrs[layer:layer + 1], slots, heads,
                                  out_ptr + layer * layer_bytes, capacity, d, bs,
                                  self._strides[layer], self.elem)

    def gather_blocks(self, block_ids: torch.Tensor, heads: torch.Tensor, out_ptr: int,
                      capacity: int, slots_out: torch.Tensor) -> None:
        """Write every slot of ``block_ids`` (int32), block by block, for every layer into
        ``[L, H, capacity, 2, d]`` at ``out_ptr``, and the slot ids into ``slots_out``."""
        d, bs = self.paged.head_dim, self.paged.block_size
        if self.uniform:
            self._ext.gather_blocks(self._ptrs, block_ids, heads, out_ptr, capacity, d, bs,
                                    self._strides[0], self.elem, slots_out=slots_out)
            return
        layer_bytes = heads.numel() * capacity * 2 * d * self.elem
        for layer in range(self.num_layers):
            self._ext.gather_blocks(self._ptrs[layer:layer + 1], block_ids, heads,
                                    out_ptr + layer * layer_bytes, capacity, d, bs,
                                    self._strides[layer], self.elem, slots_out=slots_out)


_MADV_POPULATE_WRITE = 23  # Linux 5.14: fault every page of a range in, writable, at once


def _map_stage_file(path: Path, nbytes: int) -> mmap.mmap:
    """Create ``path`` (``nbytes``, the node's group may read it) and map it shared, every page
    faulted in now rather than at the first delivery into it."""
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o660)
    try:
        os.fchmod(fd, 0o660)  # the store runs as another user of the node's group
        os.ftruncate(fd, nbytes)
        mapping = mmap.mmap(fd, nbytes, flags=mmap.MAP_SHARED)
    finally:
        os.close(fd)
    try:
        mapping.madvise(_MADV_POPULATE_WRITE)
    except (OSError, ValueError):
        np.frombuffer(mapping, dtype=np.uint8)[::mmap.PAGESIZE] = 0  # older kernels: touch
    return mapping


@dataclass
class Stage:
    """One pooled staging buffer: ``[L, H, capacity, 2, d]`` rows in HBM, and the staging file
    ``path`` the rows are delivered into (the rows, then the scale side array, if any)."""

    name: str
    path: Path
    capacity: int
    num_heads: int
    rows_bytes: int
    mapping: mmap.mmap
    device_rows: torch.Tensor
    device_slots: torch.Tensor
    host_slots: torch.Tensor
    device_blocks: torch.Tensor
    host_blocks: torch.Tensor
    """Block ids of a block round, staged through pinned memory so their upload never waits."""
    device_scales: torch.Tensor | None = None
    host_scales: torch.Tensor | None = None

    @property
    def file_addr(self) -> int:
        """The address of the file's mapping in this process."""
        return np.frombuffer(self.mapping, dtype=np.uint8).ctypes.data

    def file_bytes(self) -> np.ndarray:
        """The file's rows region as bytes (a view of the mapping, no copy)."""
        return np.frombuffer(self.mapping, dtype=np.uint8, count=self.rows_bytes)

    def release(self) -> None:
        """Unmap and delete the file (the store maps it by name, so it goes only here)."""
        try:
            self.mapping.close()
        except BufferError:  # a view of it is still held: the mapping goes with the last view
            pass
        self.path.unlink(missing_ok=True)


@dataclass
class StepGather:
    """One step's rows on their way to the host (core/everserve/state/mirror.py:374-387)."""

    n: int
    heads: tuple[HeadSlot, ...]
    stage: Stage
    filled: set[int] = field(default_factory=set)


@dataclass
class StagedJob:
    """A committed step: what the sink receives once its rows are in pinned host memory."""

    epoch: int
    step: int
    counts: dict
    gather: StepGather | None
    gathered: int = 0
    """The fence-less event behind the step's gather (0 for a step with no rows)."""
    descriptor: dict | None = None
    stage_bytes: np.ndarray | None = None
    """The staging file's rows region, valid only while the sink runs."""
    stage_path: Path | None = None
    scales: np.ndarray | None = None
    """The per-layer scales as they stood at the step's gather (a copy), when the stager has
    them."""
    done: threading.Event = field(default_factory=threading.Event)
    error: BaseException | None = None
    times: dict = field(default_factory=dict)


class StepStager:
    """The rank's step path: ``save`` per layer, ``commit`` per step, ``sink`` per staged step.

    ``kv_caches`` maps layer names to the rank's cache tensors; they are ordered by the layer
    index in their names, as the reference's ``register`` orders them (mirror.py:517-520).
    ``heads`` are the held head slots. Staging files are ``<rank_dir>/<stage_prefix><k>.rows``,
    the names the store's open reply gives (mirror.py:461-462,603-604); without ``rank_dir`` the
    stager makes a directory of its own in shared memory and removes it at :meth:`close`.
    ``sink(job)`` runs on the copy thread with ``job.descriptor``, ``job.stage_path`` and
    ``job.stage_bytes`` (the file's rows) valid. When it returns, the file goes back to the pool.
    ``depth`` bounds the steps in flight: a commit with ``depth`` steps outstanding waits for the
    oldest, as the reference's does (mirror.py:664-669). ``scales`` is an optional float32 device
    array with one entry (or row) per layer, snapshotted with every step. ``bounce_bytes`` is the
    size of each of the two pinned buffers the rows pass through, ``copy_threads`` the host
    threads that copy them into the file.
    """

    def __init__(self, ext, kv_caches: Mapping[str, torch.Tensor], heads: Sequence[HeadSlot],
                 sink: Callable[[StagedJob], None], depth: int = 2,
                 stage_prefix: str = "stage", rank_dir: str | os.PathLike | None = None,
                 scales: torch.Tensor | None = None, bounce_bytes: int = 32 << 20,
                 copy_threads: int = 8) -> None:
        if depth < 1:
            raise ValueError(f"depth must be at least 1, got {depth}")
        if bounce_bytes < 64 or bounce_bytes % 64:
            raise ValueError(f"bounce_bytes is a positive multiple of 64, got {bounce_bytes}")
        ordered = sorted((layer_index(n), n, t) for n, t in kv_caches.items())
        self.layers = [(n, t) for _, n, t in ordered]
        self._layer_of = {n: i for i, (n, _) in enumerate(self.layers)}
        self._layer_ptr = [t.data_ptr() for _, t in self.layers]
        first = self.layers[0][1]
        if not first.is_cuda:
            raise ValueError("the step path stages device caches")
        self.paged = PagedKV.of(first)
        self.device = first.device
        self.dtype = first.dtype
        if self.dtype not in DTYPE_NAMES:
            raise ValueError(f"no store dtype name for {self.dtype}")
        self.heads = tuple(sorted(int(h) for h in heads))
        self._ext = ext
        self._kernel = GatherKernel(ext, [t for _, t in self.layers], self.paged)
        self._heads_dev = torch.tensor(self.heads, dtype=torch.long, device=self.device)
        # a step of every layer is one launch whose fixed arguments are checked once, here
        self._launch = None
        if self._kernel.uniform:
            self._launch = ext.bind_gather(self._kernel._ptrs, self._heads_dev,
                                           self.paged.head_dim, self.paged.block_size,
                                           self._kernel._strides[0], self._kernel.elem)
        if scales is not None and (not scales.is_cuda or scales.device != self.device
                                   or scales.dtype != torch.float32
                                   or scales.shape[0] != len(self.layers)):
            raise ValueError("scales: a float32 tensor on the caches' device, one entry per layer")
        self._scales = scales
        self._sink = sink
        self._depth = depth
        self._prefix = stage_prefix
        self._own_dir = rank_dir is None
        if rank_dir is None:
            shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
            rank_dir = tempfile.mkdtemp(prefix="everserve-stage-", dir=shm)
        self.rank_dir = Path(rank_dir)
        if not self.rank_dir.is_dir():
            raise ValueError(f"rank_dir {self.rank_dir} is not a directory")
        self._bounce_bytes = int(bounce_bytes)
        self._bounce = [torch.empty(self._bounce_bytes, dtype=torch.uint8, pin_memory=True)
                        for _ in range(2)]
        for b in self._bounce:  # backed on first touch: touched now, not in the first delivery
            b.zero_()
        self._copy_threads = max(1, int(copy_threads))
        self._stage_seq = 0
        self._pool: list[Stage] = []
        self._pool_lock = threading.Lock()
        self._events: list[int] = []
        self._events_lock = threading.Lock()
        self._step: StepGather | None = None
        self._in_flight: dict[int, StagedJob] = {}
        self._in_flight_lock = threading.Lock()
        self._failed: BaseException | None = None
        self.stats = {"steps": 0, "step_thread_s": 0.0, "backpressure_waits": 0,
                      "backpressure_s": 0.0, "bytes_staged": 0, "bytes_sent": 0, "copy_s": 0.0}
        """``step_thread_s`` is what commits cost the step thread, ``backpressure_s`` included.
        ``bytes_staged`` counts every row copied to the host, padding included; ``bytes_sent``
        only the rows of real slots, as the reference's record does (mirror.py:785-787)."""
        self._copy_stream = torch.cuda.Stream(device=self.device)
        # The first pitched copy to the host in a process sets up the copy engine's queue, about
        # 6 ms on MI355X: one of a few bytes here keeps that out of the first step's delivery.
        probe = torch.empty(64, dtype=torch.uint8, device=self.device)  # its bytes are not read
        with torch.cuda.stream(self._copy_stream):
            ext.copy_rows_async(self._bounce[0].data_ptr(), probe.data_ptr(), 2, 16, 32,
                                self.device)
        self._copy_stream.synchronize()
        del probe
        self._ready = ext.event_create(True)  # the host reads what this one orders
        self._queue: queue.Queue[StagedJob | None] = queue.Queue()
        self._thread = threading.Thread(target=self._copy_loop, daemon=True,
                                        name="everserve-stage-copy")
        self._thread.start()

    def prepare(self, slot_counts: Sequence[int]) -> None:
        """Make the staging files (created, every page faulted in) and device buffers for steps
        of these slot counts now, into the pool, so that the first step of each size does not
        pay for them. On MI355X, C3's 640 MiB file and buffers took 93 ms to prepare; the first
        round after it took 14.4 ms (13.1 steady), where an unprepared first round took 109 ms.
        The pool keeps ``depth + 1`` of them; more are made and dropped again."""
        for n in slot_counts:
            if int(n) < 1:
                raise ValueError(f"a step stages at least one slot, not {n} slots")
            self._release(self._staging(int(n)))

    # ---------------------------------------------------------------- the step thread
    def save(self, layer_name: str, kv_layer: torch.Tensor, slots: torch.Tensor) -> None:
        """Mark this layer's rows at ``slots`` for the step's gather (mirror.py:536-566).

        Reads no device memory on the calling thread. ``slots`` may hold negative padding ids:
        the kernel reads row 0 for them and the store skips them.
        """
        self._check_failed()
        layer = self._layer_of[layer_name]
        if self._layer_ptr[layer] != kv_layer.data_ptr():
            raise ValueError(f"layer {layer_name} is not the cache tensor the stager was given")
        g = self._step
        if g is None:
            g = self._step = self._begin(slots)
        elif g.n != slots.shape[0]:
            raise ValueError(f"one slot mapping per step: layer {layer_name} has "
                             f"{slots.shape[0]} slots, the step has {g.n}")
        g.filled.add(layer)

    def _begin(self, slots: torch.Tensor) -> StepGather:
        n = int(slots.shape[0])
        stage = self._staging(n)
        # the step's own copy of its slot ids, ordered on the producing stream, so a later
        # change to the caller's tensor cannot reach the gather or the descriptor; int64 ids on
        # this device (a serving engine's slot mapping) take one copy call, anything else torch's
        if (slots.device == self.device and slots.dtype == torch.long
                and slots.is_contiguous()):
            self._ext.copy_rows_async(stage.device_slots.data_ptr(), slots.data_ptr(), 1, n * 8,
                                      n * 8, self.device)
        else:
            stage.device_slots[:n].copy_(slots.reshape(-1), non_blocking=True)
        return StepGather(n, self.heads, stage)

    def commit(self, epoch: int, step: int, committed_tokens: Mapping) -> None:
        """Gather the step's marked layers behind the forward and queue the copy; never waits
        for the device (mirror.py:644-680)."""
        self._check_failed()
        t0 = time.perf_counter()
        g, self._step = self._step, None
        job = StagedJob(epoch, step, dict(committed_tokens), g)
        job.times["commit"] = t0
        if g is not None and g.filled:
            cur = torch.cuda.current_stream(self.device)
            if (self._launch is not None and len(g.filled) == len(self.layers)
                    and torch.cuda.current_device() == self._launch.device):
                self._launch(g.stage.device_slots.data_ptr(), g.n, g.stage.device_rows.data_ptr(),
                             g.stage.capacity, cur.cuda_stream)
            else:
                self._kernel.gather(g.stage.device_slots[:g.n], self._heads_dev,
                                    g.stage.device_rows.data_ptr(), g.stage.capacity,
                                    sorted(g.filled))
            self._snapshot_scales(g.stage)
            job.gathered = self._event()
            self._ext.event_record(job.gathered, cur)
        self._enqueue(job, t0)

    def _enqueue(self, job: StagedJob, t0: float) -> None:
        """Hand ``job`` to the copy thread, first waiting for the oldest step when ``depth``
        are in flight."""
        step = job.step
        with self._in_flight_lock:
            # a step whose sink has returned is no longer in flight (a failed one is kept, for
            # fence() to raise; _check_failed raises it at the next call in any case)
            for s in [s for s, j in self._in_flight.items() if j.done.is_set() and j.error is None]:
                del self._in_flight[s]
            oldest = min(self._in_flight) if len(self._in_flight) >= self._depth else None
            waited = oldest is not None and not self._in_flight[oldest].done.is_set()
        if oldest is not None:
            tw = time.perf_counter()
            self.fence(oldest)
            if waited:
                self.stats["backpressure_waits"] += 1
                self.stats["backpressure_s"] += time.perf_counter() - tw
        with self._in_flight_lock:
            self._in_flight[step] = job
        self._queue.put(job)
        self.stats["steps"] += 1
        self.stats["step_thread_s"] += time.perf_counter() - t0

    def commit_blocks(self, epoch: int, step: int, block_ids: Sequence[int],
                      committed_tokens: Mapping | None = None) -> int:
        """Stage every slot of ``block_ids``, every layer and held head, as one step.

        This is a notice round's copy (core/everserve/reference/staging.py:51-94 chooses the
        ids). It is one ``evs_gather_blocks`` launch behind the current stream's work. The
        kernel writes the slot ids ``block * block_size + [0, block_size)`` beside the rows, and
        they become the descriptor's slots. Returns the slots staged.
        """
        self._check_failed()
        if self._step is not None:
            raise ValueError("a step's layers are marked: commit them before a block round")
        ids = [int(b) for b in block_ids]
        bs = self.paged.block_size
        if any(b < 0 or b >= self.paged.num_blocks for b in ids):
            raise ValueError(f"a block id lies outside 0..{self.paged.num_blocks}")
        n = len(ids) * bs
        g = None
        if ids:
            st = self._staging(n)
            st.host_blocks[:len(ids)] = torch.tensor(ids, dtype=torch.int32)
            st.device_blocks[:len(ids)].copy_(st.host_blocks[:len(ids)], non_blocking=True)
            g = StepGather(n, self.heads, st, set(range(len(self.layers))))
        t0 = time.perf_counter()
        job = StagedJob(epoch, step, dict(committed_tokens or {}), g)
        job.times["commit"] = t0
        if g is not None:
            self._kernel.gather_blocks(g.stage.device_blocks[:len(ids)], self._heads_dev,
                                       g.stage.device_rows.data_ptr(), g.stage.capacity,
                                       g.stage.device_slots[:n])
            self._snapshot_scales(g.stage)
            job.gathered = self._event()
            self._ext.event_record(job.gathered, torch.cuda.current_stream(self.device))
        self._enqueue(job, t0)
        return n

    def stage_round(self, window, block_tables: Mapping, num_computed: Mapping, epoch: int,
                    step: int) -> list[int]:
        """Plan a notice round with :func:`everserve_amd.state.notice.blocks_to_stage` and stage
        its blocks; updates ``window``'s counts. Returns the block ids staged."""
        from everserve_amd.state.notice import blocks_to_stage

        ids = blocks_to_stage(block_tables, num_computed, window.staged, self.paged.block_size)
        n = self.commit_blocks(epoch, step, ids, num_computed)
        window.record(len(ids), n * len(self.layers) * len(self.heads) * 2
                      * self.paged.head_dim * self._kernel.elem)
        return ids

    def fence(self, step: int) -> None:
        """Wait until the sink has taken ``step``; raise if staging it failed."""
        with self._in_flight_lock:
            job = self._in_flight.get(step)
        if job is None:
            return
        job.done.wait()
        with self._in_flight_lock:
            self._in_flight.pop(step, None)
        if job.error is not None:
            raise StagingError(f"staging step {step} failed: {job.error}") from job.error

    def flush(self) -> None:
        """Wait for every committed step."""
        with self._in_flight_lock:
            steps = sorted(self._in_flight)
        for s in steps:
            self.fence(s)

    def close(self) -> None:
        """Finish the steps in flight, stop the copy thread and free the staging memory."""
        if self._thread.is_alive():
            self._queue.put(None)
            self._thread.join()
        if self._step is not None:  # layers saved but never committed: their file goes too
            self._step.stage.release()
            self._step = None
        with self._pool_lock:
            pool, self._pool = self._pool, []
        for st in pool:
            st.release()
        if self._own_dir:
            for left in self.rank_dir.glob(f"{self._prefix}*.rows"):
                left.unlink(missing_ok=True)
            try:
                self.rank_dir.rmdir()
            except OSError:
                pass
        with self._events_lock:
            events, self._events = self._events, []
        for e in events + [self._ready]:
            self._ext.event_destroy(e)
        self._ready = 0

    def __enter__(self) -> "StepStager":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def _check_failed(self) -> None:
        if self._failed is not None:
            raise StagingError(f"the copy thread failed: {self._failed}") from self._failed

    # ---------------------------------------------------------------- staging files
    def _snapshot_scales(self, stage: Stage) -> None:
        """The scales as they stand now, behind the gather on the producing stream."""
        if self._scales is not None:
            with torch.inference_mode():
                stage.device_scales.copy_(self._scales.reshape(-1), non_blocking=True)

    def _staging(self, n: int) -> Stage:
        """A staging file with capacity ``max(8, next_pow2(n))``, from the pool when one fits."""
        capacity = capacity_for(n)
        with self._pool_lock:
            for i, st in enumerate(self._pool):
                if st.capacity == capacity and st.num_heads == len(self.heads):
                    return self._pool.pop(i)
        self._stage_seq += 1
        name = f"{self._prefix}{self._stage_seq}.rows"
        shape = (len(self.layers), len(self.heads), capacity, 2, self.paged.head_dim)
        rows_bytes = int(np.prod(shape)) * self._kernel.elem
        n_scales = 0 if self._scales is None else self._scales.numel()
        path = self.rank_dir / name
        mapping = _map_stage_file(path, rows_bytes + 4 * n_scales)
        return Stage(
            name=name,
            path=path,
            capacity=capacity,
            num_heads=len(self.heads),
            rows_bytes=rows_bytes,
            mapping=mapping,
            device_rows=torch.empty(rows_bytes, dtype=torch.uint8, device=self.device),
            device_slots=torch.empty(capacity, dtype=torch.long, device=self.device),
            host_slots=torch.empty(capacity, dtype=torch.long, pin_memory=True),
            device_blocks=torch.empty(capacity, dtype=torch.int32, device=self.device),
            host_blocks=torch.empty(capacity, dtype=torch.int32, pin_memory=True),
            device_scales=(None if not n_scales else
                           torch.empty(n_scales, dtype=torch.float32, device=self.device)),
            host_scales=(None if not n_scales else
                         torch.empty(n_scales, dtype=torch.float32, pin_memory=True)),
        )

    def _release(self, stage: Stage) -> None:
        """Return a file to the pool, keeping at most ``depth + 1``; delete the others
        (mirror.py:636-642)."""
        with self._pool_lock:
            if len(self._pool) <= self._depth:
                self._pool.append(stage)
                return
        stage.release()

    def _event(self) -> int:
        with self._events_lock:
            if self._events:
                return self._events.pop()
        return self._ext.event_create(False)

    def _recycle(self, event: int) -> None:
        with self._events_lock:
            self._events.append(event)

    # ---------------------------------------------------------------- the copy thread
    def _copy_loop(self) -> None:
        while True:
            job = self._queue.get()
            if job is None:
                return
            try:
                self._stage_job(job)
            except Exception as e:  # noqa: BLE001 - surfaced on the step thread
                job.error = e
                if self._failed is None:
                    self._failed = e
            finally:
                job.done.set()

    def _stage_job(self, job: StagedJob) -> None:
        g = job.gather
        if g is None or not g.filled:
            if g is not None:
                self._release(g.stage)
            job.times["ready"] = time.perf_counter()
            self._sink(job)
            return
        try:
            st, n = g.stage, g.n
            row_bytes = 2 * self.paged.head_dim * self._kernel.elem
            heads = len(g.heads)
            pitch = st.capacity * row_bytes
            cs = self._copy_stream
            bounce = [b.data_ptr() for b in self._bounce]
            file_addr, rows_addr = st.file_addr, st.device_rows.data_ptr()
            runs = ([(0, len(self.layers) * heads)] if len(g.filled) == len(self.layers) else
                    [(layer * heads * pitch, heads) for layer in sorted(g.filled)])
            # Everything above is worked out before the wait. The wait ends when the device has
            # finished the step's forward and gather, the moment the step thread wakes to launch
            # the next step: from then on this thread goes straight into the delivery, which runs
            # without the GIL, and does its Python bookkeeping only after it.
            self._ext.event_synchronize(job.gathered)  # a host wait: no device queue waits
            t0 = time.perf_counter()
            for at, count in runs:
                self._ext.deliver_rows(file_addr + at, pitch, rows_addr + at, pitch, count,
                                       n * row_bytes, bounce, self._bounce_bytes, cs,
                                       self._copy_threads)
            job.times["gathered"] = t0
            with torch.cuda.stream(cs):
                self._ext.copy_rows_async(st.host_slots.data_ptr(), st.device_slots.data_ptr(),
                                          1, n * 8, n * 8, self.device)
                if st.device_scales is not None:
                    nb = st.device_scales.numel() * 4
                    self._ext.copy_rows_async(st.host_scales.data_ptr(),
                                              st.device_scales.data_ptr(), 1, nb, nb, self.device)
                self._ext.event_record(self._ready, cs)
            self._ext.event_synchronize(self._ready)
            if st.host_scales is not None:
                scales = st.host_scales.numpy()
                np.frombuffer(st.mapping, dtype=np.float32, count=scales.size,
                              offset=st.rows_bytes)[:] = scales
                job.scales = scales.reshape(self._scales.shape).copy()
            job.times["ready"] = t1 = time.perf_counter()
            self.stats["copy_s"] += t1 - t0
            self.stats["bytes_staged"] += len(g.filled) * heads * n * row_bytes
            slots = st.host_slots[:n].numpy()  # the descriptor copies them out
            self.stats["bytes_sent"] += (int(np.count_nonzero(slots >= 0)) * row_bytes
                                         * len(g.filled) * heads)
            job.descriptor = describe(st.name, sorted(g.filled), g.heads, st.capacity,
                                      self.paged.head_dim, self._kernel.elem, slots,
                                      DTYPE_NAMES[self.dtype])
            job.stage_path = st.path
            job.stage_bytes = st.file_bytes()
            self._sink(job)
            job.times["sent"] = time.perf_counter()
        finally:
            job.stage_bytes = None
            self._recycle(job.gathered)
            self._release(g.stage)
