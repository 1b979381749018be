"""The slot collective's shared region and one member's handle on it, over ``evs_slot_all_reduce``.

Every process of one engine on a node shares one small region. It is a binary format: the
executor writes member orders and bounds into it, each member's kernel reads its control row and
writes its late mask there, and the watchdog reads that mask. Its words therefore sit exactly where
the reference's region puts them (core/everserve/comm/slotkernel.py:71-95): a 16-word header, one
16-word control row per member from byte 128, one 64-byte IPC handle per member after those, and
from byte 4096 the host variant's word rows, two parities of ``MAXN / 2`` eight-byte words each.

This module describes that format once, as numpy record types (:data:`HEADER`, :data:`CONTROL`,
:data:`REGION`). Everything else is read off them: the word numbers the library is checked
against (:func:`check_layout`), the device addresses the kernel is given, the views the control
path writes through. A region lives in a file in shared memory, as on a serving node, or in
pinned host memory the library maps into the device (:meth:`Region.in_pinned_memory`), for one
process holding every row or a host that does not allow registering existing memory.

:class:`SlotKernel` is one member's handle. Its buffer table (every member's word buffer) and its
member order share one small device array, rewritten with one copy at a membership change, and
its per-workgroup sequence counters are another. The kernel reads all three on every launch, so a
captured HIP graph follows a change without being captured again.
"""

from __future__ import annotations

import ctypes
import mmap
import os
import time
from collections.abc import Iterable, Sequence
from typing import Any

import numpy as np
import torch

MAXW = 8
"""Member rows in a region: up to seven ranks and the spare."""
MAXN = 64 * 1024
"""Largest tensor the kernel takes, in bf16 elements."""
VARIANTS = {"host": 0, "p2p": 1}
"""``host``: members' words in the region's host rows; ``p2p``: each member's words in its own
device buffer, which the others map through an IPC handle and push into."""
WORDS_PER_THREAD = {"host": (1, 1), "p2p": (1, 1)}
"""Eight-byte words a thread moves, for (calls up to ``SMALL_ELEMENTS``, larger calls). On
MI355X one word per thread is the fastest, or within 3 % of it, at 2 Ki, 16 Ki and 64 Ki elements
in both variants (host-memory pull of 16 Ki over 4 members: 9.4 us at 1 word, 25.0 us at 16)."""
SMALL_ELEMENTS = 4096

MAGIC = 0x45565253_4C4F5432
"""The header's first word ("EVRSLOT2", a region with member orders)."""
HANDLE_BYTES = 64

HEADER = np.dtype([("magic", "<i8"), ("variant", "<i8"), ("rows", "<i8"), ("maxn", "<i8"),
                   ("node", "<i8", (12,))])
"""The header: what the region is, then words the node's executor keeps."""

CONTROL = np.dtype([
    ("published", "<i8"),    # the row's IPC handle is readable
    ("abort", "<i8"),        # nonzero: the row's kernel stops waiting
    ("count", "<i8"),        # members in the order
    ("order", "<i8", (MAXW,)),  # rows summed, in this order
    ("late", "<i8"),         # mask of rows the row's kernel waits for past its bound
    ("bound", "<i8"),        # ns a kernel waits before it names a row late (0: never)
    ("pid", "<i8"),          # the process holding the row
    ("lost", "<i8"),         # the row's watchdog's findings
    ("step", "<i8"),         # the row's step count
])
"""One member's control row."""

WORDS_AT = 4096
ROW_WORDS = MAXN
"""Words of one host row: two parities of ``MAXN / 2``."""
PUSH_BYTES = MAXW * ROW_WORDS * 8
"""A peer-to-peer member's buffer: two parities x eight senders x ``MAXN / 2`` words."""

REGION = np.dtype({
    "names": ["header", "control", "handles", "words"],
    "formats": [HEADER, (CONTROL, (MAXW,)), ("u1", (MAXW, HANDLE_BYTES)),
                ("<i8", (MAXW, ROW_WORDS))],
    "offsets": [0, HEADER.itemsize, HEADER.itemsize + MAXW * CONTROL.itemsize, WORDS_AT],
    "itemsize": WORDS_AT + MAXW * ROW_WORDS * 8,
})
"""The whole region."""

SIZE = REGION.itemsize


def _word(field: str) -> int:
    return CONTROL.fields[field][1] // 8


def layout_words() -> dict[str, int]:
    """The format's numbers the library is built with (its ``evs_layout_constants``)."""
    return {"MAX_ROWS": MAXW, "CTRL_WORDS": CONTROL.itemsize // 8, "ABORT": _word("abort"),
            "LATE": _word("late"), "BOUND": _word("bound")}


def check_layout(ext: Any) -> None:
    """Refuse a library built for another region format: it would read and write other words.

    Raises:
        RuntimeError: naming each number that differs, as (library, this module).
    """
    differs = {name: (getattr(ext, name, None), ours) for name, ours in layout_words().items()
               if getattr(ext, name, None) != ours}
    if differs:
        raise RuntimeError(f"the slot kernels were built with another region layout than this "
                           f"module's (library, module): {differs}")


class _File:
    """A region file in shared memory, mapped in this process."""

    def __init__(self, path: str, create: bool) -> None:
        flags = os.O_RDWR | (os.O_CREAT if create else 0)
        fd = os.open(path, flags, 0o660)
        try:
            if create:
                os.fchmod(fd, 0o660)  # the node's group maps it, whatever this umask
                os.ftruncate(fd, SIZE)
            self.map = mmap.mmap(fd, SIZE)
        finally:
            os.close(fd)
        self.buffer = (ctypes.c_char * SIZE).from_buffer(self.map)
        self.device_addr = 0

    def release(self, ext: Any) -> None:
        if self.device_addr and ext is not None:
            ext.host_unregister(ctypes.addressof(self.buffer))
        self.device_addr = 0
        self.buffer = None
        self.map.close()


class _Pinned:
    """A region in pinned, coherent host memory the library allocated and mapped into the device."""

    def __init__(self, ext: Any) -> None:
        self.ext = ext
        self.host_addr, self.device_addr = ext.host_alloc_mapped(SIZE)
        self.buffer = (ctypes.c_char * SIZE).from_address(self.host_addr)

    def release(self, ext: Any) -> None:
        self.buffer = None
        ext.host_free(self.host_addr)
        self.device_addr = 0


class Region:
    """The shared slot region, as this process maps it.

    ``control`` is the control rows as a record array (``control["abort"][r]``) and ``head`` the
    header as a one-record array. ``header``, ``ctrl`` (``[MAXW, 16]``), ``handles`` and ``words``
    (``[MAXW, ROW_WORDS]``) are plain integer views of the same bytes, for code that reads words by
    number.
    """

    def __init__(self, path: str | None, create: bool = False, variant: str = "host",
                 _backing: Any = None) -> None:
        """Map the region file at ``path``; with ``create``, make it, zero it and record
        ``variant``.

        Raises:
            ValueError: for an unknown variant, or a file that is not a slot region.
        """
        if create and variant not in VARIANTS:
            raise ValueError(f"unknown slot variant {variant!r}")
        self.path = path
        self._ext = None
        self._backing = _backing if _backing is not None else _File(path, create)
        if _backing is not None:
            self._ext = _backing.ext
            create = True
        raw = np.frombuffer(self._backing.buffer, dtype=np.uint8)
        whole = raw.view(REGION)
        self.head = whole["header"]
        self.control = whole["control"][0]
        self.handles = whole["handles"][0]
        self.words = whole["words"][0]
        self.header = raw[:HEADER.itemsize].view(np.int64)
        at = REGION.fields["control"][1]
        self.ctrl = raw[at:at + MAXW * CONTROL.itemsize].view(np.int64).reshape(MAXW, -1)
        self.addr = ctypes.addressof(self._backing.buffer)
        if create:
            raw[:] = 0
            for name, value in (("variant", VARIANTS[variant]), ("rows", MAXW), ("maxn", MAXN),
                                ("magic", MAGIC)):  # the magic last: whoever sees it sees the rest
                self.head[name] = value
        elif int(self.head["magic"][0]) != MAGIC:
            raise ValueError(f"{path} is not a slot region")

    @classmethod
    def in_pinned_memory(cls, ext: Any, variant: str = "host") -> Region:
        """A region in pinned host memory mapped into the current device, for one process that
        holds every row (no other process can map it)."""
        if variant not in VARIANTS:
            raise ValueError(f"unknown slot variant {variant!r}")
        return cls(None, variant=variant, _backing=_Pinned(ext))

    @property
    def variant(self) -> str:
        kind = int(self.head["variant"][0])
        return next(name for name, v in VARIANTS.items() if v == kind)

    def _get(self, field: str, row: int):
        if not 0 <= row < MAXW:
            raise ValueError(f"slot rows are 0..{MAXW - 1}, got {row}")
        return self.control[field][row]

    def _put(self, field: str, row: int, value) -> None:
        if not 0 <= row < MAXW:
            raise ValueError(f"slot rows are 0..{MAXW - 1}, got {row}")
        self.control[field][row] = value

    # ------------------------------------------------------------------ the control path
    def set_members(self, rows: Iterable[int], order: Sequence[int]) -> None:
        """From their next call, the kernels of ``rows`` sum over the rows of ``order``, in that
        order (the members' rank positions, a spare in the place of the rank it replaced).

        Raises:
            ValueError: for a row out of range or listed twice.
        """
        members = [int(m) for m in order]
        if len(set(members)) != len(members) or any(not 0 <= m < MAXW for m in members):
            raise ValueError(f"a slot member order needs distinct rows below {MAXW}: {members}")
        padded = members + [0] * (MAXW - len(members))
        for r in rows:
            self._put("order", r, padded)
            self._put("count", r, len(members))

    def order(self, row: int) -> list[int]:
        """The rows ``row``'s kernel sums, in its order."""
        return [int(m) for m in self._get("order", row)[:int(self._get("count", row))]]

    def set_abort(self, rows: Iterable[int], value: int = 1) -> None:
        """Set (or, with 0, clear) the abort word of each row."""
        for r in rows:
            self._put("abort", r, value)

    def set_bound(self, rows: Iterable[int], bound_s: float) -> None:
        """The kernels of ``rows`` name a member they wait for longer than ``bound_s`` seconds."""
        for r in rows:
            self._put("bound", r, round(bound_s * 1e9))

    def bound(self, row: int) -> float:
        """``row``'s bound in seconds (0: its kernel names nobody)."""
        return int(self._get("bound", row)) / 1e9

    def late(self, row: int) -> set[int]:
        """The rows ``row``'s kernel still waits for past its bound."""
        mask = int(self._get("late", row))
        return {r for r in range(MAXW) if mask & (1 << r)}

    def set_pid(self, row: int, pid: int) -> None:
        self._put("pid", row, pid)

    def pid(self, row: int) -> int:
        return int(self._get("pid", row))

    # ------------------------------------------------------------------ the members' side
    def map_device(self, ext: Any) -> int:
        """The region's address in the current device, registering a file mapping if needed."""
        if not self._backing.device_addr:
            self._backing.device_addr = ext.host_register_mapped(self.addr, SIZE)
            self._ext = ext
        return self._backing.device_addr

    @property
    def device_addr(self) -> int:
        return self._backing.device_addr

    def ctrl_device(self) -> int:
        """Device address of the control rows, which the kernel indexes by row."""
        return self.device_addr + REGION.fields["control"][1]

    def row_device(self, row: int) -> int:
        """Device address of ``row``'s host word row."""
        return self.device_addr + WORDS_AT + row * ROW_WORDS * 8

    def publish(self, row: int, handle: bytes) -> None:
        """Make ``row``'s buffer handle readable by the other members."""
        self.handles[row, :len(handle)] = np.frombuffer(handle, dtype=np.uint8)
        self._put("published", row, 1)  # x86 keeps this store after the handle's

    def handle(self, row: int, timeout_s: float) -> bytes:
        """``row``'s buffer handle, once published.

        Raises:
            TimeoutError: if ``row`` publishes nothing within ``timeout_s`` seconds.
        """
        give_up = time.monotonic() + timeout_s
        while not int(self._get("published", row)):
            if time.monotonic() > give_up:
                raise TimeoutError(f"slot row {row} did not publish its buffer in {timeout_s}s")
            time.sleep(0.01)
        return bytes(self.handles[row])

    def close(self) -> None:
        """Drop this process's mapping; a region file stays until it is removed."""
        self.head = self.control = self.header = self.ctrl = self.handles = self.words = None
        self._backing.release(self._ext)


class SlotKernel:
    """One member's handle on the slot collective: ``row`` of ``region`` on GPU ``device``."""

    # the device plan: the buffer table (MAXW int64), then the order as int32 [count, rows...]
    _PLAN_WORDS = MAXW + (1 + MAXW + 1) // 2

    def __init__(self, region: Region, row: int, device: int, open_timeout_s: float = 300.0,
                 ext: Any = None) -> None:
        if ext is None:
            from everserve_amd import kernels

            ext = kernels.load()
        check_layout(ext)
        self.region, self.row, self._ext = region, row, ext
        self.device = torch.device("cuda", device)
        self._open_timeout = open_timeout_s
        self._words = WORDS_PER_THREAD[region.variant]
        self._push = region.variant == "p2p"
        self._peers: dict[int, int] = {}  # rows mapped from their IPC handles
        self._own = 0
        with torch.cuda.device(self.device):
            region.map_device(ext)
            # one counter per workgroup the kernel can launch at one word per thread, plus the
            # counter the last waiting workgroup uses to clear the late mask
            self.seq = torch.zeros(ext.slot_blocks(MAXN, 1) + 1, dtype=torch.int64,
                                   device=self.device)
            self._plan = torch.zeros(self._PLAN_WORDS, dtype=torch.int64, device=self.device)
            if self._push:
                self._own = ext.device_alloc(PUSH_BYTES)
                region.publish(row, ext.ipc_handle(self._own))
        self._table = self._plan[:MAXW]
        self._order = self._plan[MAXW:].view(torch.int32)[:1 + MAXW]
        if self._push:
            self._buffers = [0] * MAXW
            self._buffers[row] = self._own
        else:
            self._buffers = [region.row_device(r) for r in range(MAXW)]
        region.set_pid(row, os.getpid())
        self._members = region.order(row)
        self._write_plan()

    @property
    def variant(self) -> str:
        return self.region.variant

    def _write_plan(self) -> None:
        """The buffer table and the order, to the device in one copy."""
        host = np.zeros(self._PLAN_WORDS, dtype=np.int64)
        host[:MAXW] = self._buffers
        order = host[MAXW:].view(np.int32)
        order[0] = len(self._members)
        order[1:1 + len(self._members)] = self._members
        with torch.inference_mode():
            self._plan.copy_(torch.from_numpy(host))

    def _map_peers(self, rows: Iterable[int]) -> None:
        """Map the buffer of every peer in ``rows`` not mapped yet (peer-to-peer variant)."""
        if not self._push:
            return
        fresh = [r for r in rows if r != self.row and r not in self._peers]
        with torch.cuda.device(self.device):
            for r in fresh:
                self._peers[r] = self._buffers[r] = self._ext.ipc_open(
                    self.region.handle(r, self._open_timeout))
        if fresh:
            self._write_plan()

    def can_take(self, t: torch.Tensor) -> bool:
        """Whether ``t`` fits the kernel: contiguous bf16 on this device, an even element count of
        at most ``MAXN``."""
        return (t.dtype == torch.bfloat16 and t.device == self.device and t.is_contiguous()
                and t.numel() % 2 == 0 and t.numel() <= MAXN)

    def all_reduce_into(self, inp: torch.Tensor, out: torch.Tensor) -> None:
        """``out`` = the members' ``inp`` summed in order. Capturable in a HIP graph, except for a
        peer-to-peer member's first call, which maps the peers' buffers."""
        if self._push and any(m != self.row and m not in self._peers for m in self._members):
            self._map_peers(self._members)
        words = self._words[inp.numel() > SMALL_ELEMENTS]
        self._ext.slot_all_reduce(inp, out, self._table, self.region.ctrl_device(), self._order,
                                  self.seq, self.row, MAXN, words, self._push)

    def set_members(self, members: Iterable[int], epoch: int) -> None:
        """Take ``members`` as this row's order, at a step boundary with this member quiescent.
        ``epoch`` orders the change for the runtime; the kernel needs only the order."""
        del epoch
        members = [int(m) for m in members]
        self.region.set_members([self.row], members)
        self._map_peers(members)
        self._members = members
        self._write_plan()

    def abort(self) -> None:
        """Release this member's kernel from a wait on a dead peer; safe at any time."""
        self.region.set_abort([self.row], 1)

    def resume(self) -> None:
        """Start over after a change: once this member's work is done, zero its counters and its
        own words, then clear its abort word. A word left from before could otherwise carry a
        sequence number a new call expects."""
        own = self._own if self._push else self._buffers[self.row]
        with torch.cuda.device(self.device):
            torch.cuda.synchronize(self.device)
            with torch.inference_mode():
                self.seq.zero_()
            self._ext.memset_async(own, PUSH_BYTES if self._push else ROW_WORDS * 8)
            torch.cuda.synchronize(self.device)
        self.region.set_abort([self.row], 0)

    def close(self) -> None:
        """Unmap the peers' buffers and free this member's own."""
        for ptr in self._peers.values():
            self._ext.ipc_close(ptr)
        self._peers.clear()
        if self._own:
            self._ext.device_free(self._own)
            self._own = 0
