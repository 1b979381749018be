"""The slot collective on MI355X: the region every member shares, and one member's handle on it.

The same interface as the reference's ``everserve.comm.slotkernel`` (core/everserve/comm/
slotkernel.py:55-120,293-736), over this build's kernel (``evs_slot_all_reduce``):

* :class:`Region` is the shared control and word region of one engine on one node: a header, one
  control row per member (abort word, member order, late mask, bound), one IPC handle per member,
  and the host variant's word rows. Its byte layout is the reference's, word for word, because the
  executor and the watchdog (unchanged) read and write it. It maps a file in shared memory, as the
  reference does, or lives in pinned host memory the library allocates when one process holds
  every row (:meth:`Region.in_pinned_memory`; also where registering existing host memory is not
  allowed).
* :class:`SlotKernel` is one member's handle: its device sequence counters, its member order and
  buffer table in device memory, which the kernel reads on every launch, so a captured HIP graph
  follows a membership change without recapture.

A change has two halves, as in the reference: :meth:`SlotKernel.abort` at any time releases a kernel
waiting on a dead peer; at a step boundary each member calls :meth:`SlotKernel.resume` (counters and
own words zeroed, own abort word cleared) and :meth:`SlotKernel.set_members`.
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
"""Rows in a region: up to seven ranks and the spare."""
MAXN = 64 * 1024
"""Largest tensor the kernel takes, in bf16 elements."""
HOST, P2P = 0, 1
VARIANTS = {"host": HOST, "p2p": P2P}
WORDS_PER_THREAD = {"host": (1, 1), "p2p": (1, 1)}
"""Eight-byte words each thread moves, as (small calls, large calls); small is up to
``SMALL_ELEMENTS``. Measured on MI355X, one word per thread is the fastest or within 3 % of it at
2 Ki, 16 Ki and 64 Ki elements in both variants. Example: host-memory pull of 16 Ki elements over
4 members takes 9.4 us at 1 word and 25.0 us at 16. 16 is the reference's A100 setting for host
memory (core/everserve/comm/slotkernel.py:60)."""
SMALL_ELEMENTS = 4096

# the region's layout (core/everserve/comm/slotkernel.py:71-95): the executor and the watchdog read
# these words, so they stay where the reference puts them
_MAGIC = 0x45565253_4C4F5432  # "EVRSLOT2"
_HEADER_WORDS = 16
_CTRL_WORDS = 16
_HANDLE_BYTES = 64
_PUBLISHED, _ABORT, _COUNT, _ORDER = 0, 1, 2, 3
_LATE, _BOUND, _PID = 11, 12, 13
_HEADER_B = _HEADER_WORDS * 8
_CTRL_B = MAXW * _CTRL_WORDS * 8
_HANDLES_B = MAXW * _HANDLE_BYTES
_WORDS_OFF = 4096
_ROW_WORDS = 2 * (MAXN // 2)  # host rows: two parities of MAXN / 2 words
_ROW_B = _ROW_WORDS * 8
_PUSH_B = MAXW * _ROW_B  # a peer-to-peer buffer: two parities x eight senders x MAXN / 2 words
_SIZE = _WORDS_OFF + MAXW * _ROW_B


def check_layout(ext: Any) -> None:
    """The library's region layout is this module's, or no region is mapped.

    Raises:
        RuntimeError: naming each word that differs.
    """
    ours = {"MAX_ROWS": MAXW, "CTRL_WORDS": _CTRL_WORDS, "ABORT": _ABORT, "LATE": _LATE,
            "BOUND": _BOUND}
    differs = {k: (getattr(ext, k, None), v) for k, v in ours.items() if getattr(ext, k, None) != v}
    if differs:
        raise RuntimeError(f"the slot kernels were built with another region layout than this "
                           f"module's (library, module): {differs}")


class Region:
    """The shared slot region, mapped in this process (numpy views on the host side)."""

    def __init__(self, path: str | None, create: bool = False, variant: str = "host",
                 _memory: tuple[Any, int, int] | None = None) -> None:
        """Map the region at ``path``; with ``create``, size and zero it and record ``variant``.

        Raises:
            ValueError: for an unknown variant, or a file that is not a slot region.
        """
        self.path = path
        self._ext = None
        self._pinned = None
        if _memory is not None:  # pinned host memory, already mapped into the device
            ext, host_ptr, device_ptr = _memory
            self._ext, self._pinned = ext, host_ptr
            self._buf = (ctypes.c_char * _SIZE).from_address(host_ptr)
            self._mm = None
            self.device_addr = device_ptr
            create = True
        else:
            if create:
                with open(path, "wb") as f:
                    f.truncate(_SIZE)
            fd = os.open(path, os.O_RDWR)
            try:
                self._mm = mmap.mmap(fd, _SIZE)
            finally:
                os.close(fd)
            self._buf = (ctypes.c_char * _SIZE).from_buffer(self._mm)
            self.device_addr = 0
        self.addr = ctypes.addressof(self._buf)
        raw = np.frombuffer(self._buf, dtype=np.uint8)
        self.header = raw[:_HEADER_B].view(np.int64)
        self.ctrl = raw[_HEADER_B:_HEADER_B + _CTRL_B].view(np.int64).reshape(MAXW, _CTRL_WORDS)
        self.handles = raw[_HEADER_B + _CTRL_B:_HEADER_B + _CTRL_B + _HANDLES_B].reshape(
            MAXW, _HANDLE_BYTES)
        self.words = raw[_WORDS_OFF:].view(np.int64).reshape(MAXW, _ROW_WORDS)
        if create:
            if variant not in VARIANTS:
                raise ValueError(f"unknown slot variant {variant!r}")
            raw[:] = 0
            self.header[1], self.header[2], self.header[3] = VARIANTS[variant], MAXW, MAXN
            self.header[0] = _MAGIC
        elif int(self.header[0]) != _MAGIC:
            raise ValueError(f"{path} is not a slot region")

    @classmethod
    def in_pinned_memory(cls, ext: Any, variant: str = "host") -> Region:
        """A region in pinned, coherent host memory mapped into the current device, for one
        process holding every row."""
        host, dev = ext.host_alloc_mapped(_SIZE)
        return cls(None, variant=variant, _memory=(ext, host, dev))

    @property
    def variant(self) -> str:
        return "p2p" if int(self.header[1]) == P2P else "host"

    # ------------------------------------------------------------------ the control path
    def set_members(self, rows: Iterable[int], order: Sequence[int]) -> None:
        """Every row in ``rows`` sums over the rows in ``order``, in that order, from its next call.

        Raises:
            ValueError: for a row out of range or listed twice.
        """
        order = [int(m) for m in order]
        if len(set(order)) != len(order) or not all(0 <= m < MAXW for m in order):
            raise ValueError(f"a slot member order needs distinct rows below {MAXW}: {order}")
        for r in rows:
            self.ctrl[r, _ORDER:_ORDER + MAXW] = 0
            self.ctrl[r, _ORDER:_ORDER + len(order)] = order
            self.ctrl[r, _COUNT] = len(order)

    def order(self, row: int) -> list[int]:
        n = int(self.ctrl[row, _COUNT])
        return [int(m) for m in self.ctrl[row, _ORDER:_ORDER + n]]

    def set_abort(self, rows: Iterable[int], value: int = 1) -> None:
        for r in rows:
            self.ctrl[r, _ABORT] = value

    def set_bound(self, rows: Iterable[int], bound_s: float) -> None:
        """A kernel of every row in ``rows`` names a member it waits for longer than ``bound_s``."""
        for r in rows:
            self.ctrl[r, _BOUND] = int(bound_s * 1e9)

    def bound(self, row: int) -> float:
        return int(self.ctrl[row, _BOUND]) / 1e9

    def late(self, row: int) -> set[int]:
        """The rows ``row``'s kernel has waited for past its bound and still waits for."""
        v = int(self.ctrl[row, _LATE])
        return {r for r in range(MAXW) if v >> r & 1}

    def set_pid(self, row: int, pid: int) -> None:
        self.ctrl[row, _PID] = pid

    def pid(self, row: int) -> int:
        return int(self.ctrl[row, _PID])

    # ------------------------------------------------------------------ a member's side
    def map_device(self, ext: Any) -> int:
        """The region's address in the current device's address space, mapping it if needed."""
        if not self.device_addr:
            self.device_addr = ext.host_register_mapped(self.addr, _SIZE)
            self._ext = ext
        return self.device_addr

    def ctrl_device(self) -> int:
        return self.device_addr + _HEADER_B

    def row_device(self, row: int) -> int:
        return self.device_addr + _WORDS_OFF + row * _ROW_B

    def publish(self, row: int, handle: bytes) -> None:
        self.handles[row, :len(handle)] = np.frombuffer(handle, np.uint8)
        self.ctrl[row, _PUBLISHED] = 1  # after the handle: x86 keeps the stores in order

    def handle(self, row: int, timeout_s: float) -> bytes:
        deadline = time.monotonic() + timeout_s
        while not int(self.ctrl[row, _PUBLISHED]):
            if time.monotonic() >= deadline:
                raise TimeoutError(f"slot row {row} did not publish its buffer in {timeout_s}s")
            time.sleep(0.01)
        return bytes(self.handles[row])

    def close(self) -> None:
        self.header = self.ctrl = self.handles = self.words = None
        if self._pinned is not None:
            self._buf = None
            self._ext.host_free(self._pinned)
            self._pinned = None
            return
        if self.device_addr and self._ext is not None:
            self._ext.host_unregister(self.addr)
            self.device_addr = 0
        self._buf = None
        self._mm.close()


class SlotKernel:
    """One member's handle on the slot collective (the ``SlotCollective`` interface)."""

    def __init__(self, region: Region, row: int, device: int, open_timeout_s: float = 300.0,
                 ext: Any = None) -> None:
        if ext is None:
            from everserve_amd import kernels

            ext = kernels.load()
        self.region = region
        self.row = row
        self.device = torch.device("cuda", device)
        self._ext = ext
        check_layout(ext)
        self._timeout = open_timeout_s
        with torch.cuda.device(self.device):
            region.map_device(ext)
            self._words = WORDS_PER_THREAD[region.variant]
            blocks = ext.slot_blocks(MAXN, 1)  # counters for any words-per-thread setting
            self.seq = torch.zeros(blocks + 1, dtype=torch.int64, device=self.device)
            self._table = torch.zeros(MAXW, dtype=torch.int64, device=self.device)
            self._order = torch.zeros(1 + MAXW, dtype=torch.int32, device=self.device)
        self._members = region.order(row)
        region.set_pid(row, os.getpid())
        self._addrs = [0] * MAXW
        self._opened: dict[int, int] = {}
        self._own = 0
        if region.variant == "p2p":
            with torch.cuda.device(self.device):
                self._own = ext.device_alloc(_PUSH_B)
            region.publish(row, ext.ipc_handle(self._own))
            self._addrs[row] = self._own
        else:
            self._addrs = [region.row_device(r) for r in range(MAXW)]
        self._write_table()
        self._write_order()

    @property
    def variant(self) -> str:
        return self.region.variant

    def _write_table(self) -> None:
        with torch.inference_mode():
            self._table.copy_(torch.tensor(self._addrs, dtype=torch.int64))

    def _write_order(self) -> None:
        rows = [len(self._members), *self._members]
        rows += [0] * (1 + MAXW - len(rows))
        with torch.inference_mode():
            self._order.copy_(torch.tensor(rows, dtype=torch.int32))

    def _open(self, rows: Iterable[int]) -> None:
        """Map every member's buffer this process does not have yet (peer-to-peer variant)."""
        if self.variant != "p2p":
            return
        changed = False
        for r in rows:
            if r == self.row or r in self._opened:
                continue
            with torch.cuda.device(self.device):
                self._opened[r] = self._ext.ipc_open(self.region.handle(r, self._timeout))
            self._addrs[r] = self._opened[r]
            changed = True
        if changed:
            self._write_table()

    def can_take(self, t: torch.Tensor) -> bool:
        """Decode sizes: contiguous bf16 on this device, an even count of at most ``MAXN``."""
        return (t.dtype == torch.bfloat16 and t.is_contiguous() and t.device == self.device
                and t.numel() <= MAXN and t.numel() % 2 == 0)

    def all_reduce_into(self, inp: torch.Tensor, out: torch.Tensor) -> None:
        """Sum ``inp`` over the members into ``out``; capturable in a HIP graph (not the first
        call of a peer-to-peer member, which maps the peers' buffers)."""
        if self.variant == "p2p" and len(self._opened) + 1 < len(self._members):
            self._open(self._members)
        words = self._words[0] if inp.numel() <= SMALL_ELEMENTS else self._words[1]
        self._ext.slot_all_reduce(inp, out, self._table, self.region.ctrl_device(), self._order,
                                  self.seq, self.row, MAXN, words, self.variant == "p2p")

    def set_members(self, members: Iterable[int], epoch: int) -> None:
        """Take up this process's order for its row; called at a boundary, member quiescent."""
        del epoch  # the epoch fences the runtime; the kernel needs only the order
        members = [int(m) for m in members]
        self.region.set_members([self.row], members)
        self._open(members)
        self._members = members
        self._write_order()

    def abort(self) -> None:
        """Release this process from a kernel waiting on a dead peer. Safe at any time."""
        self.region.set_abort([self.row], 1)

    def resume(self) -> None:
        """Zero this process's counters and its own words once its stream is idle, then clear its
        own abort word."""
        with torch.cuda.device(self.device):
            torch.cuda.synchronize(self.device)
            with torch.inference_mode():
                self.seq.zero_()
            own_bytes = _PUSH_B if self.variant == "p2p" else _ROW_B
            self._ext.memset_async(self._addrs[self.row], own_bytes)
            torch.cuda.synchronize(self.device)
        self.region.set_abort([self.row], 0)

    def close(self) -> None:
        for p in self._opened.values():
            self._ext.ipc_close(p)
        self._opened.clear()
        if self._own:
            self._ext.device_free(self._own)
            self._own = 0
