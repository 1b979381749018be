"""The MI355X kernels: load the C-ABI library, say whether it is usable here, and expose it under
the names and argument meanings of the reference's extension module ``everserve_kernels``.

The library is ``libeverserve_mi355x.so``, built in tree by ``python -m everserve_amd.build``
(hipcc for gfx950; no torch headers). Its C entry points are declared in
``include/everserve_mi355x.h``. This module is the loader the reference's
``core/everserve/kernels.py`` is, with the same contract (core/everserve/kernels.py:1-27,
125-221):

* a build is loaded only when its stamp (the sources by content, and the GPU architectures) is
  this tree's and names this GPU: anything else raises :class:`KernelsUnavailable`, never a
  silent fallback;
* ``EVERSERVE_KERNELS_DIR`` names a build made elsewhere, loaded on the same terms;
* ``EVERSERVE_KERNELS=torch`` is the only way to run without the kernels, and :func:`available`
  then says False;
* the architecture is the device's ``gcnArchName`` (``gfx950``), not a CUDA compute capability.

:func:`load` returns a :class:`Kernels` object whose methods take the reference module's
arguments (torch tensors for the device index arrays, integers for raw addresses) and enqueue on
torch's current stream of the tensors' device, as the reference's ``gather_rows`` does
(core/csrc/gather.cu:100-135).
"""

from __future__ import annotations

import ctypes
import functools
import json
import logging
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Sequence

log = logging.getLogger(__name__)

NAME = "everserve_kernels"
LIBRARY = "libeverserve_mi355x.so"
PREBUILT_ENV = "EVERSERVE_KERNELS_DIR"
"""A directory holding a build made ahead of time, loaded when its stamp is this tree's."""
PATHS_ENV = "EVERSERVE_KERNELS"
"""``torch`` to run on the torch paths without the kernels, by choice; anything else loads them."""
STAMP = "stamp.json"
HANDLE_BYTES = 64

_PACKAGE = Path(__file__).resolve().parent

EVS_OK = 0
REDUCE_STATE_WORDS = 288
"""64-bit words of local_reduce's state record (EVS_REDUCE_STATE_WORDS in the C header)."""
ORDER_MIN_SLOTS = 1 << 18
ORDER_MIN_BYTES = 8 << 30
"""The sizes from which :meth:`Kernels.scatter_rows` sorts its pairs by slot first. Measured on
MI355X (Llama-3-8B rows, bf16, 16-slot blocks of a permuted table, median of 10 launches), sorted
against staged order, the sort's 0.11 ms included: every slot of a 262,144-slot cache, 32 layers,
11.58 against 12.17 ms; 8 layers 2.86 against 3.02; 4 layers 1.52 against 1.53; 1 layer 0.47
against 0.38 (the sort not repaid); a quarter of the cache's blocks, 32 layers, 3.12 against 3.08
(writes spread over a sparse part of a cache gain nothing from order). The call cannot see the
cache's size unless told it (``num_slots``), so a call of this many slots into a cache several
times larger sorts too, and can lose up to about 3 %: pass ``num_slots`` or ``ordered=False``
there."""


def sort_first(n: int, layers: int, heads: int, d: int, elem: int, capturing: bool,
               num_slots: int | None = None) -> bool:
    """Whether :meth:`Kernels.scatter_rows` left to choose sorts its ``n`` pairs by slot first:
    from :data:`ORDER_MIN_SLOTS` slots and :data:`ORDER_MIN_BYTES` of rows, fewer than 2^31
    pairs (the sort's limit), not while the stream is being captured, and, when the caller
    names the cache's slot count, only when the call writes at least seven eighths of the
    cache. Sorted against staged time, C4's 32 layers of a 262,144-slot cache, a random part of
    its blocks, two seeds: all of them 0.953-0.955, seven eighths 0.981-0.984, three quarters
    0.9995-1.006, five eighths 1.004-1.011, half 1.023-1.029."""
    if num_slots is not None and 8 * n < 7 * num_slots:
        return False
    return (not capturing and ORDER_MIN_SLOTS <= n < (1 << 31)
            and layers * heads * n * 2 * d * elem >= ORDER_MIN_BYTES)


class BoundGather:
    """``evs_gather_rows`` for fixed layers, heads and layout (:meth:`Kernels.bind_gather`)."""

    def __init__(self, kernels: "Kernels", lp: int, num_layers: int, hp: int, num_heads: int,
                 d: int, block_size: int, strides: list[int], elem_size: int, device: int,
                 keep: tuple) -> None:
        self._kernels = kernels
        self._fn = kernels._lib.evs_gather_rows
        self._args = (lp, num_layers, hp, num_heads, d, block_size)
        self._strides = (ctypes.c_int64 * 5)(*strides)
        self._elem = elem_size
        self.device = device
        self._keep = keep  # the tensors whose addresses the launcher holds

    def __call__(self, slots_ptr: int, n: int, out_ptr: int, capacity: int, stream: int) -> None:
        """Enqueue the gather of rows ``[0, n)`` at ``slots_ptr`` (int64 device slot ids) into
        ``[L, H, capacity, 2, d]`` at ``out_ptr`` on ``stream`` (a raw stream handle of the
        bound device, which must be the current device)."""
        lp, num_layers, hp, num_heads, d, bs = self._args
        rc = self._fn(lp, num_layers, slots_ptr, n, hp, num_heads, out_ptr, capacity, d, bs,
                      self._strides, self._elem, stream)
        if rc != EVS_OK:
            self._kernels._check(rc)


@dataclass(frozen=True)
class CommitPlan:
    """``evs_store_commit``'s per-table arguments for one set of store tables, built once."""

    T: int
    offsets: object  # int64 numpy array [T]
    tables: object  # ctypes void* arrays [T]
    steps: object
    crcs: object
    num_slots: int
    row_bytes: int
    keep: tuple  # the arrays the pointers name, kept alive


class KernelsUnavailable(RuntimeError):
    """The kernels cannot be loaded here, and why: a wrong or stale build, no GPU."""


class KernelError(RuntimeError):
    """A kernel entry point refused its arguments or the HIP runtime failed; the library's message."""


def stamp() -> dict[str, str]:
    """What this tree's sources are, by content (the build records the same digest)."""
    from everserve_amd import build

    return {"sources": build.sources_digest()}


def built_archs(archs: str) -> set[str]:
    """The GPU architectures a build names (``"gfx942;gfx950"``: both)."""
    return {a.strip().split(":")[0] for a in archs.replace(" ", ";").split(";") if a.strip()}


def device_arch() -> str | None:
    """This process's GPU architecture (``"gfx950"``), or None without a GPU."""
    import torch

    if not torch.cuda.is_available():
        return None
    return torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName.split(":")[0]


def _check_stamp(directory: Path) -> Path:
    """The library in ``directory`` when its stamp is this tree's and names this GPU.

    Raises:
        KernelsUnavailable: no usable stamp, another tree's sources, another GPU, no library.
    """
    try:
        theirs = json.loads((directory / STAMP).read_text())
    except (OSError, ValueError) as e:
        raise KernelsUnavailable(f"{directory}: no usable stamp ({e})") from e
    ours = stamp()
    if any(theirs.get(k) != v for k, v in ours.items()):
        raise KernelsUnavailable(
            f"{directory}: built against {theirs}, this tree is {ours}; "
            "rebuild with python -m everserve_amd.build"
        )
    here = device_arch()
    if here is not None and here not in built_archs(theirs.get("archs", "")):
        raise KernelsUnavailable(
            f"{directory}: built for {theirs.get('archs')}, this GPU is {here}"
        )
    so = directory / LIBRARY
    if not so.is_file():
        raise KernelsUnavailable(f"{directory}: stamped, but no {LIBRARY} in it")
    return so


def _prebuilt() -> Path | None:
    """The library of the build ``EVERSERVE_KERNELS_DIR`` names; None when it names none.

    Raises:
        KernelsUnavailable: see :func:`_check_stamp`.
    """
    directory = os.environ.get(PREBUILT_ENV, "")
    if not directory:
        return None
    return _check_stamp(Path(directory))


def library_path() -> Path:
    """The library this process loads: the named prebuilt, else the in-tree build.

    The in-tree build is made here when there is none yet; an existing one whose stamp is not
    this tree's is refused, not rebuilt around.
    """
    named = _prebuilt()
    if named is not None:
        return named
    if not (_PACKAGE / LIBRARY).is_file():
        from everserve_amd import build

        log.info("no in-tree build of %s: building it now", LIBRARY)
        build.build(_PACKAGE)
    return _check_stamp(_PACKAGE)


# (name, restype, argtypes) of every entry point in include/everserve_mi355x.h
_I64, _P, _I32 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
_SIGNATURES: tuple[tuple[str, object, tuple], ...] = (
    ("evs_last_error", ctypes.c_char_p, ()),
    ("evs_layout_constants", _I32, (_P, _I64)),
    ("evs_gather_rows", _I32, (_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P)),
    (
        "evs_gather_blocks",
        _I32,
        (_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P),
    ),
    ("evs_scatter_rows", _I32, (_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P)),
    ("evs_scatter_pairs", _I32,
     (_P, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P)),
    ("evs_scatter_ranges", _I32,
     (_P, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P)),
    ("evs_order_pairs_workspace", _I32, (_I64, _I32, _P)),
    ("evs_order_pairs", _I32, (_P, _I64, _I32, _P, _P, _P, _I64, _P)),
    ("evs_order_pairs_static", _I32, (_P, _I64, _I32, _P, _P, _P)),
    ("evs_local_reduce", _I32, (_P, _P, _P, _P, _I64, ctypes.c_uint64, _I64, _P, _P, _P)),
    ("evs_slot_all_reduce", _I32,
     (_P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _I64, _P)),
    ("evs_slot_blocks", _I32, (_I64, _I64, _P)),
    ("evs_host_register_mapped", _I32, (_P, _I64, _P)),
    ("evs_host_unregister", _I32, (_P,)),
    ("evs_host_alloc_mapped", _I32, (_I64, _P, _P)),
    ("evs_host_free", _I32, (_P,)),
    ("evs_device_alloc", _I32, (_I64, _P)),
    ("evs_device_free", _I32, (_P,)),
    ("evs_memset_async", _I32, (_P, _I64, _P)),
    ("evs_copy_rows_async", _I32, (_P, _P, _I64, _I64, _I64, _P)),
    ("evs_host_gather_ranges", _I32, (_P, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _P)),
    ("evs_host_gather_tables", _I32, (_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _P)),
    ("evs_deliver_rows", _I32, (_P, _I64, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P)),
    ("evs_store_commit", _I32,
     (_P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _P, _I64, ctypes.c_uint64, _I64, _P)),
    ("evs_crc32c", _I32, (_P, _I64, _P)),
    ("evs_crc32c_rows", _I32, (_P, _I64, _I64, _P)),
    ("evs_event_create", _I32, (_I32, _P)),
    ("evs_event_destroy", _I32, (_P,)),
    ("evs_event_record", _I32, (_P, _P)),
    ("evs_event_synchronize", _I32, (_P,)),
    ("evs_stream_handoff", _I32, (_P, _P, _P)),
    ("evs_ipc_handle", _I32, (_P, _P, _I64)),
    ("evs_ipc_open", _I32, (_P, _I64, _P)),
    ("evs_ipc_close", _I32, (_P,)),
    ("evs_wall_clock_khz", _I32, (_P,)),
)
ENTRY_POINTS = tuple(name for name, _, _ in _SIGNATURES)


def open_library(path: Path | None = None) -> ctypes.CDLL:
    """dlopen the library and declare every entry point's C signature. Needs no GPU.

    torch is imported first so the library binds to the HIP runtime torch already loaded: one
    runtime per process, so torch's stream handles are valid here.
    """
    import torch  # noqa: F401  (loads torch's HIP runtime before the library resolves it)

    lib = ctypes.CDLL(str(path or library_path()))
    for name, restype, argtypes in _SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = list(argtypes)
    return lib


def _stream_of(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def _device_ptr(t, what: str, dtype) -> int:
    """A device tensor's address, after checking it is on the GPU and of ``dtype``."""
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be on the device")
    if t.dtype != dtype:
        raise RuntimeError(f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"{what} must be contiguous")
    return t.data_ptr()


def _one_device(what: str, *tensors) -> None:
    """The tensors a launch reads must all be on one GPU: the kernel runs there."""
    devices = {t.device for t in tensors if t is not None}
    if len(devices) > 1:
        raise RuntimeError(f"{what}: tensors on several devices ({sorted(map(str, devices))})")


class Kernels:
    """The loaded library under the reference module's names (core/csrc/kernels.cpp:9-31).

    Attributes MAX_ROWS, CTRL_WORDS, ABORT, LATE and BOUND are the slot region's layout as the
    library was built with it; ``core/everserve/comm/slotkernel.py:98-120`` compares its copy.
    """

    def __init__(self, lib: ctypes.CDLL, path: Path) -> None:
        self._lib = lib
        self.__file__ = str(path)
        words = (ctypes.c_int64 * 5)()
        self._check(lib.evs_layout_constants(words, 5))
        self.MAX_ROWS, self.CTRL_WORDS, self.ABORT, self.LATE, self.BOUND = (int(w) for w in words)
        self._workspace: dict = {}  # order_pairs' workspace, per (device, stream)
        self._pairs: dict = {}  # scatter_rows' sorted pairs, per (device, stream)

    def _check(self, rc: int) -> None:
        if rc != EVS_OK:
            raise KernelError(self._lib.evs_last_error().decode(errors="replace"))

    # -------------------------------------------------------------- the step's KV rows
    def gather_rows(
        self,
        layer_ptrs,
        slots,
        heads,
        out_ptr: int,
        capacity: int,
        d: int,
        block_size: int,
        strides: Sequence[int],
        elem_size: int,
    ) -> None:
        """Copy a step's rows of every layer and held head into a [L, H, cap, 2, d] buffer.

        Same arguments as the reference's ``gather_rows`` (core/csrc/gather.cu:100-135); enqueued
        on the current stream of ``slots``'s device, without synchronising.
        """
        import torch

        if len(strides) != 5:
            raise RuntimeError("gather_rows: a layout is five strides")
        lp = _device_ptr(layer_ptrs, "gather_rows: layer_ptrs", torch.long)
        sp = _device_ptr(slots, "gather_rows: slots", torch.long)
        hp = _device_ptr(heads, "gather_rows: heads", torch.long)
        _one_device("gather_rows", layer_ptrs, slots, heads)
        st = (ctypes.c_int64 * 5)(*[int(s) for s in strides])
        with torch.cuda.device(slots.device):
            self._check(
                self._lib.evs_gather_rows(
                    lp, layer_ptrs.numel(), sp, slots.numel(), hp, heads.numel(), int(out_ptr),
                    int(capacity), int(d), int(block_size), st, int(elem_size),
                    _stream_of(slots.device),
                )
            )

    def bind_gather(self, layer_ptrs, heads, d: int, block_size: int, strides: Sequence[int],
                    elem_size: int) -> "BoundGather":
        """:meth:`gather_rows` with the arguments that stay the same from step to step (the
        layers, the held heads, the layout) checked and converted once; the returned launcher
        takes a step's slot ids, row count, output and stream. For a step path that launches
        every step, where the checks and conversions cost more host time than the launch."""
        import torch

        if len(strides) != 5:
            raise RuntimeError("gather_rows: a layout is five strides")
        lp = _device_ptr(layer_ptrs, "gather_rows: layer_ptrs", torch.long)
        hp = _device_ptr(heads, "gather_rows: heads", torch.long)
        _one_device("gather_rows", layer_ptrs, heads)
        return BoundGather(self, lp, layer_ptrs.numel(), hp, heads.numel(), int(d),
                           int(block_size), [int(s) for s in strides], int(elem_size),
                           layer_ptrs.device.index, (layer_ptrs, heads))

    def gather_blocks(
        self,
        layer_ptrs,
        block_ids,
        heads,
        out_ptr: int,
        capacity: int,
        d: int,
        block_size: int,
        strides: Sequence[int],
        elem_size: int,
        slots_out=None,
    ) -> None:
        """:meth:`gather_rows` over whole blocks of a block table (int32 ``block_ids``).

        With ``slots_out`` (int64, ``len(block_ids) * block_size``) the kernel also writes the
        expanded slot ids, the step descriptor's tags.
        """
        import torch

        if len(strides) != 5:
            raise RuntimeError("gather_blocks: a layout is five strides")
        lp = _device_ptr(layer_ptrs, "gather_blocks: layer_ptrs", torch.long)
        bp = _device_ptr(block_ids, "gather_blocks: block_ids", torch.int32)
        hp = _device_ptr(heads, "gather_blocks: heads", torch.long)
        so = 0
        if slots_out is not None:
            so = _device_ptr(slots_out, "gather_blocks: slots_out", torch.long)
            if slots_out.numel() < block_ids.numel() * block_size:
                raise RuntimeError("gather_blocks: slots_out holds fewer than blocks * block_size")
        _one_device("gather_blocks", layer_ptrs, block_ids, heads, slots_out)
        st = (ctypes.c_int64 * 5)(*[int(s) for s in strides])
        with torch.cuda.device(block_ids.device):
            self._check(
                self._lib.evs_gather_blocks(
                    lp, layer_ptrs.numel(), bp, block_ids.numel(), hp, heads.numel(),
                    int(out_ptr), int(capacity), int(d), int(block_size), st, int(elem_size),
                    so or None, _stream_of(block_ids.device),
                )
            )

    def scatter_rows(
        self,
        layer_ptrs,
        slots,
        heads,
        in_ptr: int,
        capacity: int,
        d: int,
        block_size: int,
        strides: Sequence[int],
        elem_size: int,
        ordered: bool | None = None,
        num_slots: int | None = None,
    ) -> None:
        """Write [L, H, cap, 2, d] rows back into the caches at ``slots`` and head slots ``heads``.

        The inverse of :meth:`gather_rows`; negative slots are padding and are skipped. Replaces
        the restore's ``PagedKV.write_rows`` (core/everserve/state/kvcopy.py:118-128).

        ``ordered``: write in slot order, the (slot, row) pairs sorted on the device first
        (:meth:`order_pairs`, then :meth:`scatter_pairs`, in the workspace this object keeps per
        device and stream), or in staged order (``evs_scatter_rows``, one kernel). The same bytes
        land either way. ``None`` sorts from :data:`ORDER_MIN_SLOTS` slots and
        :data:`ORDER_MIN_BYTES` of rows, where writing a whole cache through a permuted block
        table in slot order repays the sort, and never under graph capture (the sort clears its
        counters with a memset, which a captured graph must not hold). ``num_slots``, the
        caches' slot count when the caller knows it, lets that choice see how much of the cache
        the call writes (:func:`sort_first`).
        """
        import torch

        if len(strides) != 5:
            raise RuntimeError("scatter_rows: a layout is five strides")
        lp = _device_ptr(layer_ptrs, "scatter_rows: layer_ptrs", torch.long)
        sp = _device_ptr(slots, "scatter_rows: slots", torch.long)
        hp = _device_ptr(heads, "scatter_rows: heads", torch.long)
        _one_device("scatter_rows", layer_ptrs, slots, heads)
        st = (ctypes.c_int64 * 5)(*[int(s) for s in strides])
        n, nl, nh = slots.numel(), layer_ptrs.numel(), heads.numel()
        with torch.cuda.device(slots.device):
            capturing = torch.cuda.is_current_stream_capturing()
            if ordered is None:
                ordered = sort_first(n, nl, nh, int(d), int(elem_size), capturing, num_slots)
            if ordered and capturing:
                raise RuntimeError("scatter_rows: an ordered scatter cannot be captured in a graph "
                                   "(its sort clears counters with a memset)")
            if not ordered:
                self._check(
                    self._lib.evs_scatter_rows(
                        lp, nl, sp, n, hp, nh, int(in_ptr), int(capacity), int(d),
                        int(block_size), st, int(elem_size), _stream_of(slots.device),
                    )
                )
                return
            # the staged-order call's checks first (no layer: nothing is launched), so that the
            # ordered call refuses what the staged one refuses
            self._check(
                self._lib.evs_scatter_rows(lp, 0, sp, n, hp, nh, int(in_ptr), int(capacity),
                                           int(d), int(block_size), st, int(elem_size),
                                           _stream_of(slots.device))
            )
            if n == 0 or nl == 0 or nh == 0:
                return
            key = (slots.device, _stream_of(slots.device))
            pairs = self._pairs.get(key)
            if pairs is None or pairs[0].numel() < n:
                pairs = self._pairs[key] = (torch.empty(n, dtype=torch.long, device=slots.device),
                                            torch.empty(n, dtype=torch.long, device=slots.device))
            o_slots, o_rows = self.order_pairs(slots, 1 << 32, out=(pairs[0][:n], pairs[1][:n]))
        self.scatter_pairs(layer_ptrs, o_slots, o_rows, heads, in_ptr, capacity, d, block_size,
                           strides, elem_size)

    def scatter_pairs(
        self,
        layer_ptrs,
        slots,
        rows_of,
        heads,
        in_ptr: int,
        capacity: int,
        d: int,
        block_size: int,
        strides: Sequence[int],
        elem_size: int,
    ) -> None:
        """Write staged row ``rows_of[i]`` of [L, H, cap, 2, d] into the caches at ``slots[i]``.

        :meth:`scatter_rows` with the staged row of each slot named, so the caller chooses the
        order of the writes: slots listed in increasing order write each cache front to back.
        A negative slot, or a row outside ``[0, capacity)``, moves nothing.
        """
        import torch

        if len(strides) != 5:
            raise RuntimeError("scatter_pairs: a layout is five strides")
        if rows_of.numel() != slots.numel():
            raise RuntimeError(f"scatter_pairs: {slots.numel()} slots but {rows_of.numel()} rows")
        lp = _device_ptr(layer_ptrs, "scatter_pairs: layer_ptrs", torch.long)
        sp = _device_ptr(slots, "scatter_pairs: slots", torch.long)
        rp = _device_ptr(rows_of, "scatter_pairs: rows_of", torch.long)
        hp = _device_ptr(heads, "scatter_pairs: heads", torch.long)
        _one_device("scatter_pairs", layer_ptrs, slots, rows_of, heads)
        st = (ctypes.c_int64 * 5)(*[int(s) for s in strides])
        with torch.cuda.device(slots.device):
            self._check(
                self._lib.evs_scatter_pairs(
                    lp, layer_ptrs.numel(), sp, rp, slots.numel(), hp, heads.numel(), int(in_ptr),
                    int(capacity), int(d), int(block_size), st, int(elem_size),
                    _stream_of(slots.device),
                )
            )

    def scatter_ranges(
        self,
        layer_ptrs,
        starts,
        first_rows,
        num_rows: int,
        heads,
        in_ptr: int,
        capacity: int,
        d: int,
        block_size: int,
        strides: Sequence[int],
        elem_size: int,
    ) -> None:
        """Write staged rows [L, H, cap, 2, d] into the caches at the slots of written ranges:
        row t goes to ``starts[k] + t - first_rows[k]`` for the range k holding it.

        ``starts`` (R) and ``first_rows`` (R + 1: 0 first, ascending, ``num_rows`` last) are int64
        device tensors. :meth:`scatter_rows` with the slots given as (start, count) ranges;
        replaces the restore's ``PagedKV.write_rows`` of a table's written ranges
        (core/everserve/state/mirror.py:926-937).
        """
        import torch

        if len(strides) != 5:
            raise RuntimeError("scatter_ranges: a layout is five strides")
        if first_rows.numel() != starts.numel() + 1:
            raise RuntimeError(f"scatter_ranges: {starts.numel()} ranges need "
                               f"{starts.numel() + 1} first rows, got {first_rows.numel()}")
        lp = _device_ptr(layer_ptrs, "scatter_ranges: layer_ptrs", torch.long)
        sp = _device_ptr(starts, "scatter_ranges: starts", torch.long)
        fp = _device_ptr(first_rows, "scatter_ranges: first_rows", torch.long)
        hp = _device_ptr(heads, "scatter_ranges: heads", torch.long)
        _one_device("scatter_ranges", layer_ptrs, starts, first_rows, heads)
        st = (ctypes.c_int64 * 5)(*[int(s) for s in strides])
        with torch.cuda.device(starts.device):
            self._check(
                self._lib.evs_scatter_ranges(
                    lp, layer_ptrs.numel(), sp, fp, starts.numel(), int(num_rows), hp,
                    heads.numel(), int(in_ptr), int(capacity), int(d), int(block_size), st,
                    int(elem_size), _stream_of(starts.device),
                )
            )

    def order_pairs(self, slots, num_slots: int, out=None):
        """``(slots_sorted, rows_of)`` for :meth:`scatter_pairs`, ordered on the device.

        ``slots`` (int64, on the device) are the cache slots of staged rows 0..n-1 and
        ``num_slots`` the cache's slot count, which fixes the key bits compared. The result is
        ``slots`` by increasing slot and the staged row of each (stable). A padding slot
        (negative) is kept and lands anywhere; the pair scatter skips it. Enqueued on the current
        stream of the slots' device.

        ``out`` is an optional pair of int64 device tensors of ``slots``'s size to write into;
        without it they are allocated. The sort's workspace is kept by this object, per device and
        stream (so calls on different streams never share one), and grows only when a call needs
        more: repeated calls with ``out`` allocate nothing.
        """
        import torch

        sp = _device_ptr(slots, "order_pairs: slots", torch.long)
        n = slots.numel()
        bits = max(1, (int(num_slots) - 1).bit_length())
        if out is None:
            out = (torch.empty_like(slots), torch.empty_like(slots))
        out_slots, out_rows = out
        for t, what in ((out_slots, "slots_out"), (out_rows, "rows_out")):
            _device_ptr(t, f"order_pairs: {what}", torch.long)
            if t.numel() != n:
                raise RuntimeError(f"order_pairs: {what} holds {t.numel()} entries, not {n}")
        _one_device("order_pairs", slots, out_slots, out_rows)
        need = ctypes.c_int64()
        with torch.cuda.device(slots.device):
            self._check(self._lib.evs_order_pairs_workspace(n, bits, ctypes.byref(need)))
            key = (slots.device, _stream_of(slots.device))
            work = self._workspace.get(key)
            if work is None or work.numel() < need.value:
                work = torch.empty(max(1, need.value), dtype=torch.uint8, device=slots.device)
                self._workspace[key] = work
            self._check(
                self._lib.evs_order_pairs(sp, n, bits, out_slots.data_ptr(), out_rows.data_ptr(),
                                          work.data_ptr(), work.numel(),
                                          _stream_of(slots.device))
            )
        return out_slots, out_rows

    def copy_rows_async(self, dst_ptr: int, src_ptr: int, groups: int, bytes_: int, pitch: int,
                        device=None) -> None:
        """Copy ``groups`` runs of ``bytes_`` bytes spaced ``pitch`` apart on both sides, on the
        current stream (device to host into pinned memory, or host to device)."""
        import torch

        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._check(
            self._lib.evs_copy_rows_async(int(dst_ptr), int(src_ptr), int(groups), int(bytes_),
                                          int(pitch), _stream_of(dev))
        )

    def host_gather_ranges(self, src_ptr: int, src_rows: int, row_bytes: int, starts, counts,
                           dst_ptr: int, dst_rows: int, max_threads: int = 16) -> int:
        """Copy the rows of slot ranges of a host table (``src_rows`` rows) into ``dst_ptr``
        (room for ``dst_rows``) on host threads; returns the rows copied.

        ``starts`` and ``counts`` are int64 numpy arrays. A range outside the table, or more rows
        than ``dst`` holds, is refused before anything is copied.
        """
        import numpy as np

        st = np.ascontiguousarray(starts, dtype=np.int64)
        ct = np.ascontiguousarray(counts, dtype=np.int64)
        if st.shape != ct.shape:
            raise RuntimeError("host_gather_ranges: starts and counts differ in length")
        rows = ctypes.c_int64()
        self._check(
            self._lib.evs_host_gather_ranges(int(src_ptr), int(src_rows), int(row_bytes),
                                             st.ctypes.data, ct.ctypes.data, st.size,
                                             int(dst_ptr), int(dst_rows), int(max_threads),
                                             ctypes.byref(rows))
        )
        return rows.value

    def host_gather_tables(self, src_ptrs: Sequence[int], src_rows: int, row_bytes: int, starts,
                           counts, dst_ptr: int, dst_rows: int, max_threads: int = 16) -> int:
        """:meth:`host_gather_ranges` over several tables with the same ranges, in one call:
        table j's rows land at ``dst_ptr + j * dst_rows * row_bytes``. Returns the rows copied per
        table."""
        import numpy as np

        st = np.ascontiguousarray(starts, dtype=np.int64)
        ct = np.ascontiguousarray(counts, dtype=np.int64)
        if st.shape != ct.shape:
            raise RuntimeError("host_gather_tables: starts and counts differ in length")
        srcs = (ctypes.c_void_p * max(1, len(src_ptrs)))(*[int(p) for p in src_ptrs])
        rows = ctypes.c_int64()
        self._check(
            self._lib.evs_host_gather_tables(srcs, len(src_ptrs), int(src_rows), int(row_bytes),
                                             st.ctypes.data, ct.ctypes.data, st.size,
                                             int(dst_ptr), int(dst_rows), int(max_threads),
                                             ctypes.byref(rows))
        )
        return rows.value

    def deliver_rows(self, dst_ptr: int, dst_pitch: int, src_ptr: int, src_pitch: int, runs: int,
                     run_bytes: int, bounce: Sequence[int], bounce_bytes: int, stream,
                     max_threads: int = 16) -> None:
        """Copy ``runs`` runs of device rows into host memory that need not be pinned (a staging
        file), through the two pinned ``bounce`` buffers; blocks until the rows are there.
        ``stream`` is a torch stream the copies are issued on."""
        if len(bounce) != 2:
            raise RuntimeError("deliver_rows: two bounce buffers")
        self._check(
            self._lib.evs_deliver_rows(int(dst_ptr), int(dst_pitch), int(src_ptr), int(src_pitch),
                                       int(runs), int(run_bytes), int(bounce[0]), int(bounce[1]),
                                       int(bounce_bytes), int(max_threads),
                                       int(stream.cuda_stream))
        )

    # -------------------------------------------------------------- the store's commit copy
    def store_commit_plan(self, stage_offsets, tables, written_step, crc, num_slots: int,
                          row_bytes: int) -> "CommitPlan":
        """Check one set of store tables and build ``evs_store_commit``'s arrays for them once,
        for :meth:`store_commit_with` to commit step after step.

        ``stage_offsets`` is int64 [T], where each table's rows start in a stage; ``tables``,
        ``written_step`` and ``crc`` are sequences of T numpy arrays: [num_slots * row_bytes]
        uint8, [num_slots] uint64, [num_slots] uint32. The plan keeps them alive.
        """
        import numpy as np

        T = len(tables)
        if not (len(written_step) == len(crc) == len(stage_offsets) == T):
            raise RuntimeError("store_commit: one offset, table, step array and crc array each")
        for k in range(T):
            if (tables[k].dtype != np.uint8 or tables[k].size != num_slots * row_bytes
                    or written_step[k].dtype != np.uint64 or written_step[k].size != num_slots
                    or crc[k].dtype != np.uint32 or crc[k].size != num_slots
                    or not (tables[k].flags.c_contiguous and written_step[k].flags.c_contiguous
                            and crc[k].flags.c_contiguous)):
                raise RuntimeError(f"store_commit: table {k}'s arrays do not match "
                                   f"{num_slots} slots of {row_bytes} bytes")
        return CommitPlan(
            T, np.ascontiguousarray(stage_offsets, dtype=np.int64),
            (ctypes.c_void_p * max(T, 1))(*[t.ctypes.data for t in tables]),
            (ctypes.c_void_p * max(T, 1))(*[w.ctypes.data for w in written_step]),
            (ctypes.c_void_p * max(T, 1))(*[c.ctypes.data for c in crc]),
            int(num_slots), int(row_bytes), (list(tables), list(written_step), list(crc)))

    def store_commit_with(self, plan: "CommitPlan", stage, slots, step: int,
                          max_threads: int = 16) -> int:
        """Commit one staged step's rows into a plan's tables on host threads; the new slot
        count. ``stage`` is a contiguous uint8 numpy array (the staged bytes), ``slots`` the
        step's slot ids (negative: padding). store/src/storage.rs:864-957."""
        import numpy as np

        if stage.dtype != np.uint8 or not stage.flags.c_contiguous:
            raise RuntimeError("store_commit: the stage is contiguous uint8")
        sl = np.ascontiguousarray(slots, dtype=np.int64)
        fresh = ctypes.c_int64()
        self._check(self._lib.evs_store_commit(
            stage.ctypes.data, stage.size, plan.offsets.ctypes.data, plan.T, plan.tables,
            plan.steps, plan.crcs, plan.num_slots, plan.row_bytes, sl.ctypes.data, sl.size,
            int(step) & (2**64 - 1), int(max_threads), ctypes.byref(fresh)))
        return fresh.value

    def store_commit(self, stage, stage_offsets, tables, written_step, crc, num_slots: int,
                     row_bytes: int, slots, step: int, max_threads: int = 16) -> int:
        """Commit one staged step's rows into store tables on host threads; the new slot count.

        :meth:`store_commit_plan` and :meth:`store_commit_with` in one call (arguments as
        there). store/src/storage.rs:864-957.
        """
        plan = self.store_commit_plan(stage_offsets, tables, written_step, crc, num_slots,
                                      row_bytes)
        return self.store_commit_with(plan, stage, slots, step, max_threads)

    def crc32c(self, data) -> int:
        """CRC32C (Castagnoli) of a bytes-like object or a contiguous numpy array."""
        import numpy as np

        a = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else data
        a = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        out = ctypes.c_uint32()
        self._check(self._lib.evs_crc32c(a.ctypes.data if a.size else None, a.size,
                                         ctypes.byref(out)))
        return out.value

    def crc32c_rows(self, rows, row_bytes: int):
        """CRC32C of each of the consecutive rows of ``rows`` (a contiguous numpy array)."""
        import numpy as np

        a = np.ascontiguousarray(rows).view(np.uint8).reshape(-1)
        if a.size % row_bytes:
            raise RuntimeError("crc32c_rows: not a whole number of rows")
        out = np.empty(a.size // row_bytes, dtype=np.uint32)
        self._check(self._lib.evs_crc32c_rows(a.ctypes.data, int(row_bytes), out.size,
                                              out.ctypes.data))
        return out

    # -------------------------------------------------------------- the reduction stage
    def local_reduce(self, bufs, flags, order, out, epoch: int, timeout_ns: int, ctrl_ptr: int,
                     state) -> None:
        """Sum the members' bf16 buffers in ``order`` into ``out`` once their flags carry ``epoch``.

        ``bufs`` int64 [MAX_ROWS] addresses, ``flags`` 64-bit [MAX_ROWS] (a tensor, or the
        device address of host-mapped words), ``order`` int32
        [1 + MAX_ROWS] = [count, rows...], ``state`` 64-bit [REDUCE_STATE_WORDS] (zeroed once):
        all on the device.
        ``ctrl_ptr`` is the device address of this member's control row (0: none). The wait ends
        at the ABORT word or after ``timeout_ns``; the outcome is in ``state[0]``.
        """
        import torch

        if out.dtype != torch.bfloat16 or not out.is_cuda or not out.is_contiguous():
            raise RuntimeError("local_reduce: out must be a contiguous bf16 device tensor")
        bp = _device_ptr(bufs, "local_reduce: bufs", torch.long)
        if isinstance(flags, int):
            fp = flags  # a device address, e.g. host-mapped words a host thread writes
        else:
            if flags.element_size() != 8 or not flags.is_cuda or flags.numel() < self.MAX_ROWS:
                raise RuntimeError("local_reduce: flags are MAX_ROWS 64-bit words on the device")
            fp = flags.data_ptr()
        op = _device_ptr(order, "local_reduce: order", torch.int32)
        if order.numel() != 1 + self.MAX_ROWS or bufs.numel() < self.MAX_ROWS:
            raise RuntimeError("local_reduce: order is int32 [1 + MAX_ROWS], bufs [MAX_ROWS]")
        if (state.element_size() != 8 or state.numel() < REDUCE_STATE_WORDS or not state.is_cuda
                or not state.is_contiguous()):
            raise RuntimeError(f"local_reduce: state is {REDUCE_STATE_WORDS} contiguous 64-bit "
                               f"words on the device")
        _one_device("local_reduce", bufs, None if isinstance(flags, int) else flags, order, out,
                    state)
        with torch.cuda.device(out.device):
            self._check(
                self._lib.evs_local_reduce(
                    bp, fp, op, out.data_ptr(), out.numel(),
                    int(epoch) & 0xFFFFFFFFFFFFFFFF, int(timeout_ns), int(ctrl_ptr) or None,
                    state.data_ptr(), _stream_of(out.device),
                )
            )

    slot_timeout_ns = 30 * 10**9
    """How long a slot_all_reduce waits for a member before it stops by itself, ABORT aside."""

    def slot_all_reduce(self, inp, out, bufs, ctrl_ptr: int, order, seqs, row: int, maxn: int,
                        words: int, push: bool) -> None:
        """The slot collective: sum bf16 ``inp`` over the row's members, graph-capturable.

        The reference's arguments (core/csrc/slot.cu:234-281): ``bufs`` int64 [MAX_ROWS] device
        table of word buffers, ``ctrl_ptr`` the device address of the region's control rows,
        ``order`` int32 [1 + MAX_ROWS], ``seqs`` int64 counters, ``row`` this member's row.
        """
        import torch

        if inp.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
            raise RuntimeError("slot_all_reduce: bf16 only")
        if not (inp.is_cuda and out.is_cuda and bufs.is_cuda and seqs.is_cuda and order.is_cuda):
            raise RuntimeError("slot_all_reduce: tensors must be on the device")
        if not (inp.is_contiguous() and out.is_contiguous()):
            raise RuntimeError("slot_all_reduce: contiguous only")
        if out.numel() != inp.numel():
            raise RuntimeError("slot_all_reduce: out and inp differ in size")
        if order.dtype != torch.int32 or order.numel() != 1 + self.MAX_ROWS:
            raise RuntimeError(f"slot_all_reduce: the order is int32 [count, rows...] of "
                               f"{1 + self.MAX_ROWS}")
        bp = _device_ptr(bufs, "slot_all_reduce: bufs", torch.long)
        op = _device_ptr(order, "slot_all_reduce: order", torch.int32)
        if seqs.dtype != torch.long or not seqs.is_contiguous():
            raise RuntimeError("slot_all_reduce: seqs are contiguous int64")
        _one_device("slot_all_reduce", inp, out, bufs, order, seqs)
        with torch.cuda.device(inp.device):
            self._check(
                self._lib.evs_slot_all_reduce(
                    inp.data_ptr(), out.data_ptr(), inp.numel(), bp, int(ctrl_ptr),
                    op, seqs.data_ptr(), seqs.numel(), int(row), int(maxn),
                    int(words), 1 if push else 0, int(self.slot_timeout_ns),
                    _stream_of(inp.device),
                )
            )

    def slot_blocks(self, maxn: int, words: int) -> int:
        """Sequence counters for tensors up to ``maxn`` at ``words`` per thread (slot.cu:229-232)."""
        out = ctypes.c_int64()
        self._check(self._lib.evs_slot_blocks(int(maxn), int(words), ctypes.byref(out)))
        return out.value

    # -------------------------------------------------------------- memory
    def host_register_mapped(self, ptr: int, bytes_: int) -> int:
        """Pin host memory mapped into the device address space; returns the device pointer."""
        dev = ctypes.c_void_p()
        self._check(self._lib.evs_host_register_mapped(int(ptr), int(bytes_), ctypes.byref(dev)))
        return int(dev.value or 0)

    def host_unregister(self, ptr: int) -> None:
        """Undo :meth:`host_register_mapped`."""
        self._check(self._lib.evs_host_unregister(int(ptr)))

    def host_alloc_mapped(self, bytes_: int) -> tuple[int, int]:
        """Pinned coherent host memory mapped into the device: (host pointer, device pointer)."""
        host, dev = ctypes.c_void_p(), ctypes.c_void_p()
        self._check(
            self._lib.evs_host_alloc_mapped(int(bytes_), ctypes.byref(host), ctypes.byref(dev))
        )
        return int(host.value or 0), int(dev.value or 0)

    def host_free(self, ptr: int) -> None:
        self._check(self._lib.evs_host_free(int(ptr)))

    def device_alloc(self, bytes_: int) -> int:
        """Device memory outside torch's caching allocator, zeroed."""
        p = ctypes.c_void_p()
        self._check(self._lib.evs_device_alloc(int(bytes_), ctypes.byref(p)))
        return int(p.value or 0)

    def device_free(self, ptr: int) -> None:
        self._check(self._lib.evs_device_free(int(ptr)))

    def memset_async(self, ptr: int, bytes_: int) -> None:
        """Zero device memory on the current stream (a fill kernel, safe inside graph capture)."""
        import torch

        dev = torch.device("cuda", torch.cuda.current_device())
        self._check(self._lib.evs_memset_async(int(ptr), int(bytes_), _stream_of(dev)))

    # -------------------------------------------------------------- stream ordering
    def event_create(self, system_fence: bool = False) -> int:
        """A HIP event with timing off; without the system-scope fence unless asked for."""
        ev = ctypes.c_void_p()
        self._check(self._lib.evs_event_create(1 if system_fence else 0, ctypes.byref(ev)))
        return int(ev.value or 0)

    def event_destroy(self, event: int) -> None:
        self._check(self._lib.evs_event_destroy(int(event)))

    def event_record(self, event: int, stream) -> None:
        self._check(self._lib.evs_event_record(int(event), int(stream.cuda_stream)))

    def event_synchronize(self, event: int) -> None:
        self._check(self._lib.evs_event_synchronize(int(event)))

    def stream_handoff(self, producing, waiting, event: int) -> None:
        """``waiting`` runs its later work after everything ``producing`` enqueued so far."""
        self._check(self._lib.evs_stream_handoff(int(producing.cuda_stream),
                                                 int(waiting.cuda_stream), int(event)))

    def ipc_handle(self, ptr: int) -> bytes:
        """An inter-process handle for a :meth:`device_alloc` buffer (64 bytes)."""
        buf = (ctypes.c_uint8 * HANDLE_BYTES)()
        self._check(self._lib.evs_ipc_handle(int(ptr), buf, HANDLE_BYTES))
        return bytes(buf)

    def ipc_open(self, handle: bytes) -> int:
        """Map another process's buffer from its handle."""
        if len(handle) != HANDLE_BYTES:
            raise RuntimeError("ipc_open: not an IPC handle")
        buf = (ctypes.c_uint8 * HANDLE_BYTES).from_buffer_copy(handle)
        p = ctypes.c_void_p()
        self._check(self._lib.evs_ipc_open(buf, HANDLE_BYTES, ctypes.byref(p)))
        return int(p.value or 0)

    def ipc_close(self, ptr: int) -> None:
        self._check(self._lib.evs_ipc_close(int(ptr)))

    def wall_clock_khz(self) -> int:
        """The current device's wall-clock rate, in kHz."""
        khz = ctypes.c_int64()
        self._check(self._lib.evs_wall_clock_khz(ctypes.byref(khz)))
        return khz.value


_SOURCE: str = ""
"""Where this process's library came from once :func:`load` has run: ``prebuilt`` (the directory
``EVERSERVE_KERNELS_DIR`` names) or ``in-tree``."""


@functools.lru_cache(maxsize=1)
def load() -> Kernels:
    """This process's :class:`Kernels`, opened once and kept (the library lives in the process's
    one HIP runtime, as torch does).

    Raises:
        KernelsUnavailable: on a host without a GPU, or for a library whose stamp is not this
            tree's, names another GPU, or fails to open.
    """
    global _SOURCE
    import torch

    if not torch.cuda.is_available():
        raise KernelsUnavailable("no GPU in this process: the MI355X kernels cannot run")
    path = library_path()
    try:
        lib = open_library(path)
    except OSError as e:
        raise KernelsUnavailable(f"{path} did not open: {e}") from e
    kernels = Kernels(lib, path)
    _SOURCE = "prebuilt" if os.environ.get(PREBUILT_ENV) else "in-tree"
    return kernels


def source() -> str:
    """``prebuilt`` or ``in-tree`` once :func:`load` has run; empty before."""
    return _SOURCE


@functools.lru_cache(maxsize=1)
def available() -> bool:
    """True when this process moves KV and reduces on the kernels.

    Three answers, and no fourth:

    * ``EVERSERVE_KERNELS=torch`` was set: False, and nothing is loaded. Only an operator's
      choice makes a rank leave the kernels, so that every rank of an engine runs the same code;
    * the process has no GPU: False;
    * otherwise the library is loaded, and True; a library that cannot be loaded raises
      :class:`KernelsUnavailable` here rather than sending this rank down another path.
    """
    import torch

    if os.environ.get(PATHS_ENV, "") == "torch":
        log.info("kernels not loaded: %s=torch chose the torch paths", PATHS_ENV)
        return False
    if not torch.cuda.is_available():
        return False
    load()
    return True
