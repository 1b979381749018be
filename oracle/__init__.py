"""The oracle: a CPU restatement of the reference's per-worker KV data path. TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only as the checker (or, for the baseline, as the CPU path being timed). The product,
``everserve_amd``, never imports it and has no CPU fallback.

What it restates, and what pins each part (the tests under ``tests/test_oracle_*.py``):

=========================  ==========================================  =============================
function                   follows (reference file:line)               pinned by
=========================  ==========================================  =============================
gather_rows                core/csrc/gather.cu:29-47,                  brute force over the tensor
                           core/everserve/state/kvcopy.py:89-116       index (numpy), torch advanced
                                                                       indexing per layout
                                                                       (cpu_path), the reference
                                                                       tests' literal shapes
scatter_rows               core/everserve/state/kvcopy.py:118-128,     round trips, untouched rows,
                           core/everserve/state/mirror.py:926-937      torch index_put per layout
scatter_pairs              scatter_rows with each slot's staged row    scatter_rows at rows_of = i
                           named (no reference counterpart)            and on permuted rows; the
                                                                       brute-force gather of what
                                                                       it wrote; skipped pairs
member_sum                 core/everserve/reference/arith/ops.py:63-73 torch's own .to(bfloat16)
                                                                       on fp32 sums, exact integer
                                                                       sums, rounding edge cases,
                                                                       the order-sensitive inputs of
                                                                       core/tests/test_slot_kernel.py
                                                                       :50-55
layout_strides, recognise  core/everserve/state/kvcopy.py:60-72,105-116 torch's own strides of
                                                                       permuted views
staged_step, derive,       core/everserve/state/mirror.py:778-800,     the store's own byte fixture
store_commit,              store/src/storage.rs:521-540,864-957,       (store/tests/service.rs:26-68)
written_ranges             430-451                                     restated; run-copy vs per-row
                                                                       copy
blocks_to_stage,           core/everserve/reference/staging.py:51-94   the reference's literal
expand_blocks                                                          cases
                                                                       (core/tests/test_staging.py)
reduce_protocol            core/csrc/slot.cu:29-40,138-214             the abort/late invariants of
                                                                       core/tests/test_slot_kernel.py
                                                                       :196-224
crc32c, crc32c_rows        the crc32c crate 0.6.8 (store/Cargo.toml:   the published check value and
                           25), RFC 3720 B.4                           RFC 3720's vectors; the CRC's
                                                                       affine law on random data
float_to_bf16,             c10's float -> bfloat16 rule                torch's own conversion on
bf16_to_float                                                          edge cases and random values
cpu_path.*                 core/everserve/state/kvcopy.py:74-128,      equal to the C restatement
                           core/everserve/state/mirror.py:552-562,     byte for byte (gather,
                           926-937, reference/arith/ops.py:63-73       restore, member_sum)
=========================  ==========================================  =============================
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Mapping, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
CFLAGS = ["-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-std=c11", "-Wall"]

_lib: ctypes.CDLL | None = None


def build() -> Path:
    """Compile oracle.c with gcc into oracle/liboracle.so (always: the build is the check)."""
    tmp = HERE / "liboracle.so.tmp"
    subprocess.run(["gcc", *CFLAGS, str(HERE / "oracle.c"), "-o", str(tmp)], check=True)
    os.replace(tmp, LIB)
    return LIB


def lib() -> ctypes.CDLL:
    """The compiled restatement, built on first use when absent."""
    global _lib
    if _lib is None:
        if not LIB.is_file():
            build()
        L = ctypes.CDLL(str(LIB))
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        L.orc_gather_rows.argtypes = [P, I64, P, I64, P, I64, P, I64, I64, I64, P, I64]
        L.orc_gather_rows.restype = None
        L.orc_scatter_rows.argtypes = [P, I64, P, I64, P, I64, P, I64, I64, I64, P, I64]
        L.orc_scatter_rows.restype = None
        L.orc_scatter_pairs.argtypes = [P, I64, P, P, I64, P, I64, P, I64, I64, I64, P, I64]
        L.orc_scatter_pairs.restype = None
        L.orc_member_sum_bf16.argtypes = [P, I64, P, I64]
        L.orc_member_sum_bf16.restype = None
        L.orc_float_to_bf16.argtypes = [ctypes.c_float]
        L.orc_float_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


# ------------------------------------------------------------------------- layouts
KV_FIRST, BLOCKS_FIRST, COMBINED = "kv_first", "blocks_first", "combined"


def recognise(shape: Sequence[int]) -> tuple[str, int, int, int]:
    """(layout, num_blocks, block_size, head_dim) of one layer's cache shape.

    core/everserve/state/kvcopy.py:60-72: [2, nb, bs, h, d] is kv_first, [nb, 2, bs, h, d]
    blocks_first, [nb, h, bs, 2d] combined.
    """
    if len(shape) == 5 and shape[0] == 2:
        return KV_FIRST, shape[1], shape[2], shape[4]
    if len(shape) == 5 and shape[1] == 2:
        return BLOCKS_FIRST, shape[0], shape[2], shape[4]
    if len(shape) == 4 and shape[3] % 2 == 0:
        return COMBINED, shape[0], shape[2], shape[3] // 2
    raise ValueError(f"unsupported KV cache layout {tuple(shape)}")


def layout_strides(layout: str, st: Sequence[int], head_dim: int) -> tuple[int, int, int, int, int]:
    """Element strides (block, offset, head slot, K-or-V, element) of a cache with strides ``st``.

    core/everserve/state/kvcopy.py:105-116.
    """
    if layout == KV_FIRST:  # [2, nb, bs, h, d]
        return st[1], st[2], st[3], st[0], st[4]
    if layout == BLOCKS_FIRST:  # [nb, 2, bs, h, d]
        return st[0], st[2], st[3], st[1], st[4]
    return st[0], st[2], st[1], head_dim * st[3], st[3]  # [nb, h, bs, 2d]


# ------------------------------------------------------------------------- gather / scatter
def _ptr_array(ptrs: Sequence[int]) -> ctypes.Array:
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def gather_rows(layers, slots, heads, capacity: int, d: int, block_size: int, strides, elem: int,
                out=None):
    """Rows [L, H, capacity, 2, d] of raw elements (uint8/16/32) gathered from CPU ``layers``.

    ``layers`` are CPU torch tensors (any strides; the view's first element is its base), read
    through ``strides`` in elements. ``out`` (a numpy array of the right shape) keeps the rows the
    gather does not write; zeros by default.
    """
    dt = {1: np.uint8, 2: np.uint16, 4: np.uint32}[elem]
    if out is None:
        out = np.zeros((len(layers), len(heads), capacity, 2, d), dtype=dt)
    slots = np.ascontiguousarray(np.asarray(slots, dtype=np.int64))
    heads = np.ascontiguousarray(np.asarray(heads, dtype=np.int64))
    st = np.ascontiguousarray(np.asarray(strides, dtype=np.int64))
    assert out.flags.c_contiguous and out.dtype == dt
    lib().orc_gather_rows(
        _ptr_array([t.data_ptr() for t in layers]), len(layers), slots.ctypes.data, len(slots),
        heads.ctypes.data, len(heads), out.ctypes.data, capacity, d, block_size, st.ctypes.data,
        elem,
    )
    return out


def scatter_rows(layers, slots, heads, rows, capacity: int, d: int, block_size: int, strides,
                 elem: int) -> None:
    """Write ``rows`` [L, H, capacity, 2, d] into the CPU ``layers`` in place; negative slots skip."""
    slots = np.ascontiguousarray(np.asarray(slots, dtype=np.int64))
    heads = np.ascontiguousarray(np.asarray(heads, dtype=np.int64))
    st = np.ascontiguousarray(np.asarray(strides, dtype=np.int64))
    rows = np.ascontiguousarray(rows)
    lib().orc_scatter_rows(
        _ptr_array([t.data_ptr() for t in layers]), len(layers), slots.ctypes.data, len(slots),
        heads.ctypes.data, len(heads), rows.ctypes.data, capacity, d, block_size, st.ctypes.data,
        elem,
    )


def scatter_pairs(layers, slots, rows_of, heads, rows, capacity: int, d: int, block_size: int,
                  strides, elem: int) -> None:
    """Write staged row ``rows_of[i]`` at ``slots[i]`` in the CPU ``layers``, in listed order.

    A negative slot, or a row outside ``[0, capacity)``, writes nothing; :func:`scatter_rows` is
    the case ``rows_of[i] = i``.
    """
    slots = np.ascontiguousarray(np.asarray(slots, dtype=np.int64))
    rows_of = np.ascontiguousarray(np.asarray(rows_of, dtype=np.int64))
    if rows_of.shape != slots.shape:
        raise ValueError(f"{slots.size} slots but {rows_of.size} rows")
    heads = np.ascontiguousarray(np.asarray(heads, dtype=np.int64))
    st = np.ascontiguousarray(np.asarray(strides, dtype=np.int64))
    rows = np.ascontiguousarray(rows)
    lib().orc_scatter_pairs(
        _ptr_array([t.data_ptr() for t in layers]), len(layers), slots.ctypes.data,
        rows_of.ctypes.data, len(slots), heads.ctypes.data, len(heads), rows.ctypes.data,
        capacity, d, block_size, st.ctypes.data, elem,
    )


def expand_blocks(block_ids: Sequence[int], block_size: int) -> np.ndarray:
    """Slot ids of whole blocks: block * block_size + [0, block_size), block after block.

    A slot id is block * block_size + offset (core/everserve/state/kvcopy.py:20-21); a block-table
    round copies every slot of each chosen block (core/everserve/reference/staging.py:51-94).
    """
    b = np.asarray(block_ids, dtype=np.int64)
    return (b[:, None] * block_size + np.arange(block_size, dtype=np.int64)[None, :]).reshape(-1)


# ------------------------------------------------------------------------- the reduction
def float_to_bf16(x: np.ndarray) -> np.ndarray:
    """torch's float32 -> bfloat16 bits (c10 round_to_nearest_even; NaN -> 0x7FC0), vectorised."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def bf16_to_float(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def member_sum(inputs: Sequence[np.ndarray | None]) -> np.ndarray:
    """bf16 bits of the members summed in the given order in fp32 from 0.0f, rounded once.

    core/everserve/reference/arith/ops.py:63-73. ``None`` is a member that never arrived: +0.0f.
    """
    present = [x for x in inputs if x is not None]
    n = len(present[0]) if present else 0
    arrs = [None if x is None else np.ascontiguousarray(x, dtype=np.uint16) for x in inputs]
    ptrs = (ctypes.c_void_p * len(arrs))(*[0 if a is None else a.ctypes.data for a in arrs])
    out = np.empty(n, dtype=np.uint16)
    lib().orc_member_sum_bf16(ptrs, len(arrs), out.ctypes.data, n)
    return out


REDUCE_DONE, REDUCE_ABORTED, REDUCE_TIMED_OUT = 0, 1, 2


def reduce_protocol(
    buffers: Mapping[int, np.ndarray],
    flags: Mapping[int, int],
    order: Sequence[int],
    epoch: int,
    abort: bool = False,
) -> tuple[np.ndarray, int, int]:
    """What the bounded local reduction must produce: (bf16 bits, reason, late rows).

    A member whose flag is not ``epoch`` never arrives within the wait; the wait ends by the abort
    word (``abort``) or by the timeout, the missing members contribute zeros (core/csrc/slot.cu:148)
    and are named in the late mask (slot.cu:179-192). With every flag in, reason 0 and mask 0.
    """
    missing = [r for r in order if flags.get(r) != epoch]
    late = 0
    for r in missing:
        late |= 1 << r
    reason = REDUCE_DONE
    if missing:
        reason = REDUCE_ABORTED if abort else REDUCE_TIMED_OUT
    out = member_sum([None if r in missing else buffers[r] for r in order])
    return out, reason, late


# ------------------------------------------------------------------------- the store's row layout
HEAD_STRIDE = 1000
"""Table id = layer * 1000 + head slot (core/everserve/state/mirror.py:59)."""
DTYPE_BYTES = {
    "float8_e4m3fn": 1, "float8_e5m2": 1, "int8": 1, "uint8": 1,
    "float16": 2, "bfloat16": 2, "int16": 2, "float32": 4, "int32": 4, "float64": 8, "int64": 8,
}
"""store/src/storage.rs:542-551."""


def staged_step(stage: str, layers: Sequence[int], heads: Sequence[int], capacity: int,
                head_dim: int, elem: int, slots: Sequence[int], dtype: str) -> dict:
    """The StagedStep descriptor of a [L, H, capacity, 2, d] staging file.

    core/everserve/state/mirror.py:778-800 and proto/everserve/proto/mirror.proto:32-54.
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
        "slots": [int(s) for s in slots],
        "dtype": dtype,
        "shape": [2, head_dim],
    }


def derive(step: Mapping) -> list[tuple[int, int]]:
    """(table id, byte offset) of every (layer, head) the descriptor names, layer-major.

    store/src/storage.rs:521-540: offset = base + layer * layer_stride + h * head_stride with h
    the head's index in ``heads`` and the layer its id.
    """
    out = []
    for layer in step["layers"]:
        for h, head in enumerate(step["heads"]):
            out.append((layer * step["table_stride"] + head,
                        step["base_offset"] + layer * step["layer_stride"] + h * step["head_stride"]))
    return out


def store_commit(stage_bytes: np.ndarray, step: Mapping, tables: dict[int, np.ndarray],
                 num_slots: int, written: dict[int, np.ndarray], step_no: int,
                 crcs: dict[int, np.ndarray] | None = None) -> None:
    """Copy the staged rows into per-(layer, head) tables, as the store's commit does.

    store/src/storage.rs:864-957 (copy loop 916-943): for each table, runs of consecutive
    non-negative slot ids copy as one memcpy from ``offset + i * row_bytes``; padding (negative)
    is skipped; each written slot records max(step_no, 1) (Layer::note_written, :498-504) and,
    when ``crcs`` is given, the CRC32C of its row as it stands after the copy
    (Layer::mark_written, :494-497). Tables are created zeroed on first use as
    ``num_slots * row_bytes`` bytes. Every slot id is checked before anything is written.
    """
    row_bytes = step["shape"][0] * step["shape"][1] * DTYPE_BYTES[step["dtype"]]
    slots = step["slots"]
    for s in slots:
        if s >= num_slots:
            raise ValueError(f"slot {s} outside 0..{num_slots}")
    for table, offset in derive(step):
        if table not in tables:
            tables[table] = np.zeros(num_slots * row_bytes, dtype=np.uint8)
            written[table] = np.zeros(num_slots, dtype=np.uint64)
            if crcs is not None:
                crcs[table] = np.zeros(num_slots, dtype=np.uint32)
        rows, marks = tables[table], written[table]
        i = 0
        while i < len(slots):
            s = slots[i]
            if s < 0:
                i += 1
                continue
            run = 1
            while i + run < len(slots) and slots[i + run] == s + run:
                run += 1
            src = offset + i * row_bytes
            rows[s * row_bytes:(s + run) * row_bytes] = stage_bytes[src:src + run * row_bytes]
            marks[s:s + run] = max(step_no, 1)
            i += run
        if crcs is not None:
            live = np.array(sorted({s for s in slots if s >= 0}), dtype=np.int64)
            if live.size:
                crcs[table][live] = crc32c_rows(rows.reshape(num_slots, row_bytes)[live])


_CRC32C_TABLE: np.ndarray | None = None


def _crc32c_table() -> np.ndarray:
    """The byte table of the reflected Castagnoli polynomial, built bit by bit."""
    global _CRC32C_TABLE
    if _CRC32C_TABLE is None:
        t = np.zeros(256, dtype=np.uint32)
        for i in range(256):
            c = i
            for _ in range(8):
                c = (c >> 1) ^ (0x82F63B78 if c & 1 else 0)
            t[i] = c
        _CRC32C_TABLE = t
    return _CRC32C_TABLE


def crc32c_rows(rows: np.ndarray) -> np.ndarray:
    """CRC32C (Castagnoli, RFC 3720 B.4: reflected polynomial 0x82F63B78, initial value and
    final xor 0xFFFFFFFF) of every row of a [n, row_bytes] uint8 array, one byte of every row at
    a time. The store keeps one per written row (store/src/storage.rs:371-373, the crc32c crate
    0.6.8, store/Cargo.toml:25)."""
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    t = _crc32c_table()
    c = np.full(rows.shape[0], 0xFFFFFFFF, dtype=np.uint32)
    for j in range(rows.shape[1]):
        c = t[(c ^ rows[:, j]) & 0xFF] ^ (c >> np.uint32(8))
    return c ^ np.uint32(0xFFFFFFFF)


def crc32c(data) -> int:
    """CRC32C of one byte string (see crc32c_rows)."""
    a = np.frombuffer(bytes(data), dtype=np.uint8)
    return int(crc32c_rows(a.reshape(1, -1))[0])


def written_ranges(marks: np.ndarray, since_step: int = 0) -> list[tuple[int, int]]:
    """(start, count) runs of slots written after ``since_step`` (store/src/storage.rs:430-451)."""
    hit = marks > since_step
    out, i, n = [], 0, len(marks)
    while i < n:
        if hit[i]:
            start = i
            while i < n and hit[i]:
                i += 1
            out.append((start, i - start))
        else:
            i += 1
    return out


# ------------------------------------------------------------------------- block-table rounds
def blocks_to_stage(block_tables: Mapping[str, Sequence[int]], num_computed: Mapping[str, int],
                    staged: dict[str, tuple[int, tuple[int, ...]]], block_size: int) -> list[int]:
    """The blocks holding KV written since the previous round; updates ``staged`` in place.

    core/everserve/reference/staging.py:51-94. ``staged`` maps a request to (tokens staged, the
    block ids they were staged from). Staging restarts at the first block whose id changed; a
    request no longer computed is dropped.
    """
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    chosen: set[int] = set()
    for rid, n in num_computed.items():
        table = tuple(block_tables[rid])
        done, old = staged.get(rid, (0, ()))
        same = 0
        while same < min(len(old), len(table)) and old[same] == table[same]:
            same += 1
        done = min(done, same * block_size, n)
        if n > done:
            chosen.update(table[done // block_size:(n - 1) // block_size + 1])
        staged[rid] = (n, table[:(n + block_size - 1) // block_size])
    for rid in [r for r in staged if r not in num_computed]:
        del staged[rid]
    return sorted(chosen)
