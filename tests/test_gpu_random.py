"""The row kernels against the oracle over seeded random cases, byte for byte, on the GPU.

The cases are the CPU pins' (tests/cases.py:random_case, pinned in tests/test_oracle_random.py):
every layout, four element types, head dims on the 16-byte path and off it, block sizes that are
powers of two and not (the kernels' shift and division paths), held heads in any order, padding,
and caches that are views of wider tensors or permuted. A view's device copy keeps its strides.
The gather writes into a buffer filled with a sentinel, so the rows past n must keep it; the
scatters write into caches of random content, compared whole (the head a view leaves out too).
"""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.cases import NP_BITS, TORCH_BITS, bits, random_case, strides_of

pytestmark = pytest.mark.gpu

# EVERSERVE_RANDOM_CASES widens the sweep for a longer run; 40 by default
SEEDS = range(int(os.environ.get("EVERSERVE_RANDOM_CASES", "40")))
SENTINEL = {1: 0x5A, 2: 0x5A5A, 4: 0x5A5A5A5A}
SIGNED = {1: np.uint8, 2: np.int16, 4: np.int32}


def dev_long(xs):
    return torch.tensor(np.asarray(xs, dtype=np.int64), dtype=torch.long, device="cuda")


def on_device(c):
    """(CPU caches, their bases, device caches, their bases): the same views of the same bytes."""
    base_gpu = [t.cuda() for t in c["base"]]
    return ([c["view"](t) for t in c["base"]], c["base"], [c["view"](t) for t in base_gpu],
            base_gpu)


def ptrs(layers):
    return dev_long([t.data_ptr() for t in layers])


def staged_bits(c, n_layers, e):
    return c["rng"].integers(0, 1 << (8 * e), size=(n_layers, len(c["heads"]), c["cap"], 2, c["d"]),
                             dtype=np.uint64).astype(NP_BITS[e])


def gather_out(shape, e):
    return (np.full(shape, SENTINEL[e], dtype=NP_BITS[e]),
            torch.full(shape, SENTINEL[e], dtype=TORCH_BITS[e], device="cuda"))


@pytest.mark.parametrize("seed", SEEDS)
def test_gather_rows(ext, seed):
    c = random_case(seed)
    cpu, _, gpu, _ = on_device(c)
    e = cpu[0].element_size()
    want, out = gather_out((len(cpu), len(c["heads"]), c["cap"], 2, c["d"]), e)
    oracle.gather_rows(cpu, c["slots"], c["heads"], c["cap"], c["d"], c["bs"], strides_of(cpu[0]),
                       e, out=want)
    ext.gather_rows(ptrs(gpu), dev_long(c["slots"]), dev_long(c["heads"]), out.data_ptr(),
                    c["cap"], c["d"], c["bs"], list(strides_of(gpu[0])), e)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(NP_BITS[e]), want)


@pytest.mark.parametrize("seed", SEEDS)
def test_gather_blocks(ext, seed):
    c = random_case(seed)
    cpu, _, gpu, _ = on_device(c)
    e = cpu[0].element_size()
    k = int(c["rng"].integers(1, min(c["nb"], 12) + 1))
    blocks = c["rng"].choice(c["nb"], size=k, replace=False).astype(np.int32)
    if k > 1 and c["rng"].random() < 0.3:
        blocks[int(c["rng"].integers(k))] = -1  # a padding block: its rows read slot 0
    slots = oracle.expand_blocks(blocks, c["bs"])
    cap = len(slots) + int(c["rng"].integers(0, 3))
    want, out = gather_out((len(cpu), len(c["heads"]), cap, 2, c["d"]), e)
    oracle.gather_rows(cpu, slots, c["heads"], cap, c["d"], c["bs"], strides_of(cpu[0]), e,
                       out=want)
    tags = torch.full((len(slots),), -999, dtype=torch.long, device="cuda")
    ext.gather_blocks(ptrs(gpu), torch.from_numpy(blocks).cuda(), dev_long(c["heads"]),
                      out.data_ptr(), cap, c["d"], c["bs"], list(strides_of(gpu[0])), e,
                      slots_out=tags)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(NP_BITS[e]), want)
    assert tags.cpu().tolist() == slots.tolist()


@pytest.mark.parametrize("ordered", [None, True])
@pytest.mark.parametrize("seed", SEEDS)
def test_scatter_rows(ext, seed, ordered):
    """As scatter_rows runs at these sizes (staged order), and with the pairs sorted by slot
    first, as it runs from 2^18 slots and 8 GiB."""
    c = random_case(seed)
    cpu, base_cpu, gpu, base_gpu = on_device(c)
    e = cpu[0].element_size()
    staged = staged_bits(c, len(cpu), e)
    oracle.scatter_rows(cpu, c["slots"], c["heads"], staged, c["cap"], c["d"], c["bs"],
                        strides_of(cpu[0]), e)
    rows = torch.from_numpy(staged.view(SIGNED[e])).cuda()
    ext.scatter_rows(ptrs(gpu), dev_long(c["slots"]), dev_long(c["heads"]), rows.data_ptr(),
                     c["cap"], c["d"], c["bs"], list(strides_of(gpu[0])), e, ordered=ordered)
    torch.cuda.synchronize()
    for a, b in zip(base_gpu, base_cpu):
        assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("seed", SEEDS)
def test_scatter_pairs(ext, seed):
    c = random_case(seed)
    cpu, base_cpu, gpu, base_gpu = on_device(c)
    e = cpu[0].element_size()
    staged = staged_bits(c, len(cpu), e)
    n = len(c["slots"])
    rows_of = c["rng"].integers(-1, c["cap"] + 1, size=n)  # a few outside the buffer: no write
    oracle.scatter_pairs(cpu, c["slots"], rows_of, c["heads"], staged, c["cap"], c["d"], c["bs"],
                         strides_of(cpu[0]), e)
    rows = torch.from_numpy(staged.view(SIGNED[e])).cuda()
    ext.scatter_pairs(ptrs(gpu), dev_long(c["slots"]), dev_long(rows_of), dev_long(c["heads"]),
                      rows.data_ptr(), c["cap"], c["d"], c["bs"], list(strides_of(gpu[0])), e)
    torch.cuda.synchronize()
    for a, b in zip(base_gpu, base_cpu):
        assert np.array_equal(bits(a), bits(b))


def random_ranges(rng, num_slots: int, room: int):
    """Written ranges as a restore gets them: runs of a random written mask, in slot order or
    (one case in four) shuffled, with empty ranges among them, at most ``room`` rows in all.
    Returns (starts, counts)."""
    written = rng.random(num_slots) < rng.uniform(0.2, 0.9)
    edges = np.flatnonzero(np.diff(np.concatenate(([0], written.view(np.int8), [0]))))
    starts, counts = list(edges[0::2]), list(edges[1::2] - edges[0::2])
    for _ in range(int(rng.integers(0, 3))):  # empty ranges anywhere
        at = int(rng.integers(0, len(starts) + 1))
        starts.insert(at, int(rng.integers(0, num_slots)))
        counts.insert(at, 0)
    starts, counts = np.array(starts, dtype=np.int64), np.array(counts, dtype=np.int64)
    if len(starts) and rng.random() < 0.25:
        order = rng.permutation(len(starts))
        starts, counts = starts[order], counts[order]
    keep = np.cumsum(counts) <= room
    if not keep.all():  # trim to the room: the last kept range may be cut short
        k = int(np.argmin(keep))
        counts = counts[:k + 1].copy()
        counts[k] -= int(counts.sum() - room)
        starts = starts[:k + 1]
    if len(starts) == 0:
        starts, counts = np.array([0], dtype=np.int64), np.array([min(1, room)], dtype=np.int64)
    return starts, counts


@pytest.mark.parametrize("seed", SEEDS)
def test_scatter_ranges(ext, seed):
    """The range scatter writes what the slot scatter writes at the ranges' slots, expanded."""
    c = random_case(seed)
    cpu, base_cpu, gpu, base_gpu = on_device(c)
    e = cpu[0].element_size()
    staged = staged_bits(c, len(cpu), e)
    starts, counts = random_ranges(c["rng"], c["nb"] * c["bs"], c["cap"])
    slots = np.concatenate([np.arange(a, a + k, dtype=np.int64) for a, k in zip(starts, counts)])
    first_rows = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    oracle.scatter_rows(cpu, slots, c["heads"], staged, c["cap"], c["d"], c["bs"],
                        strides_of(cpu[0]), e)
    rows = torch.from_numpy(staged.view(SIGNED[e])).cuda()
    ext.scatter_ranges(ptrs(gpu), dev_long(starts), dev_long(first_rows), len(slots),
                       dev_long(c["heads"]), rows.data_ptr(), c["cap"], c["d"], c["bs"],
                       list(strides_of(gpu[0])), e)
    torch.cuda.synchronize()
    for a, b in zip(base_gpu, base_cpu):
        assert np.array_equal(bits(a), bits(b))
