"""Pins of the oracle's gather and scatter (oracle/oracle.c), on the CPU.

Three formulations must agree byte for byte: the C oracle (five strides), a brute force by
tensor dimension per layout (tests/cases.py), and the reference's torch path by advanced indexing
(oracle/cpu_path.py, restating core/everserve/state/kvcopy.py:89-128). The cases are the
reference tests' literal shapes (core/tests/test_gather_kernel.py:67-102). Planted mistakes in the
oracle's inputs (swapped strides, K and V exchanged, no padding clamp) must be caught.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_path
from tests.cases import (BS, CAPACITY, DTYPES, H, HEADS, LAYOUTS, NB, SLOTS, bits, brute_gather,
                         caches, strides_of)


def oracle_gather(layers, slots, heads, capacity=CAPACITY, strides=None):
    layout, _, bs, d = oracle.recognise(layers[0].shape)
    return oracle.gather_rows(layers, slots, heads, capacity, d, bs,
                              strides or strides_of(layers[0]), layers[0].element_size())


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("dtype", DTYPES)
def test_gather_matches_the_brute_force_and_the_torch_path(layout, d, dtype):
    layers = caches(layout, d, dtype)
    got = oracle_gather(layers, SLOTS, HEADS)
    assert np.array_equal(got, brute_gather(layers, SLOTS, HEADS, CAPACITY))
    torch_path = cpu_path.gather_step(layers, torch.tensor(SLOTS), torch.tensor(HEADS), CAPACITY)
    assert np.array_equal(got, bits(torch_path))
    # rows n..capacity-1 are not written
    assert not got[:, :, len(SLOTS):].any()


def test_a_strided_cache_view_is_read_through_its_strides():
    big = caches("kv_first", 8, torch.bfloat16)
    layers = [t[:, :, :, 1:] for t in big]  # head slots 1.. of a wider cache: not contiguous
    assert not layers[0].is_contiguous()
    got = oracle_gather(layers, SLOTS, [0, 1])
    assert np.array_equal(got, brute_gather(layers, SLOTS, [0, 1], CAPACITY))


def test_rows_of_heads_is_the_per_head_rows_in_one_gather():
    # core/tests/test_kvcopy.py:48-57: rows_of_heads[h] == rows(head).T
    for layout in LAYOUTS:
        t = caches(layout, 8, torch.bfloat16, n_layers=1)[0]
        slots = torch.tensor([0, 5, 9, 27])
        heads = torch.tensor([1, 0])
        got = cpu_path.rows_of_heads(t, slots, heads)
        for h, head in enumerate(heads.tolist()):
            assert torch.equal(got[h].transpose(0, 1), cpu_path.rows(t, slots, head))


@pytest.mark.parametrize("mistake", ["block<->offset", "k<->v", "no clamp", "head order"])
def test_planted_mistakes_are_caught(mistake):
    layers = caches("kv_first", 8, torch.bfloat16)
    want = brute_gather(layers, SLOTS, HEADS, CAPACITY)
    s = list(strides_of(layers[0]))
    slots, heads = list(SLOTS), list(HEADS)
    if mistake == "block<->offset":
        s[0], s[1] = s[1], s[0]
    elif mistake == "k<->v":
        # K and V exchanged: the base at the V half and the K/V stride stepping back to K
        s[3] = -s[3]
        layers = [t[1] for t in layers]
    elif mistake == "no clamp":
        slots = [27 if x < 0 else x for x in slots]  # padding read from another slot than 0
    else:
        heads = heads[::-1]
    got = oracle.gather_rows(layers, slots, heads, CAPACITY, 8, 4, s, 2)
    assert not np.array_equal(got, want)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
def test_scatter_inverts_the_gather_and_touches_nothing_else(layout, d):
    src = caches(layout, d, torch.bfloat16, seed=5)
    staged = oracle_gather(src, SLOTS, HEADS)
    dst = [torch.zeros_like(t) for t in src]
    _, _, bs, _ = oracle.recognise(src[0].shape)
    oracle.scatter_rows(dst, SLOTS, HEADS, staged, CAPACITY, d, bs, strides_of(dst[0]), 2)
    # gather back: the written rows round-trip; the padding row (slot 0 via -1) came from slot 0
    # of the source only where slot 0 itself was written (it is: SLOTS holds 0)
    back = oracle_gather(dst, [s for s in SLOTS if s >= 0], HEADS)
    want = oracle_gather(src, [s for s in SLOTS if s >= 0], HEADS)
    assert np.array_equal(back, want)
    # everything else is still zero: the written elements are exactly the (slot, held head) rows
    touched = sum(int((bits(t) != 0).sum()) for t in dst)
    n_written = len(src) * len(HEADS) * len([s for s in SLOTS if s >= 0]) * 2 * d
    nonzero_src = int((want != 0).sum())
    assert touched == nonzero_src <= n_written
    # the torch path (index_put per (layer, head)) writes the same bytes
    dst2 = [torch.zeros_like(t) for t in src]
    cpu_path.restore_step(dst2, torch.tensor(SLOTS), HEADS, torch.from_numpy(staged).view(torch.bfloat16))
    for a, b in zip(dst, dst2):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_scatter_skips_padding():
    src = caches("kv_first", 8, torch.bfloat16, seed=6)
    staged = oracle_gather(src, [-1, 3], [0])
    dst = [torch.zeros_like(t) for t in src]
    oracle.scatter_rows(dst, [-1, 3], [0], staged, CAPACITY, 8, 4, strides_of(dst[0]), 2)
    for t in dst:
        assert not bits(t)[:, 0, 0].any()  # slot 0 untouched although the padding row read it
        assert bits(t)[:, 0, 3, 0].any()


def test_expand_blocks_is_block_times_size_plus_offset():
    assert oracle.expand_blocks([2, 0, 5], 4).tolist() == [8, 9, 10, 11, 0, 1, 2, 3, 20, 21, 22, 23]
    assert oracle.expand_blocks([], 16).tolist() == []


def test_layout_strides_follow_the_tensor():
    # kv_first [2, nb, bs, h, d] contiguous: block = bs*h*d, offset = h*d, head = d, kv = nb*bs*h*d
    t = torch.zeros(2, 7, 4, 3, 8)
    assert strides_of(t) == (96, 24, 8, 672, 1)
    # combined as the reference's tests build it: [nb, bs, h, 2d] permuted to [nb, h, bs, 2d]
    c = torch.zeros(6, 4, 3, 16).permute(0, 2, 1, 3)
    assert oracle.recognise(c.shape) == ("combined", 6, 4, 8)
    assert strides_of(c) == (192, 48, 16, 8, 1)
    with pytest.raises(ValueError):
        oracle.recognise((3, 3, 3))


PAIR_SLOTS = [17, 5, -1, 27, 0, 9]
PAIR_ROWS = [3, 0, 1, 4, 9, 3]  # row 9 lies outside CAPACITY: that pair writes nothing


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
def test_scatter_pairs_at_the_identity_is_the_scatter(layout, d):
    src = caches(layout, d, torch.bfloat16, seed=11)
    staged = oracle_gather(src, SLOTS, HEADS)
    _, _, bs, _ = oracle.recognise(src[0].shape)
    a = [torch.zeros_like(t) for t in src]
    b = [torch.zeros_like(t) for t in src]
    oracle.scatter_rows(a, SLOTS, HEADS, staged, CAPACITY, d, bs, strides_of(a[0]), 2)
    oracle.scatter_pairs(b, SLOTS, range(len(SLOTS)), HEADS, staged, CAPACITY, d, bs,
                         strides_of(b[0]), 2)
    for x, y in zip(a, b):
        assert np.array_equal(bits(x), bits(y))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
def test_scatter_pairs_writes_the_named_rows_and_nothing_else(layout, d):
    src = caches(layout, d, torch.bfloat16, seed=12)
    staged = oracle_gather(src, list(range(CAPACITY)), HEADS)  # 8 distinct staged rows
    _, _, bs, _ = oracle.recognise(src[0].shape)
    dst = [torch.zeros_like(t) for t in src]
    oracle.scatter_pairs(dst, PAIR_SLOTS, PAIR_ROWS, HEADS, staged, CAPACITY, d, bs,
                         strides_of(dst[0]), 2)
    # the brute force (by tensor dimension, not by strides) reads back exactly the named rows
    kept = [(s, r) for s, r in zip(PAIR_SLOTS, PAIR_ROWS) if s >= 0 and 0 <= r < CAPACITY]
    back = brute_gather(dst, [s for s, _ in kept], HEADS, len(kept))
    assert np.array_equal(back, staged[:, :, [r for _, r in kept]])
    # the same as the plain scatter of the rows in pair order
    again = [torch.zeros_like(t) for t in src]
    oracle.scatter_rows(again, [s for s, _ in kept], HEADS,
                        np.ascontiguousarray(staged[:, :, [r for _, r in kept]]), len(kept), d, bs,
                        strides_of(again[0]), 2)
    for x, y in zip(dst, again):
        assert np.array_equal(bits(x), bits(y))
    # and nothing else: every other element is still zero
    touched = sum(int((bits(t) != 0).sum()) for t in dst)
    assert touched == int((back != 0).sum())


def test_scatter_pairs_refuses_mismatched_lists():
    dst = [torch.zeros(2, NB, BS, H, 8, dtype=torch.bfloat16)]
    with pytest.raises(ValueError):
        oracle.scatter_pairs(dst, [1, 2], [0], [0], np.zeros((1, 1, 8, 2, 8), np.uint16), 8, 8,
                             BS, strides_of(dst[0]), 2)
