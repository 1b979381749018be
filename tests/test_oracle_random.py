"""The oracle's gather and scatter over seeded random cases, on the CPU.

Each case (tests/cases.py:random_case) draws a layout, element type, head dim, block size (powers
of two and not), held-head list in any order, slot list with padding, spare capacity, and a
contiguous, head-sliced or permuted cache. The oracle reads and writes through five strides; the
brute forces below index by tensor dimension per layout, and the reference's torch path by
advanced indexing (oracle/cpu_path.py, restating core/everserve/state/kvcopy.py:89-128). All three
must agree byte for byte.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_path
from tests.cases import NP_BITS, bits, brute_gather, brute_scatter, random_case, strides_of

SEEDS = range(40)


@pytest.mark.parametrize("seed", SEEDS)
def test_the_gather_agrees_with_the_brute_force_and_the_torch_path(seed):
    c = random_case(seed)
    layers = [c["view"](t) for t in c["base"]]
    e = layers[0].element_size()
    got = oracle.gather_rows(layers, c["slots"], c["heads"], c["cap"], c["d"], c["bs"],
                             strides_of(layers[0]), e)
    assert np.array_equal(got, brute_gather(layers, c["slots"], c["heads"], c["cap"]))
    torch_path = cpu_path.gather_step(layers, torch.from_numpy(c["slots"]),
                                      torch.tensor(c["heads"]), c["cap"])
    assert np.array_equal(got, bits(torch_path))


@pytest.mark.parametrize("seed", SEEDS)
def test_the_scatter_agrees_with_the_brute_force(seed):
    c = random_case(seed)
    layers = [c["view"](t.clone()) for t in c["base"]]
    e = layers[0].element_size()
    staged = c["rng"].integers(0, 1 << (8 * e), size=(len(layers), len(c["heads"]), c["cap"], 2,
                                                      c["d"]), dtype=np.uint64).astype(NP_BITS[e])
    want = brute_scatter(layers, c["slots"], c["heads"], staged)
    oracle.scatter_rows(layers, c["slots"], c["heads"], staged, c["cap"], c["d"], c["bs"],
                        strides_of(layers[0]), e)
    for t, w in zip(layers, want):
        assert np.array_equal(bits(t), w)
