"""The step path's host logic, on the CPU: the staging capacity rule and the descriptor.

``capacity_for`` is core/everserve/state/mirror.py:596 (``max(8, next_pow2(n))``), checked against
the smallest power of two that holds ``n`` found by search. ``describe`` builds the ``StagedStep``
the store reads (core/everserve/state/mirror.py:778-800). It is checked against the oracle's
``staged_step``, which the store's own byte case pins. It is also checked against the offsets the
store derives (store/src/storage.rs:521-540), computed by hand for a small case.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import staging


def test_capacity_is_the_smallest_power_of_two_from_eight_that_holds_the_step():
    for n in range(1, 5000):
        c = 8
        while c < n:
            c *= 2
        assert staging.capacity_for(n) == c, n
    assert staging.capacity_for(16384) == 16384
    assert staging.capacity_for(16385) == 32768
    with pytest.raises(ValueError):
        staging.capacity_for(0)


@pytest.mark.parametrize("layers,heads,cap,d,elem,dtype", [
    ([0, 1, 2], [0, 2], 8, 8, 2, "bfloat16"),
    ([2, 0], [5], 16, 128, 1, "float8_e4m3fn"),
    (list(range(32)), list(range(8)), 16384, 128, 2, "bfloat16"),
])
def test_the_descriptor_is_the_oracles(layers, heads, cap, d, elem, dtype):
    slots = [5, -1, 17, 0, 27]
    got = staging.describe("stage3.rows", layers, heads, cap, d, elem, slots, dtype)
    want = oracle.staged_step("stage3.rows", layers, heads, cap, d, elem, slots, dtype)
    assert got == want
    # slot ids handed over as a numpy array (the stager's pinned copy): the same descriptor,
    # holding Python ints of its own
    arr = np.array(slots, dtype=np.int64)
    from_array = staging.describe("stage3.rows", layers, heads, cap, d, elem, arr, dtype)
    assert from_array == want and all(type(x) is int for x in from_array["slots"])
    arr[0] = 99
    assert from_array["slots"][0] == 5


def test_the_store_derives_the_offsets_of_the_layout():
    # two heads, capacity 8, d 4 of bf16: a row is 16 bytes, a head 128, a layer 256
    step = staging.describe("s", [1, 0], [3, 7], 8, 4, 2, [0, 1], "bfloat16")
    assert oracle.derive(step) == [(3, 0), (7, 128), (1003, 256), (1007, 384)]


def test_dtype_names_are_the_stores():
    for dt, name in staging.DTYPE_NAMES.items():
        assert oracle.DTYPE_BYTES[name] == torch.empty((), dtype=dt).element_size()
