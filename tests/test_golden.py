"""The committed golden fixtures (tests/golden/), on the CPU.

The fixtures were written by tests/golden/make_fixtures.py from the oracle on fixed seeds; the
reference stores no golden vectors of its own. Here the oracle must still produce them byte for
byte:
* the gather of the reference tests' literal case (3 layouts x d in {8, 6} x bf16, f16, f32 and
  fp8) from the stored caches;
* the scatter of the stored rows, in staged order and by the stored pairs;
* the ordered sums at {16384, 3000, 2} and the order-sensitive case;
* config C1.

The seeded inputs must also still come out of torch's and numpy's generators the same way, so
that a GPU run rebuilds exactly the inputs the fixtures were made from.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.cases import brute_scatter, strides_of
from tests.golden import make_fixtures as mf

GOLDEN = Path(__file__).resolve().parent / "golden"
G = np.load(GOLDEN / "gather_literal.npz")
R = np.load(GOLDEN / "reduce_sizes.npz")
C1 = json.loads((GOLDEN / "c1.json").read_text())
CASES = sorted({k.rsplit("_", 1)[0] for k in G.files if k.endswith("_rows")})


SIGNED = {np.dtype(np.uint8): np.uint8, np.dtype(np.uint16): np.int16,
          np.dtype(np.uint32): np.int32}


def tensors(case: str) -> list[torch.Tensor]:
    """The stored caches of a case as CPU tensors of their dtype, bit for bit."""
    layout, dname, tname = case.rsplit("_", 2)
    d = int(dname[1:])
    shape = {"kv_first": (2, 7, 4, 3, d), "blocks_first": (7, 2, 4, 3, d),
             "combined": (7, 3, 4, 2 * d)}[layout]
    bits = G[f"{case}_cache"]
    return [torch.from_numpy(b.view(SIGNED[b.dtype]).copy()).view(mf.DTYPES[tname]).reshape(shape)
            for b in bits]


def test_every_literal_case_is_present():
    assert len(CASES) == 3 * 2 * 4


@pytest.mark.parametrize("case", CASES)
def test_the_oracle_gathers_the_stored_rows(case):
    layers = tensors(case)
    e = layers[0].element_size()
    d = int(case.rsplit("_", 2)[1][1:])
    got = oracle.gather_rows(layers, G["slots"], G["heads"], int(G["capacity"]), d,
                             int(G["block_size"]), strides_of(layers[0]), e)
    assert np.array_equal(got, G[f"{case}_rows"])


@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_oracle_scatters_the_stored_rows(case):
    layers = [torch.zeros_like(t) for t in tensors(case)]
    d = int(case.rsplit("_", 2)[1][1:])
    oracle.scatter_rows(layers, G["slots"], G["heads"], G[f"{case}_rows"], int(G["capacity"]), d,
                        int(G["block_size"]), strides_of(layers[0]), 2)
    assert np.array_equal(np.stack([mf.raw(t) for t in layers]), G[f"{case}_scattered"])


@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_oracle_scatters_the_stored_pairs(case):
    layers = [torch.zeros_like(t) for t in tensors(case)]
    d = int(case.rsplit("_", 2)[1][1:])
    oracle.scatter_pairs(layers, G["pair_slots"], G["pair_rows_of"], G["heads"],
                         G[f"{case}_rows"], int(G["capacity"]), d, int(G["block_size"]),
                         strides_of(layers[0]), 2)
    assert np.array_equal(np.stack([mf.raw(t) for t in layers]), G[f"{case}_paired"])


def stored_range_slots() -> np.ndarray:
    return np.concatenate([np.arange(a, a + k, dtype=np.int64)
                           for a, k in zip(G["range_starts"], G["range_counts"])])


@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_stored_range_scatter_is_the_scatter_at_the_ranges_slots(case):
    """The range case's caches: the oracle's slot scatter at the ranges' slots writes them, and
    so does the scatter by its definition per layout (tests/cases.py:brute_scatter)."""
    slots = stored_range_slots()
    assert len(slots) == int(G["capacity"])
    layers = [torch.zeros_like(t) for t in tensors(case)]
    d = int(case.rsplit("_", 2)[1][1:])
    rows = G[f"{case}_rows"]
    brute = np.stack(brute_scatter(layers, slots, G["heads"], rows))
    oracle.scatter_rows(layers, slots, G["heads"], rows, int(G["capacity"]), d,
                        int(G["block_size"]), strides_of(layers[0]), 2)
    assert np.array_equal(np.stack([mf.raw(t) for t in layers]), G[f"{case}_ranged"])
    assert np.array_equal(brute.view(np.uint16), G[f"{case}_ranged"])


def test_the_stored_inputs_still_come_from_the_seeds():
    for case in ("kv_first_d8_bf16", "combined_d6_fp8"):
        layout, dname, tname = case.rsplit("_", 2)
        fresh = mf.caches(layout, int(dname[1:]), mf.DTYPES[tname])
        assert np.array_equal(np.stack([mf.raw(t) for t in fresh]), G[f"{case}_cache"])
    for n in (16384, 3000, 2):
        for r in range(3):
            assert np.array_equal(mf.raw(mf.member_input(r, n)), R[f"n{n}_member{r}"])


@pytest.mark.parametrize("n", [16384, 3000, 2])
def test_the_oracle_sums_the_stored_members(n):
    xs = [R[f"n{n}_member{r}"] for r in range(3)]
    for order in ("012", "201"):
        got = oracle.member_sum([xs[int(c)] for c in order])
        assert np.array_equal(got, R[f"n{n}_sum_{order}"])


def test_the_order_sensitive_sums_differ_and_match():
    xs = [R[f"ordered_member{r}"] for r in range(3)]
    a = oracle.member_sum([xs[0], xs[1], xs[2]])
    b = oracle.member_sum([xs[0], xs[2], xs[1]])
    assert np.array_equal(a, R["ordered_sum_012"]) and np.array_equal(b, R["ordered_sum_021"])
    assert not np.array_equal(a, b)


def test_c1_inputs_and_rows_match_the_digests():
    layers, slots, heads = mf.c1_inputs()
    assert mf.digest(mf.raw(t) for t in layers) == C1["cache_sha256"]
    rows = oracle.gather_rows(layers, slots, heads, len(slots), C1["head_dim"], C1["block_size"],
                              strides_of(layers[0]), 2)
    assert list(rows.shape) == C1["rows_shape"]
    assert mf.digest([rows]) == C1["rows_sha256"]
    s = C1["sample"]
    assert rows[s["layer"], s["head_index"], :s["first_rows"]].reshape(-1).tolist() == s["bits"]
