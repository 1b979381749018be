"""Write the golden fixtures under tests/golden/ from the oracle, on fixed seeds.

The reference stores no golden vectors: its tests seed generators at run time
(core/tests/test_gather_kernel.py:37, core/tests/test_slot_kernel.py:45-55). These fixtures are
therefore this build's own. They are made by the oracle (oracle/, the CPU restatement), on the
reference tests' literal shapes and seeds, and committed so that every later build of the oracle
and of the HIP path is checked against the same bytes:

* gather_literal.npz: the gather of core/tests/test_gather_kernel.py:18-20,67-102. That is 7
  blocks of 4 slots, 3 head slots and 3 layers; slots [5, -1, 17, 0, 27], held heads [0, 2],
  capacity 8. It covers the 3 layouts x d in {8, 6} x {bf16, f16, f32, fp8 e4m3}. Each case holds
  the caches' raw bits and the rows. For bf16, the caches that a scatter of those rows writes
  into zeroed caches are also included, those that the pair scatter writes for the pairs
  PAIR_SLOTS / PAIR_ROWS below, and those that the range scatter writes for the written ranges
  RANGE_STARTS / RANGE_COUNTS (the slot scatter at the ranges' slots).
* reduce_sizes.npz: the ordered sum of core/tests/test_slot_kernel.py:40-55. Members 0..2 at
  sizes {16384, 3000, 2} come from torch.Generator().manual_seed(1000 * rank + n), summed in
  orders [0, 1, 2] and [2, 0, 1]. It also holds the order-sensitive case (big * 2^20,
  small * 2^-6, -big; seed 7) in orders [0, 1, 2] and [0, 2, 1].
* c1.json: config C1 (Qwen2.5-0.5B). That is 24 layers of
  [2, 2048, 16, 2, 64] bf16 N(0, 1) from torch.Generator().manual_seed(0), 128 blocks from
  numpy.random.default_rng(1).choice(2048, 128, replace=False), and heads [0, 1]. It holds the
  sha256 of the caches and of the gathered [24, 2, 2048, 2, 64] rows (24 MiB of rows would be
  too large to commit), and a few rows verbatim.

Run from the repository root: python -m tests.golden.make_fixtures
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import torch

import oracle
from tests.cases import BS, CAPACITY, HEADS, LAYOUTS, NB, SLOTS, caches, strides_of

HERE = Path(__file__).resolve().parent
DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32,
          "fp8": torch.float8_e4m3fn}
BITS = {1: (torch.uint8, np.uint8), 2: (torch.int16, np.uint16), 4: (torch.int32, np.uint32)}
# the pair scatter's case: (slot, staged row) pairs over the literal rows, with a padding slot, a
# row outside the capacity and one row written to two slots
PAIR_SLOTS = [27, 3, -1, 9, 5, 20]
PAIR_ROWS = [0, 4, 2, 9, 1, 4]
# the range scatter's case: written (start, count) ranges over the literal rows, not in slot order
# and with an empty one, 8 rows in all (the capacity)
RANGE_STARTS = [24, 2, 9, 0]
RANGE_COUNTS = [3, 0, 4, 1]


def range_slots() -> np.ndarray:
    return np.concatenate([np.arange(a, a + k, dtype=np.int64)
                           for a, k in zip(RANGE_STARTS, RANGE_COUNTS)])


def raw(t: torch.Tensor) -> np.ndarray:
    tb, nb = BITS[t.element_size()]
    return t.contiguous().view(tb).numpy().view(nb).copy()


def gather_literal() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {
        "pair_slots": np.array(PAIR_SLOTS, dtype=np.int64),
        "pair_rows_of": np.array(PAIR_ROWS, dtype=np.int64),
        "range_starts": np.array(RANGE_STARTS, dtype=np.int64),
        "range_counts": np.array(RANGE_COUNTS, dtype=np.int64),
        "slots": np.array(SLOTS, dtype=np.int64),
        "heads": np.array(HEADS, dtype=np.int64),
        "capacity": np.array(CAPACITY, dtype=np.int64),
        "block_size": np.array(BS, dtype=np.int64),
    }
    for layout in LAYOUTS:
        for d in (8, 6):
            for name, dt in DTYPES.items():
                key = f"{layout}_d{d}_{name}"
                layers = caches(layout, d, dt)
                e = layers[0].element_size()
                rows = oracle.gather_rows(layers, SLOTS, HEADS, CAPACITY, d, BS,
                                          strides_of(layers[0]), e)
                out[f"{key}_cache"] = np.stack([raw(t) for t in layers])
                out[f"{key}_rows"] = rows
                if name == "bf16":
                    zero = [torch.zeros_like(t) for t in layers]
                    oracle.scatter_rows(zero, SLOTS, HEADS, rows, CAPACITY, d, BS,
                                        strides_of(zero[0]), e)
                    out[f"{key}_scattered"] = np.stack([raw(t) for t in zero])
                    zero = [torch.zeros_like(t) for t in layers]
                    oracle.scatter_pairs(zero, PAIR_SLOTS, PAIR_ROWS, HEADS, rows, CAPACITY, d,
                                         BS, strides_of(zero[0]), e)
                    out[f"{key}_paired"] = np.stack([raw(t) for t in zero])
                    zero = [torch.zeros_like(t) for t in layers]
                    oracle.scatter_rows(zero, range_slots(), HEADS, rows, CAPACITY, d, BS,
                                        strides_of(zero[0]), e)
                    out[f"{key}_ranged"] = np.stack([raw(t) for t in zero])
    return out


def member_input(rank: int, n: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(1000 * rank + n)
    return torch.randn(n, generator=g).to(torch.bfloat16)


def reduce_sizes() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for n in (16384, 3000, 2):
        xs = [raw(member_input(r, n)) for r in range(3)]
        for r, x in enumerate(xs):
            out[f"n{n}_member{r}"] = x
        for order in ([0, 1, 2], [2, 0, 1]):
            out[f"n{n}_sum_{''.join(map(str, order))}"] = oracle.member_sum([xs[r] for r in order])
    g = torch.Generator().manual_seed(7)
    big = torch.randn(16384, generator=g) * 2.0**20
    small = torch.randn(16384, generator=g) * 2.0**-6
    xs = [raw(big.to(torch.bfloat16)), raw(small.to(torch.bfloat16)), raw((-big).to(torch.bfloat16))]
    for r, x in enumerate(xs):
        out[f"ordered_member{r}"] = x
    for order in ([0, 1, 2], [0, 2, 1]):
        out[f"ordered_sum_{''.join(map(str, order))}"] = oracle.member_sum([xs[r] for r in order])
    return out


C1 = {"layers": 24, "num_blocks": 2048, "block_size": 16, "kv_heads": 2, "head_dim": 64,
      "cache_seed": 0, "block_seed": 1, "blocks": 128, "heads": [0, 1]}


def c1_inputs():
    """The C1 caches (CPU, bf16), the slot ids and the heads, from the fixed seeds."""
    g = torch.Generator().manual_seed(C1["cache_seed"])
    shape = (2, C1["num_blocks"], C1["block_size"], C1["kv_heads"], C1["head_dim"])
    layers = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(C1["layers"])]
    blocks = np.random.default_rng(C1["block_seed"]).choice(C1["num_blocks"], C1["blocks"],
                                                            replace=False)
    slots = oracle.expand_blocks(blocks, C1["block_size"])
    return layers, slots, C1["heads"]


def digest(chunks) -> str:
    h = hashlib.sha256()
    for c in chunks:
        h.update(np.ascontiguousarray(c).tobytes())
    return h.hexdigest()


def c1() -> dict:
    layers, slots, heads = c1_inputs()
    n = len(slots)
    rows = oracle.gather_rows(layers, slots, heads, n, C1["head_dim"], C1["block_size"],
                              strides_of(layers[0]), 2)
    return {
        **C1,
        "slots": int(n),
        "cache_sha256": digest(raw(t) for t in layers),
        "rows_sha256": digest([rows]),
        "rows_shape": list(rows.shape),
        "sample": {"layer": 5, "head_index": 1, "first_rows": 4,
                   "bits": rows[5, 1, :4].reshape(-1).tolist()},
    }


def main() -> None:
    np.savez_compressed(HERE / "gather_literal.npz", **gather_literal())
    np.savez_compressed(HERE / "reduce_sizes.npz", **reduce_sizes())
    (HERE / "c1.json").write_text(json.dumps(c1(), indent=1) + "\n")
    for f in ("gather_literal.npz", "reduce_sizes.npz", "c1.json"):
        print(f, (HERE / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
