"""The HIP path against the committed golden fixtures (tests/golden/), with no oracle in the loop.

The fixtures hold the inputs and the expected bytes (tests/golden/make_fixtures.py):
* the gather and the scatter of the reference tests' literal case, in every layout, d in {8, 6},
  and bf16, f16, f32 and fp8, and the pair and range scatters of its rows;
* the ordered sums at the reference's sizes {16384, 3000, 2}, and the order-sensitive case, through
  evs_local_reduce;
* config C1 (Qwen2.5-0.5B shape), whose rows are checked against their
  sha256 through both gather_rows and gather_blocks.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from everserve_amd.kernels import REDUCE_STATE_WORDS
from tests.cases import strides_of
from tests.golden import make_fixtures as mf
from tests.test_golden import CASES, G, R, tensors

pytestmark = pytest.mark.gpu

C1 = json.loads((Path(__file__).resolve().parent / "golden" / "c1.json").read_text())


def dev_long(xs):
    return torch.tensor([int(x) for x in xs], dtype=torch.long, device="cuda")


@pytest.mark.parametrize("case", CASES)
def test_the_gather_writes_the_stored_rows(ext, case):
    layers = [t.cuda() for t in tensors(case)]
    want = G[f"{case}_rows"]
    d = int(case.rsplit("_", 2)[1][1:])
    e = layers[0].element_size()
    out = torch.zeros(want.size * e, dtype=torch.uint8, device="cuda")
    ext.gather_rows(dev_long([t.data_ptr() for t in layers]), dev_long(G["slots"]),
                    dev_long(G["heads"]), out.data_ptr(), int(G["capacity"]), d,
                    int(G["block_size"]), list(strides_of(layers[0])), e)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(want.dtype).reshape(want.shape), want)


@pytest.mark.parametrize("ordered", [None, True])
@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_scatter_writes_the_stored_caches(ext, case, ordered):
    """scatter_rows as it runs at these sizes (staged order), and with its pairs sorted by slot
    first, as it runs from 2^18 slots and 8 GiB."""
    layers = [torch.zeros_like(t).cuda() for t in tensors(case)]
    rows = torch.from_numpy(G[f"{case}_rows"].view(np.int16).copy()).cuda()
    d = int(case.rsplit("_", 2)[1][1:])
    ext.scatter_rows(dev_long([t.data_ptr() for t in layers]), dev_long(G["slots"]),
                     dev_long(G["heads"]), rows.data_ptr(), int(G["capacity"]), d,
                     int(G["block_size"]), list(strides_of(layers[0])), 2, ordered=ordered)
    torch.cuda.synchronize()
    got = np.stack([mf.raw(t.cpu()) for t in layers])
    assert np.array_equal(got, G[f"{case}_scattered"])


@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_pair_scatter_writes_the_stored_caches(ext, case):
    layers = [torch.zeros_like(t).cuda() for t in tensors(case)]
    rows = torch.from_numpy(G[f"{case}_rows"].view(np.int16).copy()).cuda()
    d = int(case.rsplit("_", 2)[1][1:])
    ext.scatter_pairs(dev_long([t.data_ptr() for t in layers]), dev_long(G["pair_slots"]),
                      dev_long(G["pair_rows_of"]), dev_long(G["heads"]), rows.data_ptr(),
                      int(G["capacity"]), d, int(G["block_size"]), list(strides_of(layers[0])), 2)
    torch.cuda.synchronize()
    got = np.stack([mf.raw(t.cpu()) for t in layers])
    assert np.array_equal(got, G[f"{case}_paired"])


@pytest.mark.parametrize("case", [c for c in CASES if c.endswith("bf16")])
def test_the_range_scatter_writes_the_stored_caches(ext, case):
    layers = [torch.zeros_like(t).cuda() for t in tensors(case)]
    rows = torch.from_numpy(G[f"{case}_rows"].view(np.int16).copy()).cuda()
    d = int(case.rsplit("_", 2)[1][1:])
    counts = G["range_counts"]
    first_rows = np.concatenate(([0], np.cumsum(counts)))
    ext.scatter_ranges(dev_long([t.data_ptr() for t in layers]), dev_long(G["range_starts"]),
                       dev_long(first_rows), int(first_rows[-1]), dev_long(G["heads"]),
                       rows.data_ptr(), int(G["capacity"]), d, int(G["block_size"]),
                       list(strides_of(layers[0])), 2)
    torch.cuda.synchronize()
    got = np.stack([mf.raw(t.cpu()) for t in layers])
    assert np.array_equal(got, G[f"{case}_ranged"])


def reduce(ext, members, order):
    bufs = [torch.from_numpy(m.view(np.int16).copy()).cuda().view(torch.bfloat16) for m in members]
    table = dev_long([b.data_ptr() for b in bufs] + [0] * (8 - len(bufs)))
    flags = torch.ones(8, dtype=torch.long, device="cuda")
    o = torch.tensor([len(order), *order] + [0] * (8 - len(order)), dtype=torch.int32,
                     device="cuda")
    out = torch.empty_like(bufs[0])
    state = torch.zeros(REDUCE_STATE_WORDS, dtype=torch.long, device="cuda")
    ext.local_reduce(table, flags, o, out, 1, 10**9, 0, state)
    torch.cuda.synchronize()
    assert int(state[0].item()) == 1 << 16
    return out.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("n", [16384, 3000, 2])
def test_the_local_reduce_writes_the_stored_sums(ext, n):
    xs = [R[f"n{n}_member{r}"] for r in range(3)]
    for order in ("012", "201"):
        assert np.array_equal(reduce(ext, xs, [int(c) for c in order]), R[f"n{n}_sum_{order}"])


def test_the_local_reduce_keeps_the_order_of_the_stored_case(ext):
    xs = [R[f"ordered_member{r}"] for r in range(3)]
    assert np.array_equal(reduce(ext, xs, [0, 1, 2]), R["ordered_sum_012"])
    assert np.array_equal(reduce(ext, xs, [0, 2, 1]), R["ordered_sum_021"])


def test_c1_rows_match_the_digest_by_slots_and_by_blocks(ext):
    layers, slots, heads = mf.c1_inputs()
    gpu = [t.cuda() for t in layers]
    n, d, bs = len(slots), C1["head_dim"], C1["block_size"]
    ptrs = dev_long([t.data_ptr() for t in gpu])
    shape = C1["rows_shape"]
    out = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
    ext.gather_rows(ptrs, dev_long(slots), dev_long(heads), out.data_ptr(), n, d, bs,
                    list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    assert mf.digest([mf.raw(out.cpu())]) == C1["rows_sha256"]
    blocks = torch.tensor(slots[::bs] // bs, dtype=torch.int32, device="cuda")
    out2 = torch.empty_like(out)
    tags = torch.empty(n, dtype=torch.long, device="cuda")
    ext.gather_blocks(ptrs, blocks, dev_long(heads), out2.data_ptr(), n, d, bs,
                      list(strides_of(gpu[0])), 2, slots_out=tags)
    torch.cuda.synchronize()
    assert mf.digest([mf.raw(out2.cpu())]) == C1["rows_sha256"]
    assert tags.cpu().numpy().tolist() == [int(s) for s in slots]
