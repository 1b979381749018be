"""The device-side ordering of a restore's pairs (evs_order_pairs) against the host's.

``Kernels.order_pairs`` must give what ``destination_order`` gives on the host, once the padding
slots the device keeps are set aside: the same slots in the same order, and the same staged row
for each, ties in listed order. Then ordering on the device and scattering the pairs must write
the same caches as the scatter in staged order.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state.restore import destination_order
from tests.cases import strides_of

pytestmark = pytest.mark.gpu


def on_device(ext, slots, num_slots):
    s, r = ext.order_pairs(torch.from_numpy(np.asarray(slots, dtype=np.int64)).cuda(), num_slots)
    torch.cuda.synchronize()
    return s.cpu().numpy(), r.cpu().numpy()


@pytest.mark.parametrize("n,num_slots", [(1, 1), (2, 5), (777, 10_000), (65_536, 1 << 20)])
def test_the_device_order_is_the_host_order(ext, n, num_slots):
    rng = np.random.default_rng(n)
    slots = rng.choice(num_slots, size=n, replace=False).astype(np.int64)
    slots[rng.random(n) < 0.1] = -1
    got_s, got_r = on_device(ext, slots, num_slots)
    assert sorted(got_r.tolist()) == list(range(n))  # a permutation of the staged rows
    assert np.array_equal(got_s, slots[got_r])
    keep = got_s >= 0
    want_s, want_r = destination_order(slots)
    assert np.array_equal(got_s[keep], want_s) and np.array_equal(got_r[keep], want_r)


def test_ties_keep_their_listed_order(ext):
    slots = np.array([7, 3, 7, 3, 0, 7], dtype=np.int64)
    got_s, got_r = on_device(ext, slots, 8)
    assert got_s.tolist() == [0, 3, 3, 7, 7, 7]
    assert got_r.tolist() == [4, 1, 3, 0, 2, 5]


def test_nothing_to_order(ext):
    got_s, got_r = on_device(ext, [], 16)
    assert got_s.size == 0 and got_r.size == 0


def test_the_c4_block_permutation_orders_like_the_host(ext):
    nb, bs = 16384, 16
    blocks = np.random.default_rng(4).permutation(nb)
    slots = (blocks[:, None] * bs + np.arange(bs)).reshape(-1)
    got_s, got_r = on_device(ext, slots, nb * bs)
    want_s, want_r = destination_order(slots, block_size=bs)
    assert np.array_equal(got_s, want_s) and np.array_equal(got_r, want_r)


def test_ordered_on_the_device_then_scattered_equals_the_scatter(ext):
    nb, bs, h, d, L = 64, 4, 3, 8, 2
    g = torch.Generator().manual_seed(31)
    blocks = np.random.default_rng(31).permutation(nb)[:40]
    slots = oracle.expand_blocks(blocks, bs)
    slots[5] = -1  # one padding slot
    n = len(slots)
    rows = torch.randn((L, h, n, 2, d), generator=g).to(torch.bfloat16).cuda()
    layers = [torch.zeros((2, nb, bs, h, d), dtype=torch.bfloat16).cuda() for _ in range(L)]
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device="cuda")
    heads = torch.arange(h, dtype=torch.long, device="cuda")
    st = list(strides_of(layers[0]))
    s_dev = torch.from_numpy(slots).cuda()
    ext.scatter_rows(ptrs, s_dev, heads, rows.data_ptr(), n, d, bs, st, 2)
    torch.cuda.synchronize()
    want = [t.clone() for t in layers]
    for t in layers:
        t.zero_()
    o_slots, o_rows = ext.order_pairs(s_dev, nb * bs)
    ext.scatter_pairs(ptrs, o_slots, o_rows, heads, rows.data_ptr(), n, d, bs, st, 2)
    torch.cuda.synchronize()
    for a, b in zip(layers, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_repeated_orderings_into_given_outputs_allocate_nothing(ext):
    """The workspace is the shim's, kept per device and stream; with outputs given, a second and
    third call (the third smaller) allocate no device memory and equal a fresh call's result."""
    rng = np.random.default_rng(5)
    big = torch.from_numpy(rng.permutation(1 << 16).astype(np.int64)).cuda()
    small = big[:1000].clone()
    outs = {n: (torch.empty(n, dtype=torch.long, device="cuda"),
                torch.empty(n, dtype=torch.long, device="cuda")) for n in (1 << 16, 1000)}
    ext.order_pairs(big, 1 << 16, out=outs[1 << 16])  # sizes the workspace
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    for x in (big, small):
        got = ext.order_pairs(x, 1 << 16, out=outs[x.numel()])
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        want = ext.order_pairs(x.clone(), 1 << 16)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        before = torch.cuda.memory_allocated()
    with pytest.raises(RuntimeError, match="holds"):
        ext.order_pairs(small, 1 << 16, out=outs[1 << 16])
