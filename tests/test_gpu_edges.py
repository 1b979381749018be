"""Edge cases of the HIP path on the GPU, each against the oracle.

* **Ragged counts.** Slot counts that do not fill the last tile, and capacities larger than the
  count. Rows past the count must be left as they were: the output is pre-filled with a
  sentinel, and the oracle gathers into the same pre-filled rows. This covers every layout, d in
  {8, 6}, padding ids, the block gather and the scatter.
* **Empty calls.** No slots, no heads or no layers: nothing is written, and nothing fails.
* **The widest head table.** 256 head slots in one call; 257 is refused.
* **The reduce's element path.** A member or the output not 16-byte aligned; lengths that are
  not a multiple of 8; no members listed; and a length of 0, which still reports completion.
* **fp8 e5m2** moves as raw bytes, like e4m3.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.kernels import REDUCE_STATE_WORDS, KernelError
from tests.cases import LAYOUTS, bits, caches, strides_of

pytestmark = pytest.mark.gpu

NB, BS, H, L = 80, 4, 3, 2
SENTINEL = 0x5A5A


def dev_long(xs):
    return torch.tensor([int(x) for x in xs], dtype=torch.long, device="cuda")


def ptrs(layers):
    return dev_long([t.data_ptr() for t in layers])


def ragged_slots(n: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    s = rng.choice(NB * BS, size=n, replace=False).astype(np.int64)
    s[rng.random(n) < 0.1] = -1  # padding ids
    return s.tolist()


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("n", [1, 7, 9, 63, 65, 257])
def test_ragged_counts_leave_the_rows_past_n_alone(ext, layout, d, n):
    layers = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=n)
    slots, heads, cap = ragged_slots(n, n), [2, 0], n + 5
    want = np.full((L, len(heads), cap, 2, d), SENTINEL, dtype=np.uint16)
    oracle.gather_rows(layers, slots, heads, cap, d, BS, strides_of(layers[0]), 2, out=want)
    gpu = [t.cuda() for t in layers]
    out = torch.full((L, len(heads), cap, 2, d), SENTINEL, dtype=torch.int16, device="cuda")
    ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long(heads), out.data_ptr(), cap, d, BS,
                    list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("blocks", [[3], [9, 0, 77], list(range(40, 57))])
def test_ragged_block_lists(ext, layout, blocks):
    d = 8
    layers = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=len(blocks))
    slots = oracle.expand_blocks(blocks, BS)
    cap = len(slots) + 3
    want = np.full((L, H, cap, 2, d), SENTINEL, dtype=np.uint16)
    oracle.gather_rows(layers, slots, list(range(H)), cap, d, BS, strides_of(layers[0]), 2,
                       out=want)
    gpu = [t.cuda() for t in layers]
    out = torch.full((L, H, cap, 2, d), SENTINEL, dtype=torch.int16, device="cuda")
    tags = torch.full((len(slots),), -9, dtype=torch.long, device="cuda")
    ext.gather_blocks(ptrs(gpu), torch.tensor(blocks, dtype=torch.int32, device="cuda"),
                      dev_long(range(H)), out.data_ptr(), cap, d, BS, list(strides_of(gpu[0])), 2,
                      slots_out=tags)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    assert tags.cpu().tolist() == slots.tolist()


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("n", [1, 9, 65])
def test_ragged_scatter_writes_only_the_listed_rows(ext, layout, n):
    d = 6
    src = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=100 + n)
    slots, heads, cap = ragged_slots(n, 100 + n), [1, 2], n + 2
    rows = oracle.gather_rows(src, slots, heads, cap, d, BS, strides_of(src[0]), 2)
    dst = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=200 + n)
    want = [t.clone() for t in dst]
    oracle.scatter_rows(want, slots, heads, rows, cap, d, BS, strides_of(want[0]), 2)
    gpu = [t.cuda() for t in dst]
    r = torch.from_numpy(rows.view(np.int16).copy()).cuda()
    ext.scatter_rows(ptrs(gpu), dev_long(slots), dev_long(heads), r.data_ptr(), cap, d, BS,
                     list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(bits(g), bits(w))


def test_empty_calls_write_nothing(ext):
    layers = [t.cuda() for t in caches("kv_first", 8, torch.bfloat16, n_layers=L, nb=NB, h=H)]
    out = torch.full((L, H, 4, 2, 8), SENTINEL, dtype=torch.int16, device="cuda")
    st = list(strides_of(layers[0]))
    s, h = dev_long([3, 5]), dev_long([0, 1, 2])
    ext.gather_rows(ptrs(layers), s[:0], h, out.data_ptr(), 4, 8, BS, st, 2)
    ext.gather_rows(ptrs(layers), s, h[:0], out.data_ptr(), 4, 8, BS, st, 2)
    ext.gather_rows(ptrs(layers)[:0], s, h, out.data_ptr(), 4, 8, BS, st, 2)
    ext.scatter_rows(ptrs(layers), s[:0], h, out.data_ptr(), 4, 8, BS, st, 2)
    ext.gather_blocks(ptrs(layers), torch.empty(0, dtype=torch.int32, device="cuda"), h,
                      out.data_ptr(), 4, 8, BS, st, 2)
    torch.cuda.synchronize()
    assert bool((out == SENTINEL).all())


def test_256_head_slots_in_one_call_and_257_refused(ext):
    d, nb, heads = 8, 6, 256
    g = torch.Generator().manual_seed(9)
    layers = [torch.randn((2, nb, BS, heads, d), generator=g).to(torch.bfloat16)]
    slots, order = [5, 0, 23, -1], list(range(heads))[::-1]
    want = oracle.gather_rows(layers, slots, order, 4, d, BS, strides_of(layers[0]), 2)
    gpu = [t.cuda() for t in layers]
    out = torch.zeros(want.shape, dtype=torch.int16, device="cuda")
    ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long(order), out.data_ptr(), 4, d, BS,
                    list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
    with pytest.raises(KernelError, match="head slots"):
        ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long(order + [0]), out.data_ptr(), 4,
                        d, BS, list(strides_of(gpu[0])), 2)
    # both scatters write the 256 head slots back: a pair tile spans them all in 16 passes, and
    # its head offsets past the first wave's 64 come from the fill loop
    r = torch.from_numpy(want.view(np.int16).copy()).cuda()
    for how in ("rows", "pairs"):
        dst = [torch.zeros_like(t) for t in gpu]
        ref = [torch.zeros_like(t) for t in layers]
        live = [s for s in slots if s >= 0]
        if how == "rows":
            ext.scatter_rows(ptrs(dst), dev_long(slots), dev_long(order), r.data_ptr(), 4, d, BS,
                             list(strides_of(dst[0])), 2)
            oracle.scatter_rows(ref, slots, order, want, 4, d, BS, strides_of(ref[0]), 2)
        else:
            ext.scatter_pairs(ptrs(dst), dev_long(slots[::-1]), dev_long([3, 2, 1, 0]),
                              dev_long(order), r.data_ptr(), 4, d, BS, list(strides_of(dst[0])), 2)
            oracle.scatter_pairs(ref, slots[::-1], [3, 2, 1, 0], order, want, 4, d, BS,
                                 strides_of(ref[0]), 2)
        torch.cuda.synchronize()
        assert live and all(np.array_equal(bits(a), bits(b)) for a, b in zip(dst, ref))


@pytest.mark.parametrize("heads,n", [([1], 1024), ([1], 1025), ([1], 4807), ([2, 0], 1031),
                                     ([2, 0], 4800)])
def test_gathers_of_one_head_group_over_whole_and_partial_xcd_runs(ext, heads, n):
    """A gather whose tiles cover every held head deals its tiles to the XCDs in runs (16 tiles
    an XCD, 128 a round); a grid of exactly one round, one round and a few tiles, and several
    rounds and a partial one, each byte against the oracle."""
    nb, bs, layers_n = 1250, 4, 2
    layers = caches("kv_first", 128, torch.bfloat16, n_layers=layers_n, nb=nb, bs=bs, h=H,
                    seed=n)
    slots = np.random.default_rng(n).choice(nb * bs, size=n, replace=False).astype(np.int64)
    cap = n + 3
    want = np.full((layers_n, len(heads), cap, 2, 128), SENTINEL, dtype=np.uint16)
    oracle.gather_rows(layers, slots.tolist(), heads, cap, 128, bs, strides_of(layers[0]), 2,
                       out=want)
    gpu = [t.cuda() for t in layers]
    out = torch.full(want.shape, SENTINEL, dtype=torch.int16, device="cuda")
    ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long(heads), out.data_ptr(), cap, 128, bs,
                    list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("d", [8, 6])
def test_the_gather_writes_straight_into_mapped_host_memory(ext, d):
    """Zero-copy, as the reference's staging does: out is host memory mapped for the device."""
    import ctypes

    layers = caches("kv_first", d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=44)
    slots, heads, cap = ragged_slots(61, 44), [1, 2], 64
    want = np.full((L, len(heads), cap, 2, d), SENTINEL, dtype=np.uint16)
    oracle.gather_rows(layers, slots, heads, cap, d, BS, strides_of(layers[0]), 2, out=want)
    gpu = [t.cuda() for t in layers]
    host, mapped = ext.host_alloc_mapped(want.nbytes)
    try:
        h = np.ctypeslib.as_array((ctypes.c_uint16 * want.size).from_address(host))
        h[:] = SENTINEL
        ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long(heads), mapped, cap, d, BS,
                        list(strides_of(gpu[0])), 2)
        torch.cuda.synchronize()
        assert np.array_equal(h.reshape(want.shape), want)
    finally:
        ext.host_free(host)


def test_fp8_e5m2_moves_as_raw_bytes(ext):
    layers = caches("blocks_first", 8, torch.float8_e5m2, n_layers=L, nb=NB, h=H, seed=4)
    slots = ragged_slots(33, 4)
    want = oracle.gather_rows(layers, slots, [0, 1, 2], 40, 8, BS, strides_of(layers[0]), 1)
    gpu = [t.cuda() for t in layers]
    out = torch.zeros(want.shape, dtype=torch.uint8, device="cuda")
    ext.gather_rows(ptrs(gpu), dev_long(slots), dev_long([0, 1, 2]), out.data_ptr(), 40, 8, BS,
                    list(strides_of(gpu[0])), 1)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


def member(rank: int, n: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(77 * rank + n)
    return torch.randn(n, generator=g).to(torch.bfloat16)


def reduce_call(ext, members, order, out):
    table = dev_long([m.data_ptr() for m in members] + [0] * (8 - len(members)))
    flags = torch.ones(8, dtype=torch.long, device="cuda")
    o = torch.tensor([len(order), *order] + [0] * (8 - len(order)), dtype=torch.int32,
                     device="cuda")
    state = torch.zeros(REDUCE_STATE_WORDS, dtype=torch.long, device="cuda")
    ext.local_reduce(table, flags, o, out, 1, 10**9, 0, state)
    torch.cuda.synchronize()
    assert int(state[0].item()) == 1 << 16
    assert not state[1:].any()


@pytest.mark.parametrize("n", [1, 7, 9, 1001])
@pytest.mark.parametrize("misaligned", ["member", "output", "none"])
def test_the_reduce_element_path_and_tails(ext, n, misaligned):
    xs = [member(r, n) for r in range(3)]
    members = []
    for r, x in enumerate(xs):
        if misaligned == "member" and r == 1:
            big = torch.empty(n + 1, dtype=torch.bfloat16, device="cuda")
            big[1:] = x.cuda()
            members.append(big[1:])  # 2-byte aligned, not 16
        else:
            members.append(x.cuda())
    if misaligned == "output":
        out = torch.empty(n + 1, dtype=torch.bfloat16, device="cuda")[1:]
    else:
        out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    order = [1, 2, 0]
    reduce_call(ext, members, order, out)
    assert np.array_equal(bits(out), oracle.member_sum([bits(xs[r]) for r in order]))


def test_the_reduce_of_no_members_is_zeros_and_of_no_elements_completes(ext):
    xs = [member(r, 4096).cuda() for r in range(2)]
    out = torch.full((4096,), 7.0, dtype=torch.bfloat16, device="cuda")
    reduce_call(ext, xs, [], out)
    assert not out.any()
    empty = torch.empty(0, dtype=torch.bfloat16, device="cuda")
    reduce_call(ext, [x[:0] for x in xs], [0, 1], empty)


def random_pairs(n: int, cap: int, seed: int):
    """n pairs over distinct slots, with padding slots, rows outside [0, cap) and rows named
    twice (one staged row written to two slots)."""
    rng = np.random.default_rng(seed)
    slots = rng.choice(NB * BS, size=n, replace=False).astype(np.int64)
    rows_of = rng.integers(0, cap, size=n).astype(np.int64)
    slots[rng.random(n) < 0.1] = -1
    bad = rng.random(n) < 0.1
    rows_of[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -3, cap + 2)
    return slots, rows_of


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("n", [1, 2, 3, 9, 65, 300])
def test_scatter_pairs_matches_the_oracle(ext, layout, d, n):
    src = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=300 + n)
    cap = max(4, n // 2)  # fewer staged rows than pairs: some rows go to several slots
    rows = oracle.gather_rows(src, ragged_slots(cap, n), [0, 1, 2], cap, d, BS,
                              strides_of(src[0]), 2)
    slots, rows_of = random_pairs(n, cap, n)
    dst = caches(layout, d, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=400 + n)
    heads = [2, 0, 1]
    want = [t.clone() for t in dst]
    oracle.scatter_pairs(want, slots, rows_of, heads, rows, cap, d, BS, strides_of(want[0]), 2)
    gpu = [t.cuda() for t in dst]
    r = torch.from_numpy(rows.view(np.int16).copy()).cuda()
    ext.scatter_pairs(ptrs(gpu), dev_long(slots), dev_long(rows_of), dev_long(heads), r.data_ptr(),
                      cap, d, BS, list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(bits(g), bits(w))


def test_scatter_pairs_in_destination_order_equals_the_scatter(ext):
    """A permuted block table restored through destination_order + scatter_pairs writes the same
    caches as scatter_rows in staged order."""
    from everserve_amd.state.restore import destination_order

    nb, h, d = 64, 4, 128
    g = torch.Generator().manual_seed(21)
    layers = [torch.zeros((2, nb, BS, h, d), dtype=torch.bfloat16).cuda() for _ in range(3)]
    blocks = np.random.default_rng(21).permutation(nb)[:48]
    slots = oracle.expand_blocks(blocks, BS)
    n = len(slots)
    rows = torch.randn((3, h, n, 2, d), generator=g).to(torch.bfloat16).cuda()
    heads = dev_long(range(h))
    st = list(strides_of(layers[0]))
    ext.scatter_rows(ptrs(layers), dev_long(slots), heads, rows.data_ptr(), n, d, BS, st, 2)
    torch.cuda.synchronize()
    want = [t.clone() for t in layers]
    for t in layers:
        t.zero_()
    sorted_slots, rows_of = destination_order(slots, block_size=BS)
    assert (np.diff(sorted_slots) > 0).all()
    ext.scatter_pairs(ptrs(layers), dev_long(sorted_slots), dev_long(rows_of), heads,
                      rows.data_ptr(), n, d, BS, st, 2)
    torch.cuda.synchronize()
    for a, b in zip(layers, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_scatter_pairs_fp8_and_empty(ext):
    layers = caches("blocks_first", 8, torch.float8_e5m2, n_layers=L, nb=NB, h=H, seed=5)
    cap = 40
    rows = oracle.gather_rows(layers, ragged_slots(cap, 5), [0, 1, 2], cap, 8, BS,
                              strides_of(layers[0]), 1)
    slots, rows_of = random_pairs(33, cap, 5)
    dst = [torch.zeros_like(t) for t in layers]
    want = [t.clone() for t in dst]
    oracle.scatter_pairs(want, slots, rows_of, [0, 1, 2], rows, cap, 8, BS, strides_of(want[0]), 1)
    gpu = [t.cuda() for t in dst]
    r = torch.from_numpy(rows.copy()).cuda()
    ext.scatter_pairs(ptrs(gpu), dev_long(slots), dev_long(rows_of), dev_long([0, 1, 2]),
                      r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 1)
    ext.scatter_pairs(ptrs(gpu), dev_long(slots)[:0], dev_long(rows_of)[:0], dev_long([0, 1, 2]),
                      r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 1)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(bits(g), bits(w))
    with pytest.raises(RuntimeError, match="slots but"):
        ext.scatter_pairs(ptrs(gpu), dev_long(slots), dev_long(rows_of[:-1]), dev_long([0]),
                          r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 1)


def test_scatter_ranges_at_a_restore_chunks_size_equals_the_slot_scatter(ext):
    """A restore's chunk as the Restorer launches it (one layer, 8 heads, 65,536 rows of a
    [2, 16384, 16, 8, 128] bf16 cache, 256 MiB): one range, then three (a gap, an empty range,
    the last slot of the cache reached), each equal to evs_scatter_rows at the same slots."""
    nb, bs, h, d, n = 16384, 16, 8, 128, 65536
    g = torch.Generator(device="cuda").manual_seed(31)
    rows = torch.randn((1, h, n, 2, d), generator=g, device="cuda").to(torch.bfloat16)
    heads = dev_long([3, 1, 0, 2, 7, 6, 5, 4])
    for starts, counts in (([100_000], [n]),
                           ([0, 70_000, nb * bs - 30_000], [35_536, 0, 30_000])):
        slots = np.concatenate([np.arange(a, a + k, dtype=np.int64) for a, k in zip(starts, counts)])
        assert len(slots) == n
        first_rows = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
        a = torch.zeros((2, nb, bs, h, d), dtype=torch.bfloat16, device="cuda")
        b = torch.zeros_like(a)
        st = list(strides_of(a))
        ext.scatter_ranges(ptrs([a]), dev_long(starts), dev_long(first_rows), n, heads,
                           rows.data_ptr(), n, d, bs, st, 2)
        ext.scatter_rows(ptrs([b]), dev_long(slots), heads, rows.data_ptr(), n, d, bs, st, 2)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), starts
        # and against the oracle on a sample of rows: the slot scatter is pinned to it elsewhere
        pick = np.sort(np.random.default_rng(31).choice(n, 64, replace=False))
        got = a[:, slots[pick] // bs, slots[pick] % bs].cpu()      # [2, 64, h, d]
        want = rows[0][:, pick].cpu()                              # [h, 64, 2, d] in head order
        order = heads.cpu().tolist()
        for i, hs in enumerate(order):
            assert torch.equal(got[:, :, hs].view(torch.int16),
                               want[i].permute(1, 0, 2).contiguous().view(torch.int16))
        del a, b


def test_scatter_ranges_over_several_layers_and_nothing_to_move(ext):
    """Three layers in one launch with ranges that do not ascend; then n = 0 moves nothing."""
    src = caches("blocks_first", 8, torch.bfloat16, n_layers=3, nb=NB, h=H, seed=33)
    cap = 40
    starts, counts = [200, 7, 300], [10, 20, 5]
    slots = np.concatenate([np.arange(a, a + k) for a, k in zip(starts, counts)])
    rows = oracle.gather_rows(src, slots, [0, 1, 2], cap, 8, BS, strides_of(src[0]), 2)
    dst = caches("blocks_first", 8, torch.bfloat16, n_layers=3, nb=NB, h=H, seed=34)
    want = [t.clone() for t in dst]
    oracle.scatter_rows(want, slots, [2, 0, 1], rows, cap, 8, BS, strides_of(want[0]), 2)
    gpu = [t.cuda() for t in dst]
    r = torch.from_numpy(rows.view(np.int16).copy()).cuda()
    first_rows = [0, 10, 30, 35]
    ext.scatter_ranges(ptrs(gpu), dev_long(starts), dev_long(first_rows), 35, dev_long([2, 0, 1]),
                       r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 2)
    ext.scatter_ranges(ptrs(gpu), dev_long(starts), dev_long(first_rows), 0, dev_long([2, 0, 1]),
                       r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(bits(g), bits(w))
    with pytest.raises(RuntimeError, match="first rows"):
        ext.scatter_ranges(ptrs(gpu), dev_long(starts), dev_long(first_rows[:-1]), 35,
                           dev_long([0]), r.data_ptr(), cap, 8, BS, list(strides_of(gpu[0])), 2)


def range_cases():
    """(name, starts, counts) over a 16,384-slot cache: more ranges than two levels of the
    kernel's 64-way search reach (4,096), runs of empty ranges longer than the 64 ranges a tile
    reads ahead (a row past them is found by bisection), empty ranges first, and 2 and 65 ranges."""
    rng = np.random.default_rng(71)
    out = []
    counts = rng.integers(0, 4, 5000)  # 5,000 ranges of 0-3 rows, gaps of 0-1 slots between
    gaps = rng.integers(0, 2, 5000)
    starts = np.cumsum(np.concatenate(([0], (counts + gaps)[:-1])))
    out.append(("5000 ranges", starts, counts))
    starts = [5, 40] + [100] * 300 + [200, 900] + [1000] * 70 + [3000]
    counts = [3, 50] + [0] * 300 + [1, 64] + [0] * 70 + [90]
    out.append(("runs of empty ranges", np.array(starts), np.array(counts)))
    starts = [7] * 10 + [50, 16000]
    counts = [0] * 10 + [30, 384]
    out.append(("empty ranges first", np.array(starts), np.array(counts)))
    out.append(("2 ranges", np.array([900, 10]), np.array([70, 5])))
    out.append(("65 ranges", np.arange(65) * 250, np.full(65, 3)))
    return out


@pytest.mark.parametrize("case", range(5))
def test_scatter_ranges_through_many_ranges_and_runs_of_empty_ones(ext, case):
    """Each row's range is found by the tile's first wave together (a 64-way search, then 64
    ranges read ahead); these cases reach every part of that: a third search level, rows past the
    64 ranges read ahead, leading empty ranges. Equal to the oracle's slot scatter at the
    expanded slots, 64-row tiles (bf16, d = 8)."""
    name, starts, counts = range_cases()[case]
    nb, bs, h, d = 1024, 16, 2, 8
    slots = np.concatenate([np.arange(a, a + k, dtype=np.int64) for a, k in zip(starts, counts)])
    assert slots.max() < nb * bs and len(slots) == len(np.unique(slots)), name
    n = len(slots)
    first_rows = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    src = caches("kv_first", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=72)
    rows = oracle.gather_rows(src, np.arange(n) % (nb * bs), [0, 1], n, d, bs,
                              strides_of(src[0]), 2)
    dst = caches("kv_first", d, torch.bfloat16, n_layers=2, nb=nb, bs=bs, h=h, seed=73)
    want = [t.clone() for t in dst]
    oracle.scatter_rows(want, slots, [1, 0], rows, n, d, bs, strides_of(want[0]), 2)
    gpu = [t.cuda() for t in dst]
    r = torch.from_numpy(rows.view(np.int16).copy()).cuda()
    ext.scatter_ranges(ptrs(gpu), dev_long(starts), dev_long(first_rows), n, dev_long([1, 0]),
                       r.data_ptr(), n, d, bs, list(strides_of(gpu[0])), 2)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(bits(g), bits(w)), name


@pytest.mark.parametrize("layout", LAYOUTS)
def test_a_bound_gather_writes_what_gather_rows_writes(ext, layout):
    """Kernels.bind_gather (the step path's launcher, its fixed arguments checked once) against
    gather_rows on the same caches, slots (padding included) and held heads; a layout of four
    strides is refused when binding."""
    src = [t.cuda() for t in caches(layout, 8, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=41)]
    slots = dev_long([5, -1, 17, 0, 27, 300, 31])
    heads = dev_long([2, 0])
    st = list(strides_of(src[0]))
    cap = 8
    a = torch.full((L, 2, cap, 2, 8), 7, dtype=torch.bfloat16, device="cuda")
    b = torch.full_like(a, 7)
    ext.gather_rows(ptrs(src), slots, heads, a.data_ptr(), cap, 8, BS, st, 2)
    launch = ext.bind_gather(ptrs(src), heads, 8, BS, st, 2)
    launch(slots.data_ptr(), slots.numel(), b.data_ptr(), cap,
           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(RuntimeError, match="five strides"):
        ext.bind_gather(ptrs(src), heads, 8, BS, st[:4], 2)
    with pytest.raises(KernelError, match="capacity"):
        launch(slots.data_ptr(), slots.numel(), b.data_ptr(), 4,
               torch.cuda.current_stream().cuda_stream)
