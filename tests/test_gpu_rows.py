"""The HIP gather, block gather and scatter against the oracle, byte for byte, on the GPU.

Every layout, the 16-byte and the per-element path, four element types (bf16, f16, f32 and fp8
e4m3 as raw bytes), a padding slot, a held-head subset, a strided view (the reference's cases,
core/tests/test_gather_kernel.py:67-102); then the configs' shapes: the Llama-3-8B gather (C2) at a
layer subset checked against the oracle and at full size checked by round trip, the fp8 70B share
(C3) with its D2H copy, and the restore scatter (C4) round trip.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state.restore import destination_order
from tests.cases import (CAPACITY, DTYPES, HEADS, LAYOUTS, SLOTS, bits, caches,
                         fp8_scaled_layers, strides_of)

pytestmark = pytest.mark.gpu


def ptrs(layers):
    return torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device="cuda")


def run_gather(ext, layers_gpu, slots, heads, capacity, out):
    layout, _, bs, d = oracle.recognise(layers_gpu[0].shape)
    ext.gather_rows(ptrs(layers_gpu), torch.tensor(slots, dtype=torch.long, device="cuda"),
                    torch.tensor(heads, dtype=torch.long, device="cuda"), out.data_ptr(),
                    capacity, d, bs, list(strides_of(layers_gpu[0])), layers_gpu[0].element_size())


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("dtype", DTYPES)
def test_gather_writes_exactly_what_the_oracle_gathers(ext, layout, d, dtype):
    layers = caches(layout, d, dtype)
    _, _, bs, _ = oracle.recognise(layers[0].shape)
    e = layers[0].element_size()
    want = oracle.gather_rows(layers, SLOTS, HEADS, CAPACITY, d, bs, strides_of(layers[0]), e)
    gpu = [t.cuda() for t in layers]
    out = torch.zeros(want.shape, dtype=dtype, device="cuda")
    run_gather(ext, gpu, SLOTS, HEADS, CAPACITY, out)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), want)


def test_a_strided_cache_view_is_read_through_its_strides(ext):
    big = caches("kv_first", 8, torch.bfloat16)
    layers = [t[:, :, :, 1:] for t in big]
    want = oracle.gather_rows(layers, SLOTS, [0, 1], CAPACITY, 8, 4, strides_of(layers[0]), 2)
    gpu = [t.cuda()[:, :, :, 1:] for t in big]
    out = torch.zeros(want.shape, dtype=torch.bfloat16, device="cuda")
    run_gather(ext, gpu, SLOTS, [0, 1], CAPACITY, out)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), want)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
def test_block_gather_equals_the_gather_of_the_expanded_slots(ext, layout, d):
    layers = caches(layout, d, torch.bfloat16, nb=9, seed=11)
    _, _, bs, _ = oracle.recognise(layers[0].shape)
    blocks = [4, 0, 7, 2]
    slots = oracle.expand_blocks(blocks, bs)
    want = oracle.gather_rows(layers, slots, HEADS, 20, d, bs, strides_of(layers[0]), 2)
    gpu = [t.cuda() for t in layers]
    out = torch.zeros(want.shape, dtype=torch.bfloat16, device="cuda")
    tags = torch.full((len(slots),), -7, dtype=torch.long, device="cuda")
    ext.gather_blocks(ptrs(gpu), torch.tensor(blocks, dtype=torch.int32, device="cuda"),
                      torch.tensor(HEADS, dtype=torch.long, device="cuda"), out.data_ptr(), 20, d,
                      bs, list(strides_of(gpu[0])), 2, slots_out=tags)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), want)
    assert tags.cpu().tolist() == slots.tolist()


@pytest.mark.parametrize("ordered", [None, True])
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_scatter_writes_exactly_what_the_oracle_writes(ext, ordered, layout, d, dtype):
    """As scatter_rows runs at this size (staged order), and with its pairs sorted by slot first
    (order_pairs, then scatter_pairs), as it runs from 2^18 slots and 8 GiB."""
    src = caches(layout, d, dtype, seed=5)
    dst = caches(layout, d, dtype, seed=9)  # a cache that already holds other rows
    _, _, bs, _ = oracle.recognise(src[0].shape)
    e = src[0].element_size()
    staged = oracle.gather_rows(src, SLOTS, HEADS, CAPACITY, d, bs, strides_of(src[0]), e)
    target = [2, 0]  # the head slots the rows go to here (of the cache's three)
    gpu_dst = [t.cuda() for t in dst]
    oracle.scatter_rows(dst, SLOTS, target, staged, CAPACITY, d, bs, strides_of(dst[0]), e)
    rows = torch.from_numpy(staged.copy()).cuda()
    ext.scatter_rows(ptrs(gpu_dst), torch.tensor(SLOTS, dtype=torch.long, device="cuda"),
                     torch.tensor(target, dtype=torch.long, device="cuda"), rows.data_ptr(),
                     CAPACITY, d, bs, list(strides_of(gpu_dst[0])), e, ordered=ordered)
    torch.cuda.synchronize()
    for got, want in zip(gpu_dst, dst):
        assert np.array_equal(bits(got), bits(want))


def test_rejections_raise_not_launch(ext):
    from everserve_amd.kernels import KernelError

    layers = [t.cuda() for t in caches("kv_first", 8, torch.bfloat16)]
    out = torch.zeros(1, device="cuda")
    s = torch.tensor(SLOTS, dtype=torch.long, device="cuda")
    h = torch.tensor(HEADS, dtype=torch.long, device="cuda")
    st = list(strides_of(layers[0]))
    with pytest.raises(KernelError, match="capacity"):
        ext.gather_rows(ptrs(layers), s, h, out.data_ptr(), 2, 8, 4, st, 2)
    with pytest.raises(KernelError, match="element size"):
        ext.gather_rows(ptrs(layers), s, h, out.data_ptr(), 8, 8, 4, st, 3)
    with pytest.raises(RuntimeError, match="five strides"):
        ext.gather_rows(ptrs(layers), s, h, out.data_ptr(), 8, 8, 4, st[:4], 2)
    with pytest.raises(RuntimeError, match="device"):
        ext.gather_rows(ptrs(layers), s.cpu(), h, out.data_ptr(), 8, 8, 4, st, 2)
    # nothing to move: returns without launching
    ext.gather_rows(ptrs(layers), s[:0], h, out.data_ptr(), 8, 8, 4, st, 2)
    # the ordered scatter refuses what the staged one does, before it sorts anything
    for ordered in (False, True):
        with pytest.raises(KernelError, match="capacity"):
            ext.scatter_rows(ptrs(layers), s, h, out.data_ptr(), 2, 8, 4, st, 2, ordered=ordered)
        with pytest.raises(KernelError, match="element size"):
            ext.scatter_rows(ptrs(layers), s, h, out.data_ptr(), 8, 8, 4, st, 3, ordered=ordered)


def test_a_captured_gather_replays_like_an_eager_call(ext):
    """The gather records no memset: a HIP graph of it replays right each time, eager work and
    synchronisations between the replays, the slot ids changed in place between replays."""
    layers = caches("kv_first", 8, torch.bfloat16, seed=21)
    gpu = [t.cuda() for t in layers]
    s = torch.tensor(SLOTS, dtype=torch.long, device="cuda")
    h = torch.tensor(HEADS, dtype=torch.long, device="cuda")
    out = torch.zeros((len(layers), len(HEADS), CAPACITY, 2, 8), dtype=torch.bfloat16, device="cuda")
    table = ptrs(gpu)  # made before the capture: a capture records no host-to-device copy
    strides = list(strides_of(gpu[0]))
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        ext.gather_rows(table, s, h, out.data_ptr(), CAPACITY, 8, 4, strides, 2)
    for i, slots in enumerate([SLOTS, [27, 3, -1, 9, 0], SLOTS[::-1]]):
        s.copy_(torch.tensor(slots))
        out.fill_(i)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = oracle.gather_rows(layers, slots, HEADS, CAPACITY, 8, 4, strides_of(layers[0]), 2,
                                  out=np.full((len(layers), len(HEADS), CAPACITY, 2, 8),
                                              bits(torch.full((1,), float(i), dtype=torch.bfloat16))[0],
                                              dtype=np.uint16))
        assert np.array_equal(bits(out), want), i


def test_a_captured_scatter_writes_in_staged_order_and_replays_right(ext):
    """Under graph capture scatter_rows does not sort (the sort clears its counters with a memset,
    which a captured graph must not hold), and asked to sort it refuses: the graph holds the
    staged order's one kernel, and each replay writes what the oracle writes, the slot ids changed
    in place between replays and the cache reset by eager work."""
    src = caches("kv_first", 8, torch.bfloat16, seed=5)
    base = caches("kv_first", 8, torch.bfloat16, seed=9)
    staged = oracle.gather_rows(src, SLOTS, HEADS, CAPACITY, 8, 4, strides_of(src[0]), 2)
    rows = torch.from_numpy(staged.copy()).cuda()
    gpu = [t.cuda() for t in base]
    table = ptrs(gpu)
    s = torch.tensor(SLOTS, dtype=torch.long, device="cuda")
    h = torch.tensor([2, 0], dtype=torch.long, device="cuda")
    strides = list(strides_of(gpu[0]))
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        ext.scatter_rows(table, s, h, rows.data_ptr(), CAPACITY, 8, 4, strides, 2)
        with pytest.raises(RuntimeError, match="captured"):
            ext.scatter_rows(table, s, h, rows.data_ptr(), CAPACITY, 8, 4, strides, 2,
                             ordered=True)
    for i, slots in enumerate([SLOTS, [27, 3, -1, 9, 0], SLOTS[::-1]]):
        s.copy_(torch.tensor(slots))
        for g, b in zip(gpu, base):
            g.copy_(b)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = [t.clone() for t in base]
        oracle.scatter_rows(want, slots, [2, 0], staged, CAPACITY, 8, 4, strides_of(base[0]), 2)
        for got, w in zip(gpu, want):
            assert np.array_equal(bits(got), bits(w)), i


def test_sorted_calls_on_two_streams_keep_their_own_pairs(ext):
    """Two sorting scatters enqueued back to back on two streams, with no synchronisation between
    them: each stream's sort writes its own workspace and pairs, so neither reads the other's.
    Each cache ends as the oracle writes it."""
    L, NB, BS, H, D = 4, 256, 16, 4, 64
    rng = np.random.default_rng(61)
    shape = (2, NB, BS, H, D)
    jobs = []
    for k, n in enumerate((1024, 4096)):
        slots = rng.permutation(NB * BS)[:n].astype(np.int64)
        slots[rng.integers(0, n, 8)] = -1  # padding, skipped by either order
        staged = torch.randn((L, H, n, 2, D), generator=torch.Generator().manual_seed(70 + k))
        staged = staged.to(torch.bfloat16)
        base = [torch.randn(shape, generator=torch.Generator().manual_seed(80 + 10 * k + i))
                .to(torch.bfloat16) for i in range(L)]
        jobs.append((slots, staged, base, [t.cuda() for t in base]))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    keep = []
    for (slots, staged, _, gpu), stream in zip(jobs, streams):
        with torch.cuda.stream(stream):
            s = torch.from_numpy(slots).cuda()
            rows = staged.cuda()
            h = torch.arange(H, dtype=torch.long, device="cuda")
            table = ptrs(gpu)
            keep += [s, rows, h, table]
            ext.scatter_rows(table, s, h, rows.data_ptr(), len(slots), D, BS,
                             list(strides_of(gpu[0])), 2, ordered=True)
    torch.cuda.synchronize()
    for slots, staged, base, gpu in jobs:
        want = [t.clone() for t in base]
        oracle.scatter_rows(want, slots, list(range(H)), bits(staged), len(slots), D, BS,
                            strides_of(base[0]), 2)
        for got, w in zip(gpu, want):
            assert np.array_equal(bits(got), bits(w))


# ----------------------------------------------------------------- the configs' shapes
def block_table(num_blocks_cache, num_blocks, bs, seed):
    blocks = np.random.default_rng(seed).permutation(num_blocks_cache)[:num_blocks]
    return blocks, oracle.expand_blocks(blocks, bs)


def gpu_caches(n_layers, shape, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = []
    for _ in range(n_layers):
        if dtype == torch.float8_e4m3fn:
            out.append(torch.randn(shape, generator=g, device="cuda", dtype=torch.float16)
                       .clamp_(-448, 448).to(dtype))
        else:
            out.append(torch.empty(shape, dtype=dtype, device="cuda").normal_(generator=g))
    return out


def test_c2_llama3_8b_gather_matches_the_oracle_on_two_layers(ext):
    """C2's per-layer shape, two layers, every slot of the 1024 blocks checked on the CPU."""
    L, NB, BS, H, D = 2, 8192, 16, 8, 128
    layers = gpu_caches(L, (2, NB, BS, H, D), torch.bfloat16, seed=0)
    _, slots = block_table(NB, 1024, BS, seed=2)
    n = len(slots)
    out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device="cuda")
    ext.gather_rows(ptrs(layers), torch.from_numpy(slots).cuda(),
                    torch.arange(H, dtype=torch.long, device="cuda"), out.data_ptr(), n, D, BS,
                    list(strides_of(layers[0])), 2)
    torch.cuda.synchronize()
    cpu = [t.cpu() for t in layers]
    want = oracle.gather_rows(cpu, slots, list(range(H)), n, D, BS, strides_of(cpu[0]), 2)
    assert np.array_equal(bits(out), want)


def test_c2_full_size_round_trip(ext):
    """All 32 layers (16 GiB of cache): gather the 1024 blocks, scatter them into a zeroed cache,
    and the restored blocks equal the originals on every layer; nothing else was written."""
    L, NB, BS, H, D = 32, 8192, 16, 8, 128
    layers = gpu_caches(L, (2, NB, BS, H, D), torch.bfloat16, seed=0)
    blocks, slots = block_table(NB, 1024, BS, seed=2)
    n = len(slots)
    s = torch.from_numpy(slots).cuda()
    heads = torch.arange(H, dtype=torch.long, device="cuda")
    strides = list(strides_of(layers[0]))
    out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device="cuda")
    ext.gather_rows(ptrs(layers), s, heads, out.data_ptr(), n, D, BS, strides, 2)
    fresh = [torch.zeros_like(t) for t in layers[:4]]
    ext.scatter_rows(ptrs(fresh), s, heads, out.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    b = torch.from_numpy(blocks).cuda()
    for orig, back in zip(layers, fresh):
        assert torch.equal(orig[:, b].view(torch.int16), back[:, b].view(torch.int16))
        keep = torch.ones(NB, dtype=torch.bool, device="cuda")
        keep[b] = False
        assert not back[:, keep].view(torch.int16).any()
    # the other 28 layers' rows against the cache, on the device: row t of head h is block
    # slots[t] // 16, offset slots[t] % 16 of that head
    bi, oi = s // BS, s % BS
    for li in range(4, L):
        want = layers[li][:, bi, oi].permute(2, 1, 0, 3)  # [H, n, 2, D]
        assert torch.equal(out[li].view(torch.int16), want.view(torch.int16)), li


@pytest.mark.parametrize("layout", ["blocks_first", "combined"])
def test_c2_shape_round_trip_in_the_other_layouts(ext, layout):
    """The C2 per-layer shape in the other two paged layouts, four layers (512 MiB each): the
    gathered rows equal the layout's torch indexing (the reference's rows_of_heads, restated in
    oracle.cpu_path and run on the device), and scattered into zeroed caches they restore exactly
    the gathered blocks, nothing else."""
    from oracle import cpu_path

    L, NB, BS, H, D = 4, 8192, 16, 8, 128
    shape = {"blocks_first": (NB, 2, BS, H, D), "combined": (NB, H, BS, 2 * D)}[layout]
    g = torch.Generator(device="cuda").manual_seed(5)
    layers = [torch.empty(shape, dtype=torch.bfloat16, device="cuda").normal_(generator=g)
              for _ in range(L)]
    blocks, slots = block_table(NB, 1024, BS, seed=2)
    n = len(slots)
    s = torch.from_numpy(slots).cuda()
    heads = torch.arange(H, dtype=torch.long, device="cuda")
    strides = list(strides_of(layers[0]))
    out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device="cuda")
    ext.gather_rows(ptrs(layers), s, heads, out.data_ptr(), n, D, BS, strides, 2)
    fresh = [torch.zeros_like(t) for t in layers]
    ext.scatter_rows(ptrs(fresh), s, heads, out.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    b = torch.from_numpy(blocks).cuda()
    keep = torch.ones(NB, dtype=torch.bool, device="cuda")
    keep[b] = False
    for li, (orig, back) in enumerate(zip(layers, fresh)):
        want = cpu_path.rows_of_heads(orig, s, heads)  # [H, n, 2, D]
        assert torch.equal(out[li].view(torch.int16), want.contiguous().view(torch.int16)), li
        assert torch.equal(orig[b].view(torch.int16), back[b].view(torch.int16)), li
        assert not back[keep].view(torch.int16).any(), li


def test_c3_fp8_share_gather_and_copy_to_pinned_memory(ext):
    """C3: 80 layers of a one-head fp8 e4m3 cache holding fp8(N(0,1) / s_l) with per-layer scales
    s_l ~ U(0.01, 0.1), and every byte code in layer 0's first block; 2048 blocks gathered and
    copied to pinned host memory. The bytes equal the oracle's on a layer subset and the device
    staging on all."""
    L, NB, BS, H, D = 80, 8192, 16, 1, 128
    layers, _ = fp8_scaled_layers(L, (2, NB, BS, H, D), seed=3)
    blocks, _ = block_table(NB, 2048, BS, seed=3)
    if 0 not in blocks:
        blocks[-1] = 0  # the block holding every byte code, NaN and saturation codes among them
    slots = oracle.expand_blocks(blocks, BS)
    n = len(slots)
    staging = torch.empty((L, H, n, 2, D), dtype=torch.uint8, device="cuda")
    host = torch.zeros((L, H, n, 2, D), dtype=torch.uint8, pin_memory=True)
    ext.gather_rows(ptrs(layers), torch.from_numpy(slots).cuda(),
                    torch.zeros(H, dtype=torch.long, device="cuda"), staging.data_ptr(), n, D, BS,
                    list(strides_of(layers[0])), 1)
    ext.copy_rows_async(host.data_ptr(), staging.data_ptr(), L * H, n * 2 * D, n * 2 * D)
    torch.cuda.synchronize()
    assert torch.equal(host, staging.cpu())
    sub = [layers[i].cpu() for i in (0, 41, 79)]
    want = oracle.gather_rows(sub, slots, [0], n, D, BS, strides_of(sub[0]), 1)
    assert np.array_equal(host[[0, 41, 79]].numpy(), want)


def test_copy_rows_moves_only_the_filled_rows(ext):
    """A staging buffer of capacity 8 holding 5 rows per (layer, head): the 2-D copy moves the
    5 rows of each run and leaves the host's other rows alone."""
    L, H, cap, n, row = 3, 2, 8, 5, 32
    dev = torch.arange(L * H * cap * row, dtype=torch.int32, device="cuda").view(torch.uint8)
    host = torch.full((L * H * cap * row * 4,), 0xAB, dtype=torch.uint8, pin_memory=True)
    ext.copy_rows_async(host.data_ptr(), dev.data_ptr(), L * H, n * row * 4, cap * row * 4)
    torch.cuda.synchronize()
    d = dev.cpu().view(L * H, cap * row * 4)
    h = host.view(L * H, cap * row * 4)
    assert torch.equal(h[:, : n * row * 4], d[:, : n * row * 4])
    assert (h[:, n * row * 4:] == 0xAB).all()


def test_c4_restore_round_trip_full_size(ext):
    """C4: 64 seqs x 4096 tokens of Llama-3-8B rows (32 GiB) scattered into a fresh
    16384-block cache through a seeded random-permutation block table, gathered back: equal,
    three ways: scatter_rows as it chooses (at this size it sorts its pairs on the device
    first), scatter_rows in staged order, and scatter_pairs with the pairs sorted on the host."""
    L, NB, BS, H, D = 32, 16384, 16, 8, 128
    n = NB * BS
    rows = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device="cuda")
    rows.normal_(generator=torch.Generator(device="cuda").manual_seed(4))
    cache = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device="cuda") for _ in range(L)]
    _, slots = block_table(NB, NB, BS, seed=4)
    s = torch.from_numpy(slots).cuda()
    heads = torch.arange(H, dtype=torch.long, device="cuda")
    strides = list(strides_of(cache[0]))
    back = torch.empty((8, H, n, 2, D), dtype=torch.bfloat16, device="cuda")
    # each into zeroed caches; the host's order is destination_order's, from the block table
    sorted_slots, rows_of = destination_order(slots, block_size=BS)
    for how in ("as built", "staged order", "cache order"):
        for t in cache:
            t.zero_()
        if how == "as built":
            ext.scatter_rows(ptrs(cache), s, heads, rows.data_ptr(), n, D, BS, strides, 2)
        elif how == "staged order":
            ext.scatter_rows(ptrs(cache), s, heads, rows.data_ptr(), n, D, BS, strides, 2,
                             ordered=False)
        else:
            ext.scatter_pairs(ptrs(cache), torch.from_numpy(sorted_slots).cuda(),
                              torch.from_numpy(rows_of).cuda(), heads, rows.data_ptr(), n, D, BS,
                              strides, 2)
        for first in range(0, L, 8):
            ext.gather_rows(ptrs(cache[first:first + 8]), s, heads, back.data_ptr(), n, D, BS,
                            strides, 2)
            torch.cuda.synchronize()
            assert torch.equal(back.view(torch.int16),
                               rows[first:first + 8].view(torch.int16)), (how, first)
