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
from tests.cases import (CAPACITY, DTYPES, HEADS, LAYOUTS, SLOTS, bits, caches, strides_of)

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


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_scatter_writes_exactly_what_the_oracle_writes(ext, layout, d, dtype):
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
                     CAPACITY, d, bs, list(strides_of(gpu_dst[0])), e)
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
