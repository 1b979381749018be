"""The product's layout helper (everserve_amd.state.paged) on the CPU.

``PagedKV.of`` and ``layout_strides`` must give the oracle's (layout, geometry) and five strides
(oracle.recognise and oracle.layout_strides, pinned in test_oracle_rows.py against torch's own
strides), for contiguous caches, head slices, permuted copies and the shapes where the layouts
could be confused. The strides must also address the same element torch indexing reads, which
pins them without the oracle in the loop.
"""

import itertools

import pytest
import torch

import oracle
from everserve_amd.state.paged import CacheLayout, PagedKV, layer_index, strides_of

SHAPES = {
    "kv_first": (2, 7, 4, 3, 8),
    "blocks_first": (7, 2, 4, 3, 8),
    "combined": (7, 3, 4, 16),
}


def views(layout):
    """The contiguous cache, a slice of its head dimension and a permuted-then-restored copy."""
    t = torch.arange(int(torch.tensor(SHAPES[layout]).prod()), dtype=torch.float32).reshape(
        SHAPES[layout])
    yield t
    head_dim = {"kv_first": 3, "blocks_first": 3, "combined": 1}[layout]
    yield t.narrow(head_dim, 1, 2)
    order = list(reversed(range(t.dim())))
    yield t.permute(order).contiguous().permute(order)


@pytest.mark.parametrize("layout", sorted(SHAPES))
def test_geometry_and_strides_equal_the_oracles(layout):
    for t in views(layout):
        p = PagedKV.of(t)
        want = oracle.recognise(tuple(t.shape))
        assert (p.layout.value, p.num_blocks, p.block_size, p.head_dim) == want
        assert p.layout_strides(t) == oracle.layout_strides(want[0], t.stride(), want[3])
        assert p.num_slots == want[1] * want[2]


@pytest.mark.parametrize("layout", sorted(SHAPES))
def test_the_strides_address_what_torch_indexing_reads(layout):
    """Every (slot, head, kv, element) of every view, read through the five strides from the
    storage, equals the element torch's indexing of the layout picks."""
    for t in views(layout):
        p = PagedKV.of(t)
        sb, so, sh, skv, se = p.layout_strides(t)
        flat = t.as_strided((t.untyped_storage().nbytes() // 4,), (1,), 0)
        heads = t.shape[3] if p.layout is not CacheLayout.COMBINED else t.shape[1]
        for s, h, kv, j in itertools.product(range(p.num_slots), range(heads), (0, 1),
                                             range(p.head_dim)):
            b, o = divmod(s, p.block_size)
            at = t.storage_offset() + b * sb + o * so + h * sh + kv * skv + j * se
            if p.layout is CacheLayout.KV_FIRST:
                want = t[kv, b, o, h, j]
            elif p.layout is CacheLayout.BLOCKS_FIRST:
                want = t[b, kv, o, h, j]
            else:
                want = t[b, h, o, kv * p.head_dim + j]
            assert flat[at] == want


def test_num_heads_is_read_off_the_shape():
    assert PagedKV.of(torch.empty(SHAPES["kv_first"])).num_heads == 3
    assert PagedKV.of(torch.empty(SHAPES["blocks_first"])).num_heads == 3
    assert PagedKV.of(torch.empty(SHAPES["combined"])).num_heads == 3


def test_a_shape_with_two_in_both_leading_dimensions_is_kv_first():
    # the reference tests kv_first first (core/everserve/state/kvcopy.py:60-72)
    p = PagedKV.of(torch.empty(2, 2, 4, 3, 8))
    assert p.layout is CacheLayout.KV_FIRST and p.num_blocks == 2


@pytest.mark.parametrize("shape", [(3, 7, 4, 3, 8), (7, 3, 4, 15), (7, 4, 16), (2, 7, 4, 3, 8, 1)])
def test_other_shapes_are_refused(shape):
    with pytest.raises(ValueError):
        PagedKV.of(torch.empty(shape))


def test_a_stride_list_of_the_wrong_length_is_refused():
    with pytest.raises(ValueError):
        strides_of("combined", (1, 2, 3, 4, 5), 8)


def test_slot_bounds():
    p = PagedKV.of(torch.empty(SHAPES["kv_first"]))
    p.check_slots(0, p.num_slots - 1)
    for lo, hi in ((-1, 3), (0, p.num_slots)):
        with pytest.raises(ValueError):
            p.check_slots(lo, hi)


def test_layer_numbers_come_from_the_cache_name():
    assert layer_index("model.layers.12.self_attn.attn") == 12
    assert layer_index("decoder_layers.3.attn") == 3
    with pytest.raises(ValueError):
        layer_index("model.embed_tokens")
