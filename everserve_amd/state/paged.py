"""What the kernels need to know about one layer's paged KV tensor: its layout and five strides.

A cache layer is one torch tensor per layer, in one of the three layouts the reference's
connector accepts (core/everserve/state/kvcopy.py:37-72):

=================  ==================================  ===================================
layout             shape                               dimension roles
=================  ==================================  ===================================
``kv_first``       ``[2, blocks, block_size, heads, d]``  kv, block, offset, head, elem
``blocks_first``   ``[blocks, 2, block_size, heads, d]``  block, kv, offset, head, elem
``combined``       ``[blocks, heads, block_size, 2 d]``   block, head, offset, (kv, elem)
=================  ==================================  ===================================

The kernels address every layout the same way: a slot id ``s`` is ``block * block_size +
offset``, and the element ``j`` of K (``kv = 0``) or V (``kv = 1``) of head slot ``h`` sits
``block * S_block + offset * S_offset + h * S_head + kv * S_kv + j * S_elem`` elements from the
layer's base. :func:`strides_of` reads those five strides off the tensor's own strides through
the role table above, so a strided view (a head slice, a permuted copy) is addressed correctly
without being copied. In ``combined`` the last dimension holds K then V, so ``S_kv`` is ``d``
times that dimension's stride.

The order of the five strides, (block, offset, head, kv, elem), is the argument order of the
reference's ``gather_rows`` (core/csrc/gather.cu:100-102, kvcopy.py:105-116), which the C ABI
keeps.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from enum import Enum
from typing import Sequence

HeadSlot = int
"""A KV head's index in a layer's head dimension."""

STRIDE_ROLES = ("block", "offset", "head", "kv", "elem")
"""The kernels' stride order."""


class CacheLayout(str, Enum):
    """How one layer's paged K/V tensor is laid out (the names are the connector's)."""

    KV_FIRST = "kv_first"
    BLOCKS_FIRST = "blocks_first"
    COMBINED = "combined"


# role of each tensor dimension; "kv*elem" is combined's last dimension, K then V
_ROLES: dict[CacheLayout, tuple[str, ...]] = {
    CacheLayout.KV_FIRST: ("kv", "block", "offset", "head", "elem"),
    CacheLayout.BLOCKS_FIRST: ("block", "kv", "offset", "head", "elem"),
    CacheLayout.COMBINED: ("block", "head", "offset", "kv*elem"),
}


def _classify(shape: Sequence[int]) -> CacheLayout:
    """The layout a shape has. A 5-D shape with 2 in both of its first two dimensions is taken
    as ``kv_first``, the reference's precedence (kvcopy.py:60-72)."""
    if len(shape) == 5:
        if shape[0] == 2:
            return CacheLayout.KV_FIRST
        if shape[1] == 2:
            return CacheLayout.BLOCKS_FIRST
    elif len(shape) == 4 and shape[3] % 2 == 0:
        return CacheLayout.COMBINED
    raise ValueError(f"unsupported KV cache layout {tuple(shape)}")


@dataclass(frozen=True)
class PagedKV:
    """One layer's cache geometry: its layout, block count, block size, head count and head size.

    The constructor and :meth:`of` carry the connector's names (kvcopy.py:37-72) because callers
    build and pass these objects; everything else is this module's.
    """

    layout: CacheLayout
    num_blocks: int
    block_size: int
    head_dim: int
    num_heads: int = 0
    """KV heads in the layer (0 when not known, as for an object built by hand)."""

    @property
    def num_slots(self) -> int:
        """Slot ids the cache holds: ``num_blocks * block_size``."""
        return self.num_blocks * self.block_size

    @property
    def row_elems(self) -> int:
        """Elements of one row of one head slot: K then V, ``2 * head_dim``."""
        return 2 * self.head_dim

    @classmethod
    def of(cls, t) -> "PagedKV":
        """The geometry of the cache tensor ``t`` (anything with a ``shape``).

        Raises:
            ValueError: for a shape that is none of the three layouts.
        """
        shape = tuple(int(x) for x in t.shape)
        layout = _classify(shape)
        dims = dict(zip(_ROLES[layout], shape))
        if layout is CacheLayout.COMBINED:
            return cls(layout, dims["block"], dims["offset"], dims["kv*elem"] // 2, dims["head"])
        return cls(layout, dims["block"], dims["offset"], dims["elem"], dims["head"])

    def layout_strides(self, t) -> tuple[int, int, int, int, int]:
        """``t``'s element strides in the kernels' order (block, offset, head, kv, elem)."""
        return strides_of(self.layout, t.stride(), self.head_dim)

    def check_slots(self, lo: int, hi: int) -> None:
        """Refuse slot ids outside ``[0, num_slots)``: ``lo`` and ``hi`` are the smallest and
        largest of a list about to be written.

        Raises:
            ValueError: naming the first id out of range.
        """
        if lo < 0 or hi >= self.num_slots:
            bad = lo if lo < 0 else hi
            raise ValueError(f"slot {bad} lies outside this cache's {self.num_slots} slots")

    # The connector's row accessors (kvcopy.py:74-128), on the kernels: one launch each, on the
    # current stream of the tensor's device. The connector indexes with torch, where a negative
    # slot wraps to the cache's end; its callers never pass one (the snapshot clamps its slots
    # first, mirror.py:579, and a restore writes stored ranges). Here a negative slot reads slot
    # 0 and is not written, as the kernels treat padding.
    def split(self, slots):
        """Slot ids -> (block, offset in block), as int64 tensors."""
        s = slots.long()
        return s // self.block_size, s % self.block_size

    def rows_of_heads(self, t, slots, heads):
        """The K and V rows of head slots ``heads`` at ``slots``: a new ``[h, n, 2, d]`` tensor
        (the connector returns a view of the same values)."""
        import torch

        n, h = int(slots.numel()), int(heads.numel())
        out = torch.empty((1, h, n, 2, self.head_dim), dtype=t.dtype, device=t.device)
        if n and h:
            _kernels().gather_rows(_layer(t), _ids(slots, t), _ids(heads, t), out.data_ptr(), n,
                                   self.head_dim, self.block_size, self.layout_strides(t),
                                   t.element_size())
        return out[0]

    def rows(self, t, slots, head: int):
        """The K and V rows of head slot ``head`` at ``slots``, as a copy ``[2, n, d]``."""
        import torch

        heads = torch.tensor([int(head)], dtype=torch.long, device=t.device)
        return self.rows_of_heads(t, slots, heads)[0].transpose(0, 1).contiguous()

    def write_rows(self, t, slots, head: int, x) -> None:
        """Write ``x`` of shape ``[2, n, d]`` into head slot ``head`` at ``slots``, in place."""
        import torch

        n = int(slots.numel())
        if tuple(x.shape) != (2, n, self.head_dim):
            raise ValueError(f"write_rows: rows of shape {tuple(x.shape)}, expected "
                             f"{(2, n, self.head_dim)}")
        if x.dtype != t.dtype or x.device != t.device:
            raise ValueError("write_rows: the rows must have the cache's dtype and device")
        staged = x.transpose(0, 1).contiguous()  # [n, 2, d]: one layer, one head, capacity n
        heads = torch.tensor([int(head)], dtype=torch.long, device=t.device)
        if n:
            _kernels().scatter_rows(_layer(t), _ids(slots, t), heads, staged.data_ptr(), n,
                                    self.head_dim, self.block_size, self.layout_strides(t),
                                    t.element_size(), ordered=False)


def _kernels():
    """The loaded kernels (raises when they cannot load: no quiet fallback)."""
    from everserve_amd import kernels

    return kernels.load()


def _ids(ids, t):
    """``ids`` as a contiguous int64 tensor on ``t``'s device."""
    import torch

    return ids.to(device=t.device, dtype=torch.long).contiguous()


def _layer(t):
    """A one-entry device table of ``t``'s address, as the kernels take layers."""
    import torch

    return torch.tensor([t.data_ptr()], dtype=torch.long, device=t.device)


def strides_of(layout: CacheLayout | str, tensor_strides: Sequence[int],
               head_dim: int) -> tuple[int, int, int, int, int]:
    """The five kernel strides of a ``layout`` tensor whose strides are ``tensor_strides``."""
    roles = _ROLES[CacheLayout(layout)]
    if len(roles) != len(tensor_strides):
        raise ValueError(f"a {CacheLayout(layout).value} cache has {len(roles)} dimensions, "
                         f"not {len(tensor_strides)}")
    by_role = dict(zip(roles, (int(s) for s in tensor_strides)))
    packed = by_role.pop("kv*elem", None)
    if packed is not None:
        by_role["elem"] = packed
        by_role["kv"] = head_dim * packed
    return tuple(by_role[r] for r in STRIDE_ROLES)  # type: ignore[return-value]


_LAYER_NUMBER = re.compile(r"layers\.(\d+)\.")


def layer_index(name: str) -> int:
    """The layer number of a cache named like ``model.layers.12.self_attn.attn``.

    The step path orders a rank's caches by it, as the connector registers them.

    Raises:
        ValueError: for a name without one.
    """
    found = _LAYER_NUMBER.search(name)
    if found is None:
        raise ValueError(f"no layer number in the cache name {name!r}")
    return int(found.group(1))
