"""The paged KV cache's layouts, and the rows of one head slot in them.

The same interface as the reference's ``everserve.state.kvcopy`` (core/everserve/state/kvcopy.py:
37-140), so a connector written against it runs unchanged. A layer's K and V sit in one of three
layouts:

* ``kv_first``:     ``[2, blocks, block_size, heads, head_dim]``
* ``blocks_first``: ``[blocks, 2, block_size, heads, head_dim]``
* ``combined``:     ``[blocks, heads, block_size, 2 * head_dim]`` (K and V side by side)

A slot id is ``block * block_size + offset``. :meth:`PagedKV.layout_strides` reduces any of them
(and strided views of them) to the five element strides the HIP kernels address the cache with.
The torch methods (:meth:`rows`, :meth:`rows_of_heads`, :meth:`write_rows`) are the reference's
torch path, kept for callers that run with ``EVERSERVE_KERNELS=torch``; the kernels are
:mod:`everserve_amd.kernels`.
"""

from __future__ import annotations

import re
from collections.abc import Hashable
from dataclasses import dataclass
from enum import Enum

import torch

Unit = Hashable
HeadSlot = int
_LAYER_INDEX = re.compile(r"layers\.(\d+)\.")


class CacheLayout(str, Enum):
    """How one layer's paged K/V tensor is laid out."""

    KV_FIRST = "kv_first"
    BLOCKS_FIRST = "blocks_first"
    COMBINED = "combined"


@dataclass(frozen=True)
class PagedKV:
    """One layer's paged-cache shape, and how to read and write the rows of one head slot."""

    layout: CacheLayout
    num_blocks: int
    block_size: int
    head_dim: int

    @property
    def num_slots(self) -> int:
        """Total slot ids in the cache."""
        return self.num_blocks * self.block_size

    @classmethod
    def of(cls, t: torch.Tensor) -> PagedKV:
        """Recognise the layout of a layer's cache tensor.

        Raises:
            ValueError: for a shape that is none of the three layouts.
        """
        shape = tuple(t.shape)
        if len(shape) == 5 and shape[0] == 2:
            return cls(CacheLayout.KV_FIRST, shape[1], shape[2], shape[4])
        if len(shape) == 5 and shape[1] == 2:
            return cls(CacheLayout.BLOCKS_FIRST, shape[0], shape[2], shape[4])
        if len(shape) == 4 and shape[3] % 2 == 0:
            return cls(CacheLayout.COMBINED, shape[0], shape[2], shape[3] // 2)
        raise ValueError(f"unsupported KV cache layout {shape}")

    def split(self, slots: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Slot ids -> (block, offset)."""
        slots = slots.long()
        return slots // self.block_size, slots % self.block_size

    def layout_strides(self, t: torch.Tensor) -> tuple[int, int, int, int, int]:
        """``t``'s element strides as (block, offset in block, head slot, K-or-V, element)."""
        st = t.stride()
        if self.layout is CacheLayout.KV_FIRST:
            return st[1], st[2], st[3], st[0], st[4]
        if self.layout is CacheLayout.BLOCKS_FIRST:
            return st[0], st[2], st[3], st[1], st[4]
        return st[0], st[2], st[1], self.head_dim * st[3], st[3]

    def rows(self, t: torch.Tensor, slots: torch.Tensor, head: HeadSlot) -> torch.Tensor:
        """The K and V rows of head slot ``head`` at ``slots``, as a copy of shape ``[2, n, d]``."""
        b, o = self.split(slots)
        if self.layout is CacheLayout.KV_FIRST:
            return t[:, b, o, head]
        if self.layout is CacheLayout.BLOCKS_FIRST:
            return t[b, :, o, head].transpose(0, 1)
        x = t[b, head, o]
        return torch.stack([x[:, : self.head_dim], x[:, self.head_dim :]])

    def rows_of_heads(
        self, t: torch.Tensor, slots: torch.Tensor, heads: torch.Tensor
    ) -> torch.Tensor:
        """The K and V rows of head slots ``heads`` at ``slots``, as a view ``[h, n, 2, d]``."""
        b, o = self.split(slots)
        if self.layout is CacheLayout.KV_FIRST:
            return t[:, b, o].index_select(2, heads).permute(2, 1, 0, 3)
        if self.layout is CacheLayout.BLOCKS_FIRST:
            return t[b, :, o].index_select(2, heads).permute(2, 0, 1, 3)
        x = t[b, :, o].index_select(1, heads)
        return x.view(x.shape[0], x.shape[1], 2, self.head_dim).permute(1, 0, 2, 3)

    def write_rows(
        self, t: torch.Tensor, slots: torch.Tensor, head: HeadSlot, x: torch.Tensor
    ) -> None:
        """Write ``x`` of shape ``[2, n, d]`` into head slot ``head`` at ``slots``, in place."""
        b, o = self.split(slots)
        if self.layout is CacheLayout.KV_FIRST:
            t[:, b, o, head] = x
        elif self.layout is CacheLayout.BLOCKS_FIRST:
            t[b, :, o, head] = x.transpose(0, 1)
        else:
            t[b, head, o] = torch.cat([x[0], x[1]], -1)


def layer_index(name: str) -> int:
    """The layer number in a cache name such as ``model.layers.12.self_attn.attn``.

    Raises:
        ValueError: if the name carries no layer index.
    """
    m = _LAYER_INDEX.search(name)
    if m is None:
        raise ValueError(f"cannot find a layer index in cache name {name!r}")
    return int(m.group(1))
