"""The reference's CPU path, restated in torch on the CPU. TEST INFRASTRUCTURE.

This is how the reference moves rows when the kernels are not in use: torch advanced indexing on
the cache tensors. It serves twice:

* as a second, independent formulation of the gather and the scatter (indexing by tensor
  dimensions, no strides), which the C oracle must agree with byte for byte;
* as ``bench.py``'s CPU baseline: the reference's CPU path timed on the GPU box's host cores.

Follows core/everserve/state/kvcopy.py:74-128 (split, rows, rows_of_heads, write_rows),
core/everserve/state/mirror.py:552-562 (one gather per layer copied into the staging file
[L, H, cap, 2, d]) and core/everserve/state/mirror.py:926-937 (the restore: index_select of the
written rows, then write_rows at the head slot they go to).
"""

from __future__ import annotations

from typing import Sequence

import torch

from oracle import BLOCKS_FIRST, KV_FIRST, recognise


def split(slots: torch.Tensor, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Slot ids -> (block, offset)."""
    slots = slots.long()
    return slots // block_size, slots % block_size


def rows(t: torch.Tensor, slots: torch.Tensor, head: int) -> torch.Tensor:
    """K and V rows of head slot ``head`` at ``slots``: [2, n, d] (kvcopy.py:79-87)."""
    layout, _, bs, d = recognise(t.shape)
    b, o = split(slots, bs)
    if layout == KV_FIRST:
        return t[:, b, o, head]
    if layout == BLOCKS_FIRST:
        return t[b, :, o, head].transpose(0, 1)
    x = t[b, head, o]
    return torch.stack([x[:, :d], x[:, d:]])


def rows_of_heads(t: torch.Tensor, slots: torch.Tensor, heads: torch.Tensor) -> torch.Tensor:
    """K and V rows of head slots ``heads`` at ``slots``: a view [h, n, 2, d] (kvcopy.py:89-103)."""
    layout, _, bs, d = recognise(t.shape)
    b, o = split(slots, bs)
    if layout == KV_FIRST:
        return t[:, b, o].index_select(2, heads).permute(2, 1, 0, 3)
    if layout == BLOCKS_FIRST:
        return t[b, :, o].index_select(2, heads).permute(2, 0, 1, 3)
    x = t[b, :, o].index_select(1, heads)
    return x.view(x.shape[0], x.shape[1], 2, d).permute(1, 0, 2, 3)


def write_rows(t: torch.Tensor, slots: torch.Tensor, head: int, x: torch.Tensor) -> None:
    """Write ``x`` [2, n, d] into head slot ``head`` at ``slots`` in place (kvcopy.py:118-128)."""
    layout, _, bs, _ = recognise(t.shape)
    b, o = split(slots, bs)
    if layout == KV_FIRST:
        t[:, b, o, head] = x
    elif layout == BLOCKS_FIRST:
        t[b, :, o, head] = x.transpose(0, 1)
    else:
        t[b, head, o] = torch.cat([x[0], x[1]], -1)


def gather_step(layers: Sequence[torch.Tensor], slots: torch.Tensor, heads: torch.Tensor,
                capacity: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """A step's rows of every layer as the torch path stages them: [L, H, capacity, 2, d].

    mirror.py:552-562 per layer: rows_of_heads on the slots clamped at 0 (mirror.py:579), copied
    into the staging tensor's first n rows.
    """
    _, _, _, d = recognise(layers[0].shape)
    n = slots.numel()
    if out is None:
        out = torch.zeros(len(layers), heads.numel(), capacity, 2, d, dtype=layers[0].dtype)
    clamped = slots.clamp(min=0)
    for i, t in enumerate(layers):
        out[i, :, :n].copy_(rows_of_heads(t, clamped, heads))
    return out


def restore_step(layers: Sequence[torch.Tensor], slots: torch.Tensor, heads: Sequence[int],
                 staged: torch.Tensor) -> None:
    """Write staged rows [L, H, cap, 2, d] back at ``slots`` and head slots ``heads``.

    The restore per (layer, head) table (mirror.py:926-937): the written rows (non-negative slots)
    are selected, then write_rows puts them at the head slot they go to.
    """
    keep = (slots >= 0).nonzero().flatten()
    idx = slots.index_select(0, keep)
    for i, t in enumerate(layers):
        for h, head in enumerate(heads):
            x = staged[i, h].index_select(0, keep)  # [n, 2, d]
            write_rows(t, idx, int(head), x.transpose(0, 1))


def member_sum(inputs: Sequence[torch.Tensor]) -> torch.Tensor:
    """The members summed in order in fp32 from zero, rounded once (ops.py:63-73)."""
    acc = torch.zeros(inputs[0].shape, dtype=torch.float32)
    for x in inputs:
        acc += x.float()
    return acc.to(inputs[0].dtype)
