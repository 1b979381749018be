"""Staging a doomed rank's KV to its replacement during a preemption notice, in block rounds.

Same interface as the reference's ``everserve.reference.staging``
(core/everserve/reference/staging.py:1-94). A notice names a rank and a deadline. Until the
deadline the rank keeps serving, and its KV moves to the replacement in rounds:
* the first round moves every block in use;
* each later round moves only the blocks written since the round before.

Block ids are the scheduler's, shared by every tensor-parallel rank, so the replacement takes
each block at the same id.

This module plans the rounds: :func:`blocks_to_stage` picks the block ids, and
:class:`StagingWindow` keeps the counts. The bytes move through
:meth:`everserve_amd.state.staging.StepStager.commit_blocks`. That is one ``evs_gather_blocks``
launch per round: every layer and held head, the slot tags written beside the rows, then the
DMA copy to pinned host memory.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping, Sequence

BlockId = int
RequestId = str


@dataclass
class StagedRequest:
    """How far one request's KV has been staged (core/everserve/reference/staging.py:24-31)."""

    tokens: int
    """Tokens whose KV the replacement holds."""
    blocks: tuple[BlockId, ...]
    """The block ids those tokens were staged from, in table order."""


@dataclass
class StagingWindow:
    """Bookkeeping for one notice, from receipt to the deadline (staging.py:34-49)."""

    rank: int
    deadline: float
    """Unix seconds at which the rank leaves."""
    rounds: int = 0
    blocks_copied: int = 0
    bytes_copied: int = 0
    staged: dict[RequestId, StagedRequest] = field(default_factory=dict)

    def seconds_left(self, now: float) -> float:
        """Time to the deadline at ``now`` (Unix seconds); negative once it has passed."""
        return self.deadline - now


def _common_prefix(a: Sequence[BlockId], b: Sequence[BlockId]) -> int:
    n = min(len(a), len(b))
    for i in range(n):
        if a[i] != b[i]:
            return i
    return n


def blocks_to_stage(block_tables: Mapping[RequestId, Sequence[BlockId]],
                    num_computed: Mapping[RequestId, int],
                    staged: dict[RequestId, StagedRequest], block_size: int) -> list[BlockId]:
    """The sorted distinct block ids holding KV written since the previous round.

    Updates ``staged`` in place (core/everserve/reference/staging.py:51-94):
    * A request's staged tokens are cut back to the first block whose id changed since it was
      staged. A preempted and recomputed request sits in new blocks at the same token count,
      so it is staged again from there.
    * The blocks from the staged token to the last computed token are chosen.
    * A request missing from ``num_computed`` is forgotten.
    """
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    chosen: set[BlockId] = set()
    for rid, n in num_computed.items():
        table = tuple(block_tables[rid])
        prior = staged.get(rid)
        kept = 0
        if prior is not None:
            kept = min(prior.tokens, _common_prefix(prior.blocks, table) * block_size)
        kept = min(kept, n)
        if n > kept:
            chosen.update(table[kept // block_size:(n - 1) // block_size + 1])
        n_blocks = (n + block_size - 1) // block_size
        staged[rid] = StagedRequest(tokens=n, blocks=table[:n_blocks])
    for rid in [r for r in staged if r not in num_computed]:
        del staged[rid]
    return sorted(chosen)
