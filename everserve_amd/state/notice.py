"""Notice rounds: which cache blocks a doomed rank copies to its replacement, round by round.

When a rank is given notice it keeps serving until a deadline, and its KV moves to the spare
that will take its place in rounds. The rule (the reference's, core/everserve/reference/
staging.py:51-94, which the notice protocol's other side relies on) is:

* a request is staged up to the tokens its KV holds (``num_computed``);
* in each round, a request's staged prefix is kept only as far as its block table still starts
  with the blocks it was staged from; a request preempted and recomputed into other blocks is
  staged again from its first changed block;
* the round copies every block holding a token past the kept prefix, up to the last computed
  token; a block shared by several requests is copied once; the ids go out sorted;
* a request no longer computed (finished, or dropped) is forgotten.

Block ids are the scheduler's, the same on every tensor-parallel rank, so the replacement puts
each block at the id it had. This module plans; the bytes move through
``StepStager.commit_blocks`` (one ``evs_gather_blocks`` launch per round).

The planner compares block tables with numpy, one vector comparison per request, and keeps for
each request only its token count and the block ids that hold those tokens.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping, Sequence

import numpy as np

BlockId = int
RequestId = str


@dataclass
class StagedRequest:
    """One request as the replacement holds it: ``tokens`` staged, from ``blocks`` (the first
    ``ceil(tokens / block_size)`` ids of its block table at that round)."""

    tokens: int
    blocks: tuple[BlockId, ...]


@dataclass
class StagingWindow:
    """One notice: the rank, its deadline (Unix seconds), what has moved so far, and each
    request's staged state, which :func:`blocks_to_stage` updates."""

    rank: int
    deadline: float
    rounds: int = 0
    blocks_copied: int = 0
    bytes_copied: int = 0
    staged: dict[RequestId, StagedRequest] = field(default_factory=dict)

    def seconds_left(self, now: float) -> float:
        """Seconds from ``now`` to the deadline, negative after it."""
        return self.deadline - now

    def record(self, blocks: int, nbytes: int) -> None:
        """Count one round that copied ``blocks`` blocks, ``nbytes`` bytes."""
        self.rounds += 1
        self.blocks_copied += blocks
        self.bytes_copied += nbytes


def _unchanged_blocks(before: Sequence[BlockId], now: np.ndarray) -> int:
    """How many leading ids of ``now`` equal those of ``before``."""
    k = min(len(before), now.size)
    if k == 0:
        return 0
    differ = np.flatnonzero(np.asarray(before[:k], dtype=np.int64) != now[:k])
    return int(differ[0]) if differ.size else k


def blocks_to_stage(block_tables: Mapping[RequestId, Sequence[BlockId]],
                    num_computed: Mapping[RequestId, int],
                    staged: dict[RequestId, StagedRequest], block_size: int) -> list[BlockId]:
    """This round's block ids, sorted and distinct; ``staged`` is brought up to date.

    ``block_tables`` maps each request to its block ids in scheduler order, ``num_computed`` to
    the tokens its KV holds now. Only the requests in ``num_computed`` are planned; the others
    are dropped from ``staged``.

    Raises:
        ValueError: for a block size below 1.
    """
    if block_size < 1:
        raise ValueError(f"block_size must be positive, got {block_size}")
    picked: list[np.ndarray] = []
    for rid, tokens in num_computed.items():
        table = np.asarray(block_tables[rid], dtype=np.int64).reshape(-1)
        held = staged.get(rid)
        kept = 0
        if held is not None:
            kept = min(held.tokens, _unchanged_blocks(held.blocks, table) * block_size)
        kept = min(kept, tokens)
        used = -(-tokens // block_size)  # blocks holding tokens [0, tokens)
        if tokens > kept:
            picked.append(table[kept // block_size:used])
        staged[rid] = StagedRequest(tokens, tuple(int(b) for b in table[:used]))
    for rid in set(staged) - set(num_computed):
        del staged[rid]
    if not picked:
        return []
    return np.unique(np.concatenate(picked)).tolist()
