"""Pins of the block-table staging plan (oracle.blocks_to_stage), on the CPU.

The plan (core/everserve/reference/staging.py:51-94) picks, each notice round, the cache blocks
whose KV was written since the round before. It is pinned here by what a replica built from its
rounds must be: a decoding batch is simulated on a small paged cache (every token written as a
value that names its request, position and generation), each round's chosen blocks are copied
into a replica, and after every round the replica must equal the cache on each block in use.
On top of that, the first round must be exactly the blocks in use, a later round exactly the
blocks that took a token since, a request recomputed into new blocks (preemption) is staged
again, and a finished one is dropped. The reference's own tests state the same properties over
their mock cache (core/tests/test_staging.py:1-116); the scenarios below are this file's.
"""

import numpy as np
import pytest

import oracle

BLOCK = 16
POOL = 96


class Batch:
    """A paged cache under decoding requests: each request owns a list of block ids taken from a
    seeded free pool, and its token t lives at offset t % BLOCK of its (t // BLOCK)-th block.
    Other tests build on it (the product planner's pins, the GPU notice rounds)."""

    def __init__(self, prompts: dict[str, int], seed: int, pool_blocks: int = POOL):
        self.rng = np.random.default_rng(seed)
        self.pool = [int(b) for b in self.rng.permutation(pool_blocks)]
        self.blocks: dict[str, list[int]] = {}
        self.length: dict[str, int] = {}
        self.generation: dict[str, int] = {}
        self.ident: dict[str, int] = {}
        self.cache = np.zeros((pool_blocks, BLOCK), dtype=np.int64)
        for r, n in prompts.items():
            self.admit(r, n)

    def admit(self, r: str, n: int) -> None:
        """A new request, prefilled with n tokens."""
        self.blocks[r], self.length[r], self.generation[r] = [], 0, 0
        self.ident[r] = len(self.ident) + 1
        self.append(r, n)

    def value(self, r: str, t: int) -> int:
        return (self.ident[r] << 40) | (self.generation[r] << 32) | (t + 1)

    def on_token(self, b: int, offset: int, r: str, t: int) -> None:
        self.cache[b, offset] = self.value(r, t)

    def append(self, r: str, n: int) -> set[int]:
        """Write n more tokens of r; returns the blocks written."""
        touched = set()
        for _ in range(n):
            t = self.length[r]
            if t % BLOCK == 0:
                self.blocks[r].append(self.pool.pop())
            b = self.blocks[r][t // BLOCK]
            self.on_token(b, t % BLOCK, r, t)
            self.length[r] = t + 1
            touched.add(b)
        return touched

    def release(self, r: str) -> None:
        for b in self.blocks[r]:
            self.cache[b] = 0
        self.pool = [int(b) for b in self.rng.permutation(self.pool + self.blocks[r])]
        self.blocks[r] = []

    def recompute(self, r: str) -> None:
        """Preemption: r's blocks go back to the pool and its tokens are written again into new
        ones (a new generation, so a stale copy of the old blocks shows)."""
        n = self.length[r]
        self.release(r)
        self.length[r] = 0
        self.generation[r] += 1
        self.append(r, n)

    def finish(self, r: str) -> None:
        self.release(r)
        del self.blocks[r], self.length[r], self.generation[r], self.ident[r]

    def in_use(self) -> list[int]:
        return sorted(b for bs in self.blocks.values() for b in bs)


class Replica:
    """The copy a spare builds, one notice round at a time."""

    def __init__(self):
        self.cache = np.zeros((POOL, BLOCK), dtype=np.int64)
        self.staged: dict = {}

    def round(self, batch: Batch) -> list[int]:
        ids = oracle.blocks_to_stage(batch.blocks, dict(batch.length), self.staged, BLOCK)
        self.cache[ids] = batch.cache[ids]
        return ids

    def matches(self, batch: Batch) -> bool:
        live = batch.in_use()
        return bool(np.array_equal(self.cache[live], batch.cache[live]))


@pytest.mark.parametrize("prompts", [{"a": 1, "b": 16, "c": 17, "d": 47},
                                     {"x": 64}, {"p": 5, "q": 5, "r": 5}])
def test_the_first_round_takes_every_block_in_use(prompts):
    batch = Batch(prompts, seed=11)
    rep = Replica()
    assert rep.round(batch) == batch.in_use()
    assert rep.matches(batch)


@pytest.mark.parametrize("seed", [21, 22])
def test_each_later_round_takes_exactly_the_blocks_written_since(seed):
    batch = Batch({f"r{i}": 9 + 7 * i for i in range(6)}, seed=seed)
    rep = Replica()
    rep.round(batch)
    rng = np.random.default_rng(seed)
    for _ in range(60):
        touched = set()
        for r in batch.length:  # some requests idle this step, some take two tokens
            touched |= batch.append(r, int(rng.integers(0, 3)))
        assert set(rep.round(batch)) == touched
        assert rep.matches(batch)
    assert rep.round(batch) == []  # nothing written since: nothing to stage


def test_a_recomputed_request_is_staged_again_and_a_finished_one_dropped():
    batch = Batch({"u": 40, "v": 20, "w": 33}, seed=31)
    rep = Replica()
    rep.round(batch)
    batch.append("u", 3)
    batch.recompute("v")
    batch.finish("w")
    ids = set(rep.round(batch))
    assert set(batch.blocks["v"]) <= ids  # every new block of v, written or not before
    assert "w" not in rep.staged
    assert rep.matches(batch)
    batch.recompute("u")  # recomputed between rounds, with no new token
    assert set(rep.round(batch)) == set(batch.blocks["u"])
    assert rep.matches(batch)


@pytest.mark.parametrize("steps", [(16, 1, 31, 2, 48), (15, 17, 1, 64)])
def test_appends_across_several_blocks(steps):
    batch = Batch({"m": 3, "n": 16, "o": 30}, seed=41)
    rep = Replica()
    rep.round(batch)
    for k in steps:
        touched = set()
        for r in batch.length:
            touched |= batch.append(r, k)
        assert set(rep.round(batch)) == touched
        assert rep.matches(batch)


def test_a_non_positive_block_size_is_refused():
    for bs in (0, -16):
        with pytest.raises(ValueError):
            oracle.blocks_to_stage({}, {}, {}, bs)


def test_planted_mistakes_are_caught():
    """Two wrong plans fail the replica check: one that stages only each request's last block
    (a prefill's earlier blocks are lost), and one that keeps the staged count across a
    recompute (the new blocks are never copied)."""
    batch = Batch({"a": 40, "b": 2}, seed=51)
    rep = Replica()
    last = sorted({bs[(batch.length[r] - 1) // BLOCK] for r, bs in batch.blocks.items()})
    rep.cache[last] = batch.cache[last]
    assert not rep.matches(batch)

    rep = Replica()
    rep.round(batch)
    batch.recompute("a")
    # a plan that tracks counts only: it takes the staged blocks to be whatever the table holds now
    counts_only = {r: (n, tuple(batch.blocks[r])) for r, (n, _) in rep.staged.items()}
    ids = oracle.blocks_to_stage(batch.blocks, dict(batch.length), counts_only, BLOCK)
    rep.cache[ids] = batch.cache[ids]
    assert not rep.matches(batch)
