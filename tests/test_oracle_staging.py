"""Pins of the block-table staging plan (oracle.blocks_to_stage), on the CPU.

The reference's scenarios (core/tests/test_staging.py:1-116): a mock paged cache written token by
token by decoding requests, staged round by round into a replacement copy. The first round
copies every block in use; a later round copies exactly the blocks that received tokens since the
previous one; a preempted request (new block ids, same token count) is staged again and a
finished one dropped; multi-token steps across block boundaries; after each round the replacement
equals the source on every block in use.
"""

import random

import numpy as np
import pytest

import oracle

BS, NB = 16, 64


class Cache:
    """Block tables plus per-block contents, written one token at a time."""

    def __init__(self, n_req: int, prompt: int, seed: int = 0):
        self.rng = random.Random(seed)
        self.free = list(range(NB))
        self.rng.shuffle(self.free)
        self.tables = {str(i): [] for i in range(n_req)}
        self.n = {str(i): 0 for i in range(n_req)}
        self.kv = np.zeros((NB, BS), dtype=np.int64)
        for rid in self.tables:
            self.write(rid, prompt)

    def write(self, rid: str, k: int) -> None:
        for _ in range(k):
            pos = self.n[rid]
            if pos // BS >= len(self.tables[rid]):
                self.tables[rid].append(self.free.pop())
            self.kv[self.tables[rid][pos // BS], pos % BS] = self.rng.randrange(1, 1 << 30)
            self.n[rid] += 1

    def preempt(self, rid: str) -> None:
        n = self.n[rid]
        for b in self.tables[rid]:
            self.kv[b] = 0
            self.free.append(b)
        self.tables[rid], self.n[rid] = [], 0
        self.rng.shuffle(self.free)
        self.write(rid, n)

    def finish(self, rid: str) -> None:
        for b in self.tables.pop(rid):
            self.kv[b] = 0
            self.free.append(b)
        del self.n[rid]

    def in_use(self) -> list[int]:
        return sorted(b for t in self.tables.values() for b in t)


def stage(src: Cache, dst: np.ndarray, staged: dict) -> list[int]:
    ids = oracle.blocks_to_stage(src.tables, dict(src.n), staged, BS)
    dst[ids] = src.kv[ids]
    return ids


def test_the_first_round_copies_every_block_in_use():
    c = Cache(4, 37)
    dst, staged = np.zeros((NB, BS), np.int64), {}
    assert stage(c, dst, staged) == c.in_use()
    assert np.array_equal(dst[c.in_use()], c.kv[c.in_use()])


def test_rounds_copy_only_changed_blocks_and_end_equal():
    c = Cache(8, 50, seed=1)
    dst, staged = np.zeros((NB, BS), np.int64), {}
    stage(c, dst, staged)
    for _ in range(40):
        before = dict(c.n)
        for rid in c.n:
            c.write(rid, 1)
        ids = stage(c, dst, staged)
        touched = {c.tables[rid][p // BS] for rid in c.n for p in range(before[rid], c.n[rid])}
        assert set(ids) == touched
        assert len(ids) <= len(c.n)
    assert np.array_equal(dst[c.in_use()], c.kv[c.in_use()])


def test_a_preempted_request_is_restaged_and_a_finished_one_dropped():
    c = Cache(4, 30, seed=2)
    dst, staged = np.zeros((NB, BS), np.int64), {}
    stage(c, dst, staged)
    for rid in c.n:
        c.write(rid, 5)
    c.preempt("1")
    c.finish("3")
    stage(c, dst, staged)
    assert "3" not in staged
    assert np.array_equal(dst[c.in_use()], c.kv[c.in_use()])


def test_multi_token_steps_across_block_boundaries():
    c = Cache(3, 15, seed=3)
    dst, staged = np.zeros((NB, BS), np.int64), {}
    stage(c, dst, staged)
    for k in (1, 2, 17, 3, 33):
        for rid in c.n:
            c.write(rid, k)
        stage(c, dst, staged)
        assert np.array_equal(dst[c.in_use()], c.kv[c.in_use()])


def test_block_size_must_be_positive():
    with pytest.raises(ValueError):
        oracle.blocks_to_stage({}, {}, {}, 0)


def test_a_planted_mistake_is_caught():
    """Staging only the last block of each request each round loses a prefill's earlier blocks."""
    c = Cache(4, 40, seed=4)
    dst = np.zeros((NB, BS), np.int64)
    ids = sorted({c.tables[r][(c.n[r] - 1) // BS] for r in c.n})
    dst[ids] = c.kv[ids]
    assert not np.array_equal(dst[c.in_use()], c.kv[c.in_use()])
