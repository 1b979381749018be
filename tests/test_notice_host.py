"""The product's notice-round planner against the oracle's, on the CPU.

``everserve_amd.state.notice.blocks_to_stage`` is the product's. The oracle's restatement of the
reference (core/everserve/reference/staging.py:51-94) is pinned in test_oracle_staging.py. The two
are run here side by side over seeded random histories of that file's simulated batch: decode and
multi-token steps, prefills of new requests, preemptions into new blocks and finished requests.
The same block ids and the same staged state are wanted after every round.
"""

import random

import pytest

import oracle
from everserve_amd.state import notice
from tests.test_oracle_staging import BLOCK, Batch


def as_oracle(staged):
    return {r: (s.tokens, tuple(s.blocks)) for r, s in staged.items()}


@pytest.mark.parametrize("seed", range(12))
def test_the_plan_is_the_oracles_round_after_round(seed):
    rng = random.Random(seed)
    batch = Batch({f"q{i}": rng.randrange(1, 40) for i in range(rng.randrange(1, 6))}, seed=seed,
                  pool_blocks=128)
    ours, theirs = {}, {}
    admitted = len(batch.blocks)
    for _ in range(30):
        got = notice.blocks_to_stage(batch.blocks, dict(batch.length), ours, BLOCK)
        want = oracle.blocks_to_stage(batch.blocks, dict(batch.length), theirs, BLOCK)
        assert got == want
        assert as_oracle(ours) == theirs
        event = rng.random()
        if event < 0.1 and batch.length:
            batch.recompute(rng.choice(sorted(batch.length)))
        elif event < 0.2 and len(batch.length) > 1:
            batch.finish(rng.choice(sorted(batch.length)))
        elif event < 0.3 and len(batch.pool) > 8:
            batch.admit(f"q{admitted}", rng.randrange(1, 20))
            admitted += 1
        for r in list(batch.length):
            if len(batch.pool) > 4:
                batch.append(r, rng.choice((1, 1, 1, 2, 17)))


def test_the_window_counts_down_to_the_deadline():
    w = notice.StagingWindow(rank=3, deadline=100.0)
    assert w.seconds_left(40.0) == 60.0
    assert w.seconds_left(101.0) == -1.0
    assert (w.rounds, w.blocks_copied, w.bytes_copied, w.staged) == (0, 0, 0, {})
    w.record(5, 1000)
    w.record(2, 24)
    assert (w.rounds, w.blocks_copied, w.bytes_copied) == (2, 7, 1024)


def test_a_table_that_changed_under_a_staged_request_restarts_at_the_first_changed_block():
    staged = {}
    assert notice.blocks_to_stage({"a": [4, 5, 6]}, {"a": 40}, staged, 16) == [4, 5, 6]
    # recomputed into new blocks from the second one, one token more
    assert notice.blocks_to_stage({"a": [4, 9, 8]}, {"a": 41}, staged, 16) == [8, 9]
    assert staged["a"].tokens == 41 and staged["a"].blocks == (4, 9, 8)
    # nothing new: nothing staged; a finished request is forgotten
    assert notice.blocks_to_stage({"a": [4, 9, 8]}, {"a": 41}, staged, 16) == []
    assert notice.blocks_to_stage({}, {}, staged, 16) == [] and staged == {}


def test_block_size_must_be_positive():
    with pytest.raises(ValueError):
        notice.blocks_to_stage({}, {}, {}, 0)
