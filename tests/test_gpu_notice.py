"""Notice rounds on the GPU: a doomed rank's cache staged block round by block round, then restored.

The reference's scenario (core/tests/test_staging.py:1-116) is a cache written token by token while
rounds copy the blocks that changed. Here the cache is on the GPU, every layer and head slot, and
each round goes through the product path:
1. ``StepStager.stage_round`` plans the round and gathers the blocks with the slot tags.
2. The rows are delivered into the round's staging file in the rank directory.
3. The oracle's store commit maps that file by its name and copies the rows into tables
   (store/src/storage.rs:864-957).

After the last round the product ``Restorer`` writes the tables' written ranges into a fresh cache
(core/everserve/state/mirror.py:916-937). The fresh cache must equal the doomed one on every block
in use, bit for bit. Also checked: each round's block ids are those the reference's planner picks,
and the tags the kernel wrote are ``block * block_size + [0, block_size)``.
"""

import random

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import notice, staging
from everserve_amd.state.restore import Restorer, Table
from tests.cases import bits

pytestmark = pytest.mark.gpu

L, NB, BS, H, D = 3, 64, 16, 3, 8
HEADS = [0, 2]


class GpuCache:
    """Block tables on the host, the KV on the GPU (kv_first bf16), written token by token."""

    def __init__(self, n_req, prompt, seed):
        self.rng = random.Random(seed)
        self.free = list(range(NB))
        self.rng.shuffle(self.free)
        self.tables = {str(i): [] for i in range(n_req)}
        self.n = {str(i): 0 for i in range(n_req)}
        self.layers = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device="cuda")
                       for _ in range(L)]
        for rid in self.tables:
            self.write(rid, prompt)

    def write(self, rid, k):
        for _ in range(k):
            pos = self.n[rid]
            if pos // BS >= len(self.tables[rid]):
                self.tables[rid].append(self.free.pop())
            b = self.tables[rid][pos // BS]
            # a token's KV depends on (request, position) only, as in the reference's mock: a
            # recomputed request writes the same values again
            g = torch.Generator().manual_seed(int(rid) * 100_003 + pos)
            vals = torch.randn((L, 2, H, D), generator=g).to(torch.bfloat16).cuda()
            for layer, t in enumerate(self.layers):
                t[:, b, pos % BS] = vals[layer]
            self.n[rid] += 1

    def preempt(self, rid):
        n = self.n[rid]
        for b in self.tables[rid]:
            for t in self.layers:
                t[:, b].zero_()
            self.free.append(b)
        self.tables[rid], self.n[rid] = [], 0
        self.rng.shuffle(self.free)
        self.write(rid, n)

    def in_use(self):
        return sorted(b for t in self.tables.values() for b in t)


def test_rounds_then_restore_rebuild_every_block_in_use(ext):
    c = GpuCache(4, 37, seed=7)
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    tables, written, tags = {}, {}, []

    def sink(job):
        if job.descriptor is None:
            return
        tags.append(list(job.descriptor["slots"]))
        # the store maps the staging file the descriptor names, in the stager's rank directory
        staged = np.memmap(st.rank_dir / job.descriptor["stage"], dtype=np.uint8, mode="r")
        oracle.store_commit(np.asarray(staged), job.descriptor, tables, NB * BS, written, job.step)

    window = notice.StagingWindow(rank=1, deadline=0.0)
    shadow = {}
    with staging.StepStager(ext, dict(zip(names, c.layers)), HEADS, sink) as st:
        for rnd in range(1, 9):
            want_ids = oracle.blocks_to_stage(c.tables, dict(c.n), shadow, BS)
            ids = st.stage_round(window, c.tables, dict(c.n), epoch=1, step=rnd)
            assert ids == want_ids
            st.flush()
            if ids:
                assert tags[-1] == oracle.expand_blocks(ids, BS).tolist()
            # the rank keeps serving: tokens, a preemption, a multi-token step
            for rid in c.n:
                c.write(rid, 1 if rnd % 3 else 17)
            if rnd == 4:
                c.preempt("2")
        ids = st.stage_round(window, c.tables, dict(c.n), epoch=1, step=9)
        st.flush()
    assert window.rounds == 9 and window.blocks_copied > 0
    # the replacement: a fresh cache written from the tables' written ranges, head for head
    fresh = [torch.zeros_like(t) for t in c.layers]
    rest = Restorer(ext, fresh)
    row_bytes = 2 * D * 2
    tabs = [Table(t, tables[t], oracle.written_ranges(written[t])) for t in sorted(tables)]
    assert all(tb.rows.nbytes == NB * BS * row_bytes for tb in tabs)
    rest.restore(tabs, {h: h for h in HEADS})
    use = torch.tensor(c.in_use(), device="cuda")
    for src, dst in zip(c.layers, fresh):
        for h in HEADS:
            assert np.array_equal(bits(dst[:, use, :, h]), bits(src[:, use, :, h]))
        # head slots not held stay untouched
        assert not dst[:, :, :, 1].any()
