"""Notice rounds on the GPU: a doomed rank's cache staged block round by block round, then restored.

A decoding batch (test_oracle_staging.Batch's block bookkeeping) writes its KV into a GPU cache,
every layer and head slot, while rounds copy the blocks that changed (the plan of
core/everserve/reference/staging.py:51-94). Each round goes through the product path:
1. ``StepStager.stage_round`` plans the round and gathers the blocks with the slot tags.
2. The rows are delivered into the round's staging file in the rank directory.
3. The oracle's store commit maps that file by its name and copies the rows into tables
   (store/src/storage.rs:864-957).

After the last round the product ``Restorer`` writes the tables' written ranges into a fresh cache
(core/everserve/state/mirror.py:916-937). The fresh cache must equal the doomed one on every block
in use, bit for bit. Also checked: each round's block ids are those the oracle's planner picks,
and the tags the kernel wrote are ``block * block_size + [0, block_size)``.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import notice, staging
from everserve_amd.state.restore import Restorer, Table
from tests.cases import bits
from tests.test_oracle_staging import BLOCK as BS
from tests.test_oracle_staging import Batch

pytestmark = pytest.mark.gpu

L, NB, H, D = 3, 64, 3, 8
HEADS = [0, 2]


class GpuBatch(Batch):
    """The batch's KV in a kv_first bf16 cache on the GPU: a token's values for every layer and
    head slot are drawn from a generator seeded by its (request, generation, position) value, so
    a recomputed request writes new values."""

    def __init__(self, prompts, seed):
        self.layers = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device="cuda")
                       for _ in range(L)]
        super().__init__(prompts, seed, pool_blocks=NB)

    def on_token(self, b, offset, r, t):
        super().on_token(b, offset, r, t)
        g = torch.Generator().manual_seed(self.value(r, t) % (1 << 62))
        vals = torch.randn((L, 2, H, D), generator=g).to(torch.bfloat16).cuda()
        for layer, cache in enumerate(self.layers):
            cache[:, b, offset] = vals[layer]

    def release(self, r):
        for b in self.blocks[r]:
            for cache in self.layers:
                cache[:, b].zero_()
        super().release(r)


def test_rounds_then_restore_rebuild_every_block_in_use(ext):
    c = GpuBatch({"a": 29, "b": 50, "c": 8, "d": 33}, seed=7)
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
            want_ids = oracle.blocks_to_stage(c.blocks, dict(c.length), shadow, BS)
            ids = st.stage_round(window, c.blocks, dict(c.length), epoch=1, step=rnd)
            assert ids == want_ids
            st.flush()
            if ids:
                assert tags[-1] == oracle.expand_blocks(ids, BS).tolist()
            # the rank keeps serving: tokens, a preemption, a multi-token step
            for r in c.length:
                c.append(r, 1 if rnd % 3 else 17)
            if rnd == 4:
                c.recompute("c")
        ids = st.stage_round(window, c.blocks, dict(c.length), epoch=1, step=9)
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
