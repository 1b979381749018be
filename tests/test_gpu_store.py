"""The whole per-worker path on the GPU, product code end to end, the oracle only as the checker.

1. A rank's steps are staged by StepStager: the gather kernel, then the delivery of the rows
   into a staging file in shared memory.
2. They are committed by StoreTables, the store's commit copy with per-row CRC32C, on host
   threads.
3. A spare's fresh cache is rebuilt from the store's written ranges by the Restorer: host gather,
   H2D, then the scatter kernel.

Every written slot's rows in the spare's cache must equal the source's, at the head slots the
restore maps them to. The checksums the store recorded must be the oracle's CRC32C of those rows.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import staging
from everserve_amd.state.restore import Restorer
from everserve_amd.state.store import StoreTables
from tests.cases import caches, strides_of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("layout", ["kv_first", "combined"])
def test_stage_commit_restore_round_trip(ext, layout):
    L, nb, bs, h, d = 3, 32, 4, 3, 8
    cpu = caches(layout, d, torch.bfloat16, n_layers=L, nb=nb, bs=bs, h=h, seed=71)
    gpu = [t.cuda() for t in cpu]
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    held = [0, 2]
    store = StoreTables(ext, nb * bs, threads=4)
    steps = [[5, 6, 7, -1, 100], list(range(40, 60)), [3, 2, 1, 127]]
    with staging.StepStager(ext, dict(zip(names, gpu)), held, store.sink) as st:
        for k, slots in enumerate(steps, start=1):
            sl = torch.tensor(slots, dtype=torch.long, device="cuda")
            for name, t in zip(names, gpu):
                st.save(name, t, sl)
            st.commit(1, k, {})
        st.flush()
    live = sorted({s for sl in steps for s in sl if s >= 0})
    fresh = [torch.zeros_like(t) for t in gpu]
    moves = {0: 1, 2: 0}
    rows = Restorer(ext, fresh, chunk_bytes=1024).restore(store.restore_tables(), moves)
    assert rows == len(live) * L * len(held)
    back = [t.cpu() for t in fresh]
    for theirs, ours in moves.items():
        got = oracle.gather_rows(back, live, [ours], len(live), d, bs, strides_of(back[0]), 2)
        want = oracle.gather_rows(cpu, live, [theirs], len(live), d, bs, strides_of(cpu[0]), 2)
        assert np.array_equal(got, want), (theirs, ours)
    for layer in range(L):
        for head in held:
            t = store.tables[layer * 1000 + head]
            table_rows = np.asarray(t.rows).reshape(nb * bs, -1)
            assert np.array_equal(t.crc[live], oracle.crc32c_rows(table_rows[live]))
            assert not t.crc[[s for s in range(nb * bs) if s not in live]].any()
