"""The step path (StepStager) on the GPU, end to end through the store's commit, against the oracle.

What the reference's step path does (core/everserve/state/mirror.py:536-800): save per layer, one
gather per step, a descriptor per step. The test runs it and commits every staged step into
tables with the oracle's restatement of the store's copy (store/src/storage.rs:864-957). It then
asks for tables equal byte for byte to those the oracle builds from the cache as it stood at each
commit. The other cases are:

* padding ids;
* a step of only some layers (mirror.py:699-704);
* a later step of another size, on a pooled buffer of another capacity;
* a cache that the next "forward" changes on the same stream straight after the commit (the
  rows staged are the ones before the change);
* a sink that fails, which surfaces on the step thread;
* save and commit never reading device memory or waiting on the device on the step thread.

Each step's descriptor is also checked against the oracle's.
"""

import threading

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import staging
from tests.cases import bits, caches, strides_of

pytestmark = pytest.mark.gpu

NB, BS, H, D = 16, 4, 3, 8
HEADS = [0, 2]
NUM_SLOTS = NB * BS


def names(n):
    return [f"model.layers.{i}.self_attn.attn" for i in range(n)]


class Store:
    """The oracle's store: tables filled by every staged step the sink receives."""

    def __init__(self):
        self.tables, self.written, self.descriptors = {}, {}, []
        self.lock = threading.Lock()

    def __call__(self, job):
        if job.descriptor is None:
            return
        with self.lock:
            self.descriptors.append((job.step, job.descriptor))
            oracle.store_commit(job.stage_bytes, job.descriptor, self.tables, NUM_SLOTS,
                                self.written, job.step)


def expected(cpu_layers, steps):
    """The tables the oracle builds: gather each step's rows from the cache as committed."""
    tables, written = {}, {}
    e = cpu_layers[0][0].element_size()
    for step_no, (state, slots, layers) in enumerate(zip(cpu_layers, *zip(*steps)), start=1):
        cap = staging.capacity_for(len(slots))
        rows = oracle.gather_rows(state, slots, HEADS, cap, D, BS, strides_of(state[0]), e)
        desc = oracle.staged_step("x", layers, HEADS, cap, D, e, slots, "bfloat16")
        oracle.store_commit(rows.view(np.uint8).reshape(-1), desc, tables, NUM_SLOTS, written,
                            step_no)
    return tables


def test_steps_land_in_the_store_as_the_oracle_puts_them(ext):
    L = 3
    cpu = caches("kv_first", D, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=21)
    gpu = [t.cuda() for t in cpu]
    kv = dict(zip(names(L), gpu))
    steps = [  # slots, layers saved
        ([5, -1, 17, 0, 27], [0, 1, 2]),
        (list(range(40, 52)), [0, 1, 2]),
        ([63, 1, -1, 2], [0, 2]),
        ([9, 8, 7, 6, 5, 4, 3, 2, 1], [0, 1, 2]),
    ]
    store = Store()
    states = []
    with staging.StepStager(ext, kv, HEADS, store, depth=2) as st:
        for step_no, (slots, layers) in enumerate(steps, start=1):
            states.append([t.clone() for t in cpu])
            sl = torch.tensor(slots, dtype=torch.long, device="cuda")
            for layer in layers:
                st.save(names(L)[layer], gpu[layer], sl)
            st.commit(epoch=1, step=step_no, committed_tokens={"r": step_no})
            # the next forward rewrites every element on the same stream, at once
            for t in gpu:
                t.neg_()
            for t in cpu:
                t.neg_()
        st.flush()
        assert st.stats["steps"] == len(steps)
        row_bytes = 2 * D * 2
        assert st.stats["bytes_sent"] == sum(
            sum(1 for x in slots if x >= 0) * len(layers) * len(HEADS) * row_bytes
            for slots, layers in steps)
        assert st.stats["bytes_staged"] == sum(
            len(slots) * len(layers) * len(HEADS) * row_bytes for slots, layers in steps)
    want = expected(states, steps)
    assert sorted(store.tables) == sorted(want)
    for table in want:
        assert np.array_equal(store.tables[table], want[table]), table
    for (step_no, desc), (slots, layers) in zip(sorted(store.descriptors,
                                                       key=lambda x: x[0]), steps):
        cap = staging.capacity_for(len(slots))
        ref = oracle.staged_step(desc["stage"], layers, HEADS, cap, D, 2, slots, "bfloat16")
        assert desc == ref


def test_save_and_commit_never_read_device_memory_on_the_step_thread(ext, monkeypatch):
    """The reference's rule (core/tests/test_mirror_client.py:345-375): reading a tensor on the
    host from the step thread drains the GPU, a forward pass paid inside commit(). Every host-side
    read of a tensor (cpu, tolist, item, numpy, bool) and every host wait on the device
    (torch.cuda.synchronize, a stream's or event's synchronize, the library's event wait) is
    forbidden on the step thread while steps and a block round are saved and committed; the copy
    thread does all of them. The sink still gets every step, padding ids included."""
    L = 2
    gpu = [t.cuda() for t in caches("kv_first", D, torch.bfloat16, n_layers=L, nb=NB, h=H,
                                    seed=29)]
    kv = dict(zip(names(L), gpu))
    store = Store()
    st = staging.StepStager(ext, kv, HEADS, store, depth=2)
    steps = [[3, 9, -1], list(range(20, 33)), [0, 63]]
    slot_tensors = [torch.tensor(s, dtype=torch.long, device="cuda") for s in steps]
    torch.cuda.synchronize()
    step_thread = threading.current_thread()

    def forbid(owner, name):
        real = getattr(owner, name)

        def guarded(*args, **kwargs):
            if threading.current_thread() is step_thread:
                raise AssertionError(f"{name} on the step thread")
            return real(*args, **kwargs)

        monkeypatch.setattr(owner, name, guarded)

    for name in ("cpu", "tolist", "item", "numpy", "__bool__"):
        forbid(torch.Tensor, name)
    forbid(torch.cuda, "synchronize")
    forbid(torch.cuda.Stream, "synchronize")
    forbid(torch.cuda.Event, "synchronize")
    forbid(ext, "event_synchronize")
    for step_no, sl in enumerate(slot_tensors, start=1):
        for name, t in kv.items():
            st.save(name, t, sl)
        st.commit(epoch=1, step=step_no, committed_tokens={"r": step_no})
    st.commit_blocks(epoch=1, step=len(steps) + 1, block_ids=[5, 2])
    st.flush()
    monkeypatch.undo()
    st.close()
    got = {step: desc["slots"] for step, desc in store.descriptors}
    assert got == {1: steps[0], 2: steps[1], 3: steps[2],
                   4: [5 * BS + i for i in range(BS)] + [2 * BS + i for i in range(BS)]}


def test_the_llama_shaped_decode_step(ext):
    """32 layers of [2, 512, 16, 8, 128] bf16, 64 decode slots: every row staged and committed."""
    L, nb, bs, h, d = 32, 512, 16, 8, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    gpu = [torch.randn((2, nb, bs, h, d), generator=g, device="cuda").to(torch.bfloat16)
           for _ in range(L)]
    kv = dict(zip(names(L), gpu))
    heads = list(range(h))
    slots = (torch.randperm(nb * bs, generator=torch.Generator().manual_seed(6))[:64]).tolist()
    got = {}

    def sink(job):
        if job.descriptor is not None:
            got["desc"] = job.descriptor
            got["bytes"] = job.stage_bytes.copy()

    with staging.StepStager(ext, kv, heads, sink) as st:
        sl = torch.tensor(slots, dtype=torch.long, device="cuda")
        for name, t in kv.items():
            st.save(name, t, sl)
        st.commit(0, 1, {})
        st.flush()
    cap = staging.capacity_for(64)
    rows = got["bytes"].view(np.uint16).reshape(L, h, cap, 2, d)[:, :, :64]
    idx = torch.tensor(slots, device="cuda")
    for layer in (0, 17, 31):
        t = gpu[layer]
        # kv_first: [2, nb, bs, h, d]; the rows of head j are t[:, s // bs, s % bs, j]
        want = t[:, idx // bs, idx % bs].permute(2, 1, 0, 3)  # [h, n, 2, d]
        assert np.array_equal(rows[layer], bits(want))
    assert got["desc"] == oracle.staged_step(got["desc"]["stage"], range(L), heads, cap, d, 2,
                                             slots, "bfloat16")


def test_a_failing_sink_surfaces_on_the_step_thread(ext):
    gpu = [t.cuda() for t in caches("kv_first", D, torch.bfloat16, n_layers=2, nb=NB, h=H)]
    kv = dict(zip(names(2), gpu))

    def sink(job):
        raise OSError("the store is gone")

    st = staging.StepStager(ext, kv, HEADS, sink)
    try:
        sl = torch.tensor([1, 2], dtype=torch.long, device="cuda")
        for name, t in kv.items():
            st.save(name, t, sl)
        st.commit(0, 1, {})
        with pytest.raises(staging.StagingError, match="the store is gone"):
            st.fence(1)
        with pytest.raises(staging.StagingError):
            st.save(names(2)[0], gpu[0], sl)
    finally:
        st.close()


def test_pooled_buffers_are_reused(ext):
    gpu = [t.cuda() for t in caches("kv_first", D, torch.bfloat16, n_layers=2, nb=NB, h=H)]
    kv = dict(zip(names(2), gpu))
    seen = []
    with staging.StepStager(ext, kv, HEADS, lambda j: seen.append(j.descriptor["stage"]),
                            depth=1) as st:
        for step in range(1, 7):
            sl = torch.tensor([step, step + 1, 30], dtype=torch.long, device="cuda")
            for name, t in kv.items():
                st.save(name, t, sl)
            st.commit(0, step, {})
        st.flush()
    assert len(seen) == 6
    assert len(set(seen)) <= 2  # depth + 1 pairs at most


def test_prepared_files_serve_the_first_steps_of_their_sizes(ext):
    """prepare makes the pooled file of a size before any step: the first step of that size
    takes it (no file is made then) and lands as the oracle puts it; a size not prepared makes
    its own; more sizes than the pool keeps are made and dropped again."""
    cpu = caches("kv_first", D, torch.bfloat16, n_layers=2, nb=NB, h=H, seed=31)
    gpu = [t.cuda() for t in cpu]
    kv = dict(zip(names(2), gpu))
    store = Store()
    with staging.StepStager(ext, kv, HEADS, store, depth=1) as st:
        st.prepare([3, 20])
        made = sorted(p.name for p in st.rank_dir.iterdir())
        assert len(made) == 2 and st._stage_seq == 2
        steps = [([5, 6, 7], [0, 1]), (list(range(20, 40)), [0, 1]), ([1, 2, 3, 4, 9], [0, 1]),
                 (list(range(10, 50)), [0, 1])]
        for step, (slots, layers) in enumerate(steps, start=1):
            sl = torch.tensor(slots, dtype=torch.long, device="cuda")
            for name, t in kv.items():
                st.save(name, t, sl)
            st.commit(0, step, {})
            st.flush()
            # 3 and 5 slots take the capacity-8 file, 20 the capacity-32 one; 40 makes its own
            assert st._stage_seq == (2 if step < 4 else 3)
        with pytest.raises(ValueError, match="slots"):
            st.prepare([-1])
        st.prepare([100, 200, 300, 400])  # depth 1: the pool keeps 2
        assert len(st._pool) <= 2
    want = expected([cpu] * 4, steps)
    assert sorted(store.tables) == sorted(want)
    for table in want:
        assert np.array_equal(store.tables[table], want[table]), table
