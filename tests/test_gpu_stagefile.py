"""The step's staging files on the GPU: rows delivered into shared-memory files the store maps by
name, and fp8 per-layer scales carried beside the rows.

* ``evs_deliver_rows`` copies device rows into memory that is not pinned (a heap array, a
  ``/dev/shm`` mapping) through two pinned bounce buffers: runs smaller and larger than a bounce
  buffer, with pitches on both sides, byte for byte, and the gaps between runs untouched.
* ``StepStager`` writes each step into ``<rank_dir>/<prefix><k>.rows``; a store that opens that
  file by the descriptor's ``stage`` name (as store/src/shm.rs:39-45 maps it) and commits it with
  the oracle's restatement of the store's copy (store/src/storage.rs:864-957) gets the oracle's
  tables. At most depth + 1 files exist; closing the stager deletes them.
* C3, the Llama-3-70B one-rank share in fp8-e4m3 with per-layer scales U(0.01, 0.1) and values
  fp8(N(0, 1) / s_l): 2048 blocks staged as a notice round, committed by StoreTables, restored by
  the Restorer into a fresh cache. Every byte of every restored block is the source's (the rows
  move raw: the NaN and saturation codes too), and the scales come back exactly.
"""

import os
import stat

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.state import staging
from everserve_amd.state.restore import Restorer
from everserve_amd.state.store import StoreTables
from tests.cases import bits, caches, fp8_scaled_layers, strides_of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("runs,run_bytes,pitch,bounce", [
    (1, 1000, 1000, 64),            # one run, many batches of one piece
    (37, 5000, 8192, 16384),        # three runs a batch
    (5, 100000, 100032, 4096),      # each run cut into pieces
    (256, 32768, 65536, 32 << 20),  # a decode step's shape: one batch
    (3, 64, 128, 64),               # a run exactly a bounce buffer
    (1, 4096, 64, 1024),            # one run: its pitch, smaller than the run, is not used
    # the last batch split into 1/2, 1/4, 1/8, 1/8: by bytes within 3 runs of an odd length,
    # by bytes after two full batches, and by runs
    (3, (3 << 20) + 100, (3 << 20) + 128, 16 << 20),
    (10, 2 << 20, 2 << 20, 8 << 20),
    (20, 300000, 300032, 8 << 20),
])
def test_deliver_rows_into_memory_that_is_not_pinned(ext, runs, run_bytes, pitch, bounce):
    rng = np.random.default_rng(runs)
    span = max(pitch, run_bytes)
    src = torch.from_numpy(rng.integers(0, 256, size=runs * span, dtype=np.uint8)).cuda()
    dst = np.full(runs * span + 64, 0xEE, dtype=np.uint8)  # heap memory, pageable
    pitch = span if runs > 1 else pitch
    bufs = [torch.empty(bounce, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    ext.deliver_rows(dst.ctypes.data, pitch, src.data_ptr(), pitch, runs, run_bytes,
                     [b.data_ptr() for b in bufs], bounce, stream, 4)
    want = src.cpu().numpy().reshape(runs, span)
    got = dst[:runs * span].reshape(runs, span)
    assert np.array_equal(got[:, :run_bytes], want[:, :run_bytes])
    assert (got[:, run_bytes:] == 0xEE).all() and (dst[runs * span:] == 0xEE).all()


def test_deliver_rows_refuses_bad_arguments(ext):
    from everserve_amd.kernels import KernelError

    src = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    dst = np.zeros(1024, dtype=np.uint8)
    b = [torch.empty(128, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    s = torch.cuda.current_stream()
    ptrs = [x.data_ptr() for x in b]
    with pytest.raises(KernelError, match="multiple of 64"):
        ext.deliver_rows(dst.ctypes.data, 512, src.data_ptr(), 512, 2, 512, ptrs, 100, s)
    with pytest.raises(KernelError, match="must differ"):
        ext.deliver_rows(dst.ctypes.data, 512, src.data_ptr(), 512, 2, 512, [ptrs[0]] * 2, 128, s)
    with pytest.raises(KernelError, match="pitches"):
        ext.deliver_rows(dst.ctypes.data, 256, src.data_ptr(), 512, 2, 512, ptrs, 128, s)
    ext.deliver_rows(dst.ctypes.data, 512, src.data_ptr(), 512, 0, 512, ptrs, 128, s)  # nothing


NB, BS, H, D = 16, 4, 3, 8
HEADS = [0, 2]


def names(n):
    return [f"model.layers.{i}.self_attn.attn" for i in range(n)]


def test_steps_land_in_files_the_store_maps_by_name(ext, tmp_path):
    L = 3
    cpu = caches("kv_first", D, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=23)
    gpu = [t.cuda() for t in cpu]
    kv = dict(zip(names(L), gpu))
    rank_dir = tmp_path / "rank0"
    rank_dir.mkdir()
    steps = [[5, -1, 17, 0, 27], list(range(40, 52)), [63, 1, -1, 2], list(range(9, 0, -1))]
    tables, written, seen = {}, {}, []

    def store(job):
        desc = job.descriptor
        path = rank_dir / desc["stage"]  # the store knows only the rank directory and the name
        assert job.stage_path == path
        mode = stat.S_IMODE(os.stat(path).st_mode)
        assert mode == 0o660, oct(mode)
        mapped = np.memmap(path, dtype=np.uint8, mode="r")
        seen.append((desc["stage"], len(os.listdir(rank_dir))))
        oracle.store_commit(np.asarray(mapped), desc, tables, NB * BS, written, job.step)

    states = []
    with staging.StepStager(ext, kv, HEADS, store, depth=1, stage_prefix="s7_",
                            rank_dir=rank_dir, bounce_bytes=256) as st:
        for k, slots in enumerate(steps, start=1):
            states.append([t.clone() for t in cpu])
            sl = torch.tensor(slots, dtype=torch.long, device="cuda")
            for name, t in kv.items():
                st.save(name, t, sl)
            st.commit(1, k, {})
            for t in gpu:
                t.neg_()
            for t in cpu:
                t.neg_()
        st.flush()
        # the pool keeps at most depth + 1 files, and only pooled files are left
        pooled = sorted(x.name for x in st._pool)
        assert len(pooled) <= 2 and sorted(os.listdir(rank_dir)) == pooled
    assert all(name.startswith("s7_") and name.endswith(".rows") for name, _ in seen)
    assert os.listdir(rank_dir) == []  # closing deleted them; the directory was the caller's
    want_tables, want_written = {}, {}
    for k, (state, slots) in enumerate(zip(states, steps), start=1):
        cap = staging.capacity_for(len(slots))
        rows = oracle.gather_rows(state, slots, HEADS, cap, D, BS, strides_of(state[0]), 2)
        desc = oracle.staged_step("x", range(L), HEADS, cap, D, 2, slots, "bfloat16")
        oracle.store_commit(rows.view(np.uint8).reshape(-1), desc, want_tables, NB * BS,
                            want_written, k)
    assert sorted(tables) == sorted(want_tables)
    for t in want_tables:
        assert np.array_equal(tables[t], want_tables[t]), t


def test_the_stagers_own_directory_goes_at_close(ext):
    gpu = [t.cuda() for t in caches("kv_first", D, torch.bfloat16, n_layers=2, nb=NB, h=H)]
    st = staging.StepStager(ext, dict(zip(names(2), gpu)), HEADS, lambda job: None)
    d = st.rank_dir
    sl = torch.tensor([1, 2, 3], dtype=torch.long, device="cuda")
    for name, t in zip(names(2), gpu):
        st.save(name, t, sl)
    st.commit(0, 1, {})
    st.flush()
    assert d.is_dir() and any(d.iterdir())
    st.close()
    assert not d.exists()


def test_c3_fp8_share_with_scales_through_the_stager_the_store_and_a_restore(ext, tmp_path):
    """C3 at full size: 80 layers of [2, 8192, 16, 1, 128] fp8-e4m3, 2048 blocks in one notice
    round (640 MiB of rows through one staging file), the store's tables, and a fresh cache."""
    L, nb, bs, h, d = 80, 8192, 16, 1, 128
    layers, scales = fp8_scaled_layers(L, (2, nb, bs, h, d), seed=3)
    dev_scales = torch.from_numpy(scales).cuda()
    blocks = np.random.default_rng(3).permutation(nb)[:2048]
    if 0 not in blocks:
        blocks[-1] = 0  # the block holding every byte code
    kv = dict(zip(names(L), layers))
    store = StoreTables(ext, nb * bs, threads=16)
    tails = []

    def sink(job):
        store.sink(job)
        tail = np.memmap(job.stage_path, dtype=np.float32, mode="r",
                         offset=job.descriptor["layer_stride"] * L, shape=(L,))
        tails.append(np.array(tail))

    with staging.StepStager(ext, kv, [0], sink, rank_dir=tmp_path, scales=dev_scales) as st:
        n = st.commit_blocks(1, 1, blocks.tolist())
        st.flush()
        dev_scales.mul_(2)  # a later change must not reach the committed step
    assert n == 2048 * bs
    assert np.array_equal(tails[0], scales) and np.array_equal(store.scales, scales)
    fresh = [torch.zeros_like(t) for t in layers]
    fresh_scales = torch.zeros(L, dtype=torch.float32, device="cuda")
    rows = Restorer(ext, fresh, scales=fresh_scales).restore(
        store.restore_tables(), {0: 0}, scales=store.restore_scales())
    assert rows == 2048 * bs * L
    assert np.array_equal(fresh_scales.cpu().numpy(), scales)
    b = torch.from_numpy(blocks).cuda()
    keep = torch.ones(nb, dtype=torch.bool, device="cuda")
    keep[b] = False
    for li in range(L):
        src, dst = layers[li].view(torch.uint8), fresh[li].view(torch.uint8)
        assert torch.equal(dst[:, b], src[:, b]), li
        assert not dst[:, keep].any(), li
    # the NaN and saturation codes were among the bytes, where a staged block holds them
    codes = layers[0].view(torch.uint8).view(-1)[:256].cpu().numpy()
    assert codes.tolist() == list(range(256))


def test_closing_with_a_step_saved_but_not_committed_leaves_no_file(ext, tmp_path):
    gpu = [t.cuda() for t in caches("kv_first", D, torch.bfloat16, n_layers=2, nb=NB, h=H)]
    st = staging.StepStager(ext, dict(zip(names(2), gpu)), HEADS, lambda job: None,
                            rank_dir=tmp_path)
    sl = torch.tensor([1, 2, 3], dtype=torch.long, device="cuda")
    st.save(names(2)[0], gpu[0], sl)  # the step's file exists from its first save
    assert len(os.listdir(tmp_path)) == 1
    st.close()
    assert os.listdir(tmp_path) == []


def _store_process(rank_dir, conn, num_slots):
    """A store in its own process: it knows the rank directory, maps each staging file by the
    descriptor's name, commits it (the oracle's restatement of storage.rs:864-957) and answers
    when done, as the store acknowledges a commit. It never touches the GPU."""
    import os

    import numpy as np

    import oracle

    tables, written = {}, {}
    while True:
        msg = conn.recv()
        if msg is None:
            break
        step_no, desc = msg
        staged = np.memmap(os.path.join(rank_dir, desc["stage"]), dtype=np.uint8, mode="r")
        oracle.store_commit(np.asarray(staged), desc, tables, num_slots, written, step_no)
        del staged
        conn.send("ok")
    conn.send({t: (rows.tobytes(), written[t].tobytes()) for t, rows in tables.items()})


def test_a_store_in_another_process_maps_the_staging_files_by_name(ext, tmp_path):
    import multiprocessing as mp

    L = 2
    cpu = caches("blocks_first", D, torch.bfloat16, n_layers=L, nb=NB, h=H, seed=29)
    gpu = [t.cuda() for t in cpu]
    kv = dict(zip(names(L), gpu))
    ctx = mp.get_context("spawn")
    here, there = ctx.Pipe()
    proc = ctx.Process(target=_store_process, args=(str(tmp_path), there, NB * BS))
    proc.start()
    steps = [[3, 4, 5, -1], list(range(20, 40)), [63, 0, 1]]
    try:
        def sink(job):  # only the descriptor crosses: the rows are in the named file
            here.send((job.step, job.descriptor))
            assert here.recv() == "ok"  # the store has taken the step: the file may be reused

        with staging.StepStager(ext, kv, HEADS, sink, depth=1, rank_dir=tmp_path) as st:
            for k, slots in enumerate(steps, start=1):
                sl = torch.tensor(slots, dtype=torch.long, device="cuda")
                for name, t in kv.items():
                    st.save(name, t, sl)
                st.commit(1, k, {})
            st.flush()
        here.send(None)
        got = here.recv()
    finally:
        proc.join(timeout=60)
        if proc.is_alive():
            proc.terminate()
    want_tables, want_written = {}, {}
    for k, slots in enumerate(steps, start=1):
        cap = staging.capacity_for(len(slots))
        rows = oracle.gather_rows(cpu, slots, HEADS, cap, D, BS, strides_of(cpu[0]), 2)
        desc = oracle.staged_step("x", range(L), HEADS, cap, D, 2, slots, "bfloat16")
        oracle.store_commit(rows.view(np.uint8).reshape(-1), desc, want_tables, NB * BS,
                            want_written, k)
    assert sorted(got) == sorted(want_tables)
    for t in want_tables:
        assert got[t][0] == want_tables[t].tobytes(), t
        assert got[t][1] == want_written[t].tobytes(), t
