"""Benchmark of the per-worker KV data path on one MI355X; prints ONE JSON line.

Headline (``value``): the KV snapshot gather at the Llama-3-8B shape (
"C2"): 32 layers of a kv_first bf16 cache [2, 8192, 16, 8, 128] filled N(0, 1), 1024 blocks
chosen by seeded block tables of 64 sequences (16,384 slots), every one of the 8 KV heads, gathered
by ``gather_rows`` into a [32, 8, 16384, 2, 128] staging buffer in HBM. One step = one launch.
Throughput counts the algorithmic bytes, read plus write: 2 * 32 * 8 * 16384 * 512 B = 4 GiB.

``roofline`` is that kernel's HBM roofline: algorithmic bytes per launch over its average
duration, timed with HIP events around each launch on the stream it runs on, against 8 TB/s.
``traffic`` is the HBM bytes per launch that rocprofv3's FETCH_SIZE and WRITE_SIZE counters
measured (profiles/gather_c2_llama3_8b_pmc.txt), or null when that profile is absent.

``cpu_baseline`` is the reference's CPU path, the torch gather per layer of
core/everserve/state/mirror.py:552-562 restated in oracle/cpu_path.py, timed on this host's cores
over a bounded sample of the same workload (4 of the 32 layers, the same 1024 blocks).

``extra`` carries the other configs' figures, each measured the same way: the block-table gather
(C2 via ``gather_blocks``), the fp8 70B share with its D2H copy to pinned memory (C3), the restore
scatter (C4), the local reduction (C5), and the µs a per-step snapshot adds to a Llama-3-8B
decode-step proxy. Data is synthetic.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--quick] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PEAK_HBM_GBS = 8000.0
GIB = 1 << 30
PMC_PROFILE = ROOT / "profiles" / "gather_c2_llama3_8b_pmc.txt"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------ helpers
def layout_strides(t):
    from everserve_amd.state.paged import PagedKV

    return list(PagedKV.of(t).layout_strides(t))


def random_cache_layers(n_layers, shape, dtype, device, seed):
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    return [torch.empty(shape, dtype=dtype, device=device).normal_(generator=g)
            for _ in range(n_layers)]


def block_table_slots(num_blocks_cache, num_blocks, block_size, seed):
    """Slots of ``num_blocks`` distinct blocks from a seeded permutation, block after block."""
    import numpy as np

    blocks = np.random.default_rng(seed).permutation(num_blocks_cache)[:num_blocks]
    slots = (blocks[:, None] * block_size + np.arange(block_size)[None, :]).reshape(-1)
    return blocks.astype(np.int32), slots.astype(np.int64)


def time_launches(fn, steps, warmup, stream):
    """Per-launch durations (ms) from HIP events recorded on ``stream`` around each launch."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, wall


def pinned_copy_gbs(nbytes, to_host, repeats=5):
    """GB/s of a plain copy between pinned host memory and HBM (torch's copy of a contiguous
    tensor, one hipMemcpyAsync): the measured ceiling the PCIe-bound copies are set against."""
    import torch

    dev = torch.device("cuda", 0)
    d = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    h = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)

    def copy():
        if to_host:
            h.copy_(d, non_blocking=True)
        else:
            d.copy_(h, non_blocking=True)

    per, _ = time_launches(copy, repeats, 1, torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    del d, h
    return nbytes / (sum(per) / len(per)) / 1e6


_SETTLE = {"probe": None, "idle_ms": None, "waited_s": 0.0}


def settle_device(ext):
    """Return torch's cached device memory to the driver, then wait until the copy engines are
    free again before the next leg times anything. The driver clears released device memory in
    the background on a copy engine: after 48 GiB was released, a pitched device-to-host copy ran
    at 15 GB/s for about a second, where it runs at 56 GB/s otherwise. The wait ends when a probe
    copy (32 MiB, pitched) runs within 25 % of its time on the idle device, or after 10 s; the
    time waited is reported (``extra.settle_s``)."""
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if _SETTLE["probe"] is None:  # made once, at the first call, on the idle device
        _SETTLE["probe"] = (torch.empty(64 << 20, dtype=torch.uint8, device=dev),
                            torch.empty(64 << 20, dtype=torch.uint8, pin_memory=True))
    d, h = _SETTLE["probe"]

    def probe_ms():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ext.copy_rows_async(h.data_ptr(), d.data_ptr(), 64, 512 << 10, 1 << 20, dev)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    if _SETTLE["idle_ms"] is None:
        probe_ms()
        _SETTLE["idle_ms"] = min(probe_ms() for _ in range(3))
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 10.0 and probe_ms() > 1.25 * _SETTLE["idle_ms"]:
        time.sleep(0.05)
    _SETTLE["waited_s"] += time.perf_counter() - t0


def pmc_traffic():
    """HBM bytes per launch from the committed rocprofv3 counter profile (its latest
    measurement: the last traffic line), or None."""
    if not PMC_PROFILE.is_file():
        return None
    found = re.findall(r"^traffic_bytes_per_launch:\s*([0-9.]+)", PMC_PROFILE.read_text(), re.M)
    return float(found[-1]) if found else None


# ------------------------------------------------------------------------------ C2 gather
def bench_c2(ext, steps, warmup, blocks_too=True):
    import torch

    L, NB, BS, H, D = 32, 8192, 16, 8, 128
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    log(f"C2: allocating {L} x [2, {NB}, {BS}, {H}, {D}] bf16 ({L * 2 * NB * BS * H * D * 2 / GIB:.0f} GiB)")
    layers = random_cache_layers(L, (2, NB, BS, H, D), torch.bfloat16, dev, seed=0)
    blocks, slots = block_table_slots(NB, 1024, BS, seed=2)
    n = len(slots)
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device=dev)
    s = torch.from_numpy(slots).to(dev)
    b = torch.from_numpy(blocks).to(dev)
    heads = torch.arange(H, dtype=torch.long, device=dev)
    out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device=dev)
    strides = layout_strides(layers[0])
    payload = L * H * n * 2 * D * 2
    algo = 2 * payload

    def gather():
        ext.gather_rows(ptrs, s, heads, out.data_ptr(), n, D, BS, strides, 2)

    per, wall = time_launches(gather, steps, warmup, stream)
    res = {"per_launch_ms": per, "wall_s": wall, "algo_bytes": algo, "payload_bytes": payload,
           "n_slots": n}
    # a spot check of the staged rows against the cache, on the device: block 0 of the table
    b0 = int(blocks[0])
    want = layers[5][:, b0, :, 3]  # [2, 16, D] for head 3 of layer 5
    got = out[5, 3, :BS].permute(1, 0, 2)
    res["spot_check"] = bool(torch.equal(got.view(torch.int16), want.view(torch.int16)))
    if blocks_too:
        out2 = torch.empty_like(out)
        tags = torch.empty(n, dtype=torch.long, device=dev)

        def gather_blocks():
            ext.gather_blocks(ptrs, b, heads, out2.data_ptr(), n, D, BS, strides, 2, slots_out=tags)

        per_b, _ = time_launches(gather_blocks, steps, warmup, stream)
        res["blocks_per_launch_ms"] = per_b
        res["blocks_equal"] = bool(torch.equal(out.view(torch.int16), out2.view(torch.int16)))
        del out2
    del layers, out
    settle_device(ext)
    return res


def cpu_baseline_c2(seconds=10.0):
    """The reference's torch CPU path on 4 layers of the C2 workload; GB/s of algorithmic bytes."""
    import torch

    from oracle import cpu_path

    threads = torch.get_num_threads()
    L, NB, BS, H, D = 4, 8192, 16, 8, 128
    g = torch.Generator().manual_seed(0)
    layers = [torch.randn((2, NB, BS, H, D), generator=g, dtype=torch.bfloat16) for _ in range(L)]
    _, slots = block_table_slots(NB, 1024, BS, seed=2)
    s = torch.from_numpy(slots)
    heads = torch.arange(H)
    n = len(slots)
    staged = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16)
    cpu_path.gather_step(layers, s, heads, n, out=staged)  # warm
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        cpu_path.gather_step(layers, s, heads, n, out=staged)
        reps += 1
    el = time.perf_counter() - t0
    algo = 2 * L * H * n * 2 * D * 2
    return {
        "value": round(algo * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"C2 gather at 4 of 32 layers ([2,8192,16,8,128] bf16 each), the same 1024 "
                  f"blocks x 8 heads, torch rows_of_heads + copy per layer (mirror.py:552-562), "
                  f"{reps} steps in {el:.1f} s; os.cpu_count()={os.cpu_count()}, "
                  f"affinity={len(os.sched_getaffinity(0))}, torch threads={threads}",
    }


def cpu_baselines_more(seconds=5.0):
    """The reference's torch CPU path for the restore (C4, on one layer) and the reduce (C5)."""
    import numpy as np
    import torch

    from oracle import cpu_path

    threads = torch.get_num_threads()
    out = {}
    # C4: staged rows written back at a random permutation of whole blocks, every head slot
    L, NB, BS, H, D = 1, 16384, 16, 8, 128
    n = NB * BS
    staged = torch.ones((L, H, n, 2, D), dtype=torch.bfloat16)  # a copy: the values do not matter
    layers = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16) for _ in range(L)]
    perm = np.random.default_rng(4).permutation(NB).astype(np.int64)
    slots = torch.from_numpy((perm[:, None] * BS + np.arange(BS)[None, :]).reshape(-1))
    heads = list(range(H))
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < seconds:
        cpu_path.restore_step(layers, slots, heads, staged)
        reps += 1
    el = time.perf_counter() - t0
    out["c4_restore"] = {
        "value": round(2 * L * H * n * 2 * D * 2 * reps / el / 1e9, 3), "unit": "GB/s",
        "cores": threads, "kind": "port",
        "sample": f"C4 restore on 1 of 32 layers (16384-block cache, random block permutation, 8 "
                  f"heads): index_select + write_rows per (layer, head) (mirror.py:926-937), "
                  f"{reps} steps in {el:.1f} s"}
    del staged, layers
    # C5: 8 members of 2,097,152 bf16, summed in order in fp32
    K, N = 8, 256 * 8192
    members = [torch.randn(N, generator=torch.Generator().manual_seed(5 + i)).to(torch.bfloat16)
               for i in range(K)]
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < seconds:
        cpu_path.member_sum(members)
        reps += 1
    el = time.perf_counter() - t0
    out["c5_reduce"] = {
        "value": round(el / reps * 1e6, 1), "unit": "us per call", "cores": threads,
        "kind": "port",
        "sample": f"C5 member_sum of 8 x 2,097,152 bf16 (ops.py:63-73), {reps} calls in {el:.1f} s"}
    return out


# ------------------------------------------------------------------------------ C1
def bench_c1(ext, steps, warmup):
    """Config C1 (Qwen2.5-0.5B shape, the reference's CPU-runnable
    case): 24 layers of [2, 2048, 16, 2, 64] bf16, 128 random blocks, both heads. The gather on the
    GPU beside the reference's torch CPU path on the same workload (mirror.py:552-562)."""
    import numpy as np
    import torch

    from oracle import cpu_path

    L, NB, BS, H, D = 24, 2048, 16, 2, 64
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator().manual_seed(0)
    cpu_layers = [torch.randn((2, NB, BS, H, D), generator=g).to(torch.bfloat16) for _ in range(L)]
    blocks = np.random.default_rng(1).choice(NB, 128, replace=False)
    slots = (blocks[:, None] * BS + np.arange(BS)[None, :]).reshape(-1).astype(np.int64)
    n = len(slots)
    layers = [t.to(dev) for t in cpu_layers]
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device=dev)
    s = torch.from_numpy(slots).to(dev)
    heads = torch.arange(H, dtype=torch.long, device=dev)
    out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device=dev)
    strides = layout_strides(layers[0])
    algo = 2 * L * H * n * 2 * D * 2
    per, _ = time_launches(lambda: ext.gather_rows(ptrs, s, heads, out.data_ptr(), n, D, BS,
                                                   strides, 2), steps, warmup, stream)
    ms = sum(per) / len(per)
    staged = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16)
    cs, ch = torch.from_numpy(slots), torch.arange(H)
    cpu_path.gather_step(cpu_layers, cs, ch, n, out=staged)
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < 2.0:
        cpu_path.gather_step(cpu_layers, cs, ch, n, out=staged)
        reps += 1
    cpu_ms = (time.perf_counter() - t0) / reps * 1e3
    same = bool(torch.equal(out.cpu().view(torch.int16), staged.view(torch.int16)))
    return {"config": "C1 Qwen2.5-0.5B: 24 x [2, 2048, 16, 2, 64] bf16, 128 blocks, heads [0, 1]",
            "bytes": algo, "gpu_ms": round(ms, 4), "gpu_gbs": round(algo / ms / 1e6, 1),
            "cpu_ms": round(cpu_ms, 3), "cpu_gbs": round(algo / cpu_ms / 1e6, 2),
            "cpu_threads": torch.get_num_threads(), "rows_equal_cpu_path": same}


# ------------------------------------------------------------------------------ C2 per layout
def bench_c2_layouts(ext, steps, warmup):
    """The C2 gather and scatter in each of the three paged layouts (kvcopy.py:37-72), the same
    1024 blocks; the median of 3 rounds of ``steps`` launches each."""
    import torch

    L, NB, BS, H, D = 32, 8192, 16, 8, 128
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    shapes = {"kv_first": (2, NB, BS, H, D), "blocks_first": (NB, 2, BS, H, D),
              "combined": (NB, H, BS, 2 * D)}
    _, slots = block_table_slots(NB, 1024, BS, seed=2)
    n = len(slots)
    s = torch.from_numpy(slots).to(dev)
    heads = torch.arange(H, dtype=torch.long, device=dev)
    rows = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device=dev)
    algo = 2 * L * H * n * 2 * D * 2
    out = {}
    # one allocation, viewed in each layout in turn: nothing is released between layouts
    layer_elems = 2 * NB * BS * H * D
    flat = torch.empty(L * layer_elems, dtype=torch.bfloat16, device=dev)
    for name, shape in shapes.items():
        layers = [flat[i * layer_elems:(i + 1) * layer_elems].view(shape).normal_()
                  for i in range(L)]
        ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device=dev)
        strides = layout_strides(layers[0])
        g, w = [], []
        for _ in range(3):
            per, _ = time_launches(lambda: ext.gather_rows(ptrs, s, heads, rows.data_ptr(), n, D,
                                                           BS, strides, 2), steps, warmup, stream)
            g.append(algo / (sum(per) / len(per)) / 1e6)
            per, _ = time_launches(lambda: ext.scatter_rows(ptrs, s, heads, rows.data_ptr(), n, D,
                                                            BS, strides, 2), steps, warmup, stream)
            w.append(algo / (sum(per) / len(per)) / 1e6)
        out[name] = {"strides": list(strides), "gather_gbs": round(sorted(g)[1], 1),
                     "scatter_gbs": round(sorted(w)[1], 1)}
        del layers
    del flat, rows
    settle_device(ext)
    return out


# ------------------------------------------------------------------------------ store commit
def bench_store_commit(ext, steps, warmup):
    """The store's commit copy (store/src/storage.rs:864-957) of a staged step into tables of the
    C2 shape, with per-row CRC32C, on the host. It commits the C2 step (16,384 slots) and a decode
    step (64 slots) into warm tables (pages touched at creation, as the store does), on 1 thread
    and on 16. The sample is 4 of the 32 layers, 32 tables of [131072, 2, 128] bf16: GB/s does
    not depend on the table count."""
    import numpy as np

    from everserve_amd.state import staging
    from everserve_amd.state.store import StoreTables

    L, NB, BS, H, D = 4, 8192, 16, 8, 128
    rb = 2 * D * 2
    _, c2_slots = block_table_slots(NB, 1024, BS, seed=2)
    out = {"config": "4 of 32 layers: 32 tables of [131072, 2, 128] bf16 (2 GiB), warm; the C2 "
                     "step and its first 64 slots as a decode step"}
    for name, slots in (("c2_step", c2_slots), ("decode_step", c2_slots[:64])):
        n = len(slots)
        cap = staging.capacity_for(n)
        stage = np.full(L * H * cap * rb, 7, dtype=np.uint8)  # every page touched
        desc = staging.describe("s", range(L), range(H), cap, D, 2, slots.tolist(), "bfloat16")
        store = StoreTables(ext, NB * BS)
        store.commit(stage, desc, 1)  # creates (and touches) the tables
        res = {}
        for threads in (1, 16):
            store.threads = threads
            reps = max(1, min(steps, 20 if name == "c2_step" else steps))
            t0 = time.perf_counter()
            for k in range(reps):
                store.commit(stage, desc, 2 + k)
            el = (time.perf_counter() - t0) / reps
            res[f"threads_{threads}"] = {"ms": round(el * 1e3, 3),
                                         "gbs": round(L * H * n * rb / el / 1e9, 2)}
        out[name] = {"slots": n, "bytes": L * H * n * rb, **res}
        del store, stage
    return out


# ------------------------------------------------------------------------------ C3 fp8 + D2H
def bench_c3(ext, steps, warmup):
    import ctypes

    import numpy as np
    import torch

    L, NB, BS, H, D = 80, 8192, 16, 1, 128
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    # per-layer scales s_l ~ U(0.01, 0.1) and values fp8(N(0,1) / s_l), clamped to e4m3's range
    scales = torch.from_numpy(np.random.default_rng(3).uniform(0.01, 0.1, L).astype(np.float32))
    g = torch.Generator(device=dev).manual_seed(3)
    layers = [(torch.randn((2, NB, BS, H, D), generator=g, device=dev, dtype=torch.float16)
               / float(sl)).clamp_(-448, 448).to(torch.float8_e4m3fn) for sl in scales.tolist()]
    blocks, slots = block_table_slots(NB, 2048, BS, seed=3)
    n = len(slots)
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device=dev)
    s = torch.from_numpy(slots).to(dev)
    heads = torch.zeros(H, dtype=torch.long, device=dev)
    staging = torch.empty((L, H, n, 2, D), dtype=torch.uint8, device=dev)
    host = torch.empty((L, H, n, 2, D), dtype=torch.uint8, pin_memory=True)
    host_scales = torch.empty(L, dtype=torch.float32, pin_memory=True)
    dev_scales = scales.to(dev)
    strides = layout_strides(layers[0])
    payload = L * H * n * 2 * D
    row_bytes = 2 * D

    def gather():
        ext.gather_rows(ptrs, s, heads, staging.data_ptr(), n, D, BS, strides, 1)

    def d2h():
        ext.copy_rows_async(host.data_ptr(), staging.data_ptr(), L * H, n * row_bytes,
                            n * row_bytes, dev)
        host_scales.copy_(dev_scales, non_blocking=True)

    def both():
        gather()
        d2h()

    g_per, _ = time_launches(gather, steps, warmup, stream)
    c_per, _ = time_launches(d2h, max(3, steps // 4), 2, stream)
    b_per, _ = time_launches(both, max(3, steps // 4), 2, stream)
    torch.cuda.synchronize()
    ok = bool(torch.equal(host[7, 0, :BS].view(-1).cpu(),
                          staging[7, 0, :BS].view(-1).cpu()))
    # the reference's way: the gather writes the rows straight into host memory mapped for the
    # device (here hipHostMalloc'd, since registering existing memory is refused on this pool)
    host_ptr, mapped_ptr = ext.host_alloc_mapped(payload)
    try:
        def zero_copy():
            ext.gather_rows(ptrs, s, heads, mapped_ptr, n, D, BS, strides, 1)

        z_per, _ = time_launches(zero_copy, max(3, steps // 4), 2, stream)
        torch.cuda.synchronize()
        mapped = np.ctypeslib.as_array((ctypes.c_uint8 * payload).from_address(host_ptr))
        ok_zero_copy = bool(np.array_equal(mapped[:1 << 20], staging.view(-1)[:1 << 20].cpu().numpy())
                            and np.array_equal(mapped[-(1 << 20):],
                                               staging.view(-1)[-(1 << 20):].cpu().numpy()))
    finally:
        ext.host_free(host_ptr)
    z_ms = sum(z_per) / len(z_per)
    delivery = c3_file_delivery(ext, staging, L * H, n * row_bytes, dev)
    delivery["stager_round"] = c3_stager_round(ext, layers, blocks, dev)
    del layers, staging
    settle_device(ext)
    plain = pinned_copy_gbs(payload, to_host=True)
    for k in ("deliver_gbs", "deliver_16_threads_gbs", "deliver_from_own_thread_gbs",
              "pageable_copy_gbs"):
        delivery[k.replace("_gbs", "_frac_of_plain_d2h")] = round(delivery[k] / plain, 4)
    g_ms, c_ms, b_ms = (sum(x) / len(x) for x in (g_per, c_per, b_per))
    return {
        "config": "C3 Llama-3-70B one-rank share, fp8 e4m3 [2,8192,16,1,128] x 80, 2048 blocks",
        "payload_bytes": payload,
        "gather_ms": round(g_ms, 4),
        "gather_hbm_gbs": round(2 * payload / g_ms / 1e6, 1),
        "gather_frac_of_8tbs": round(2 * payload / g_ms / 1e6 / PEAK_HBM_GBS, 4),
        "d2h_ms": round(c_ms, 3),
        "d2h_pcie_gbs": round(payload / c_ms / 1e6, 2),
        "d2h_frac_of_64gbs": round(payload / c_ms / 1e6 / 64.0, 4),
        "d2h_plain_memcpy_gbs": round(plain, 2),
        "d2h_frac_of_plain_memcpy": round(payload / c_ms / 1e6 / plain, 4),
        "gather_plus_d2h_ms": round(b_ms, 3),
        "zero_copy_gather_ms": round(z_ms, 3),
        "zero_copy_gather_gbs": round(payload / z_ms / 1e6, 2),
        "zero_copy_bytes_equal": ok_zero_copy,
        "scales": "80 fp32 per-layer scales U(0.01, 0.1) copied beside the rows (not inside "
                  "them); values fp8(N(0,1) / scale)",
        "bytes_equal_after_d2h": ok,
        "staging_file": delivery,
    }


def c3_file_delivery(ext, staging, runs, run_bytes, dev, repeats=5):
    """The C3 rows from HBM into a staging file in shared memory, the store's side of the
    boundary: ``evs_deliver_rows`` (two 32 MiB pinned bounce buffers, host threads copying into
    the file), and for comparison one pageable copy straight into the file's mapping.

    Every repeat's time is kept, with the host's CPU set and threading environment, and the
    delivery's two halves are timed apart: the host copy alone (the bounce buffer into the file
    on the same threads, no copy engine at work) and the same delivery called from a thread of
    its own, as the ``StepStager``'s copy thread calls it."""
    import tempfile
    import threading

    import numpy as np
    import torch

    from everserve_amd.state.staging import _map_stage_file

    payload = runs * run_bytes
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    path = Path(shm) / f"everserve-bench-c3-{os.getpid()}.rows"
    mapping = _map_stage_file(path, payload)
    bounce_bytes = 32 << 20
    bounce = [torch.empty(bounce_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    for b in bounce:  # touched once, as the StepStager does when it is built
        b.zero_()
    side = torch.cuda.Stream(device=dev)
    view = np.frombuffer(mapping, dtype=np.uint8)
    addr = view.ctypes.data
    out = {"file": str(path.parent), "bounce_bytes": bounce_bytes,
           "host": {"cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
                    "affinity": sorted(os.sched_getaffinity(0)), "numa": host_numa(),
                    "threading_env": {k: v for k, v in sorted(os.environ.items())
                                      if k.startswith(("OMP_", "GOMP_", "KMP_", "MKL_"))}}}

    def deliver(threads):
        ext.deliver_rows(addr, run_bytes, staging.data_ptr(), run_bytes, runs, run_bytes,
                         [b.data_ptr() for b in bounce], bounce_bytes, side, threads)

    def timed(fn, key):
        times = []
        for _ in range(repeats):
            view[::1 << 20] = 0xEE
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        ms = sorted(times)[len(times) // 2] * 1e3
        out[f"{key}_ms"] = round(ms, 3)
        out[f"{key}_gbs"] = round(payload / ms / 1e6, 2)
        out[f"{key}_repeats_ms"] = [round(t * 1e3, 2) for t in times]

    try:
        torch.cuda.synchronize()
        for threads, key in ((8, "deliver"), (16, "deliver_16_threads")):
            timed(lambda: deliver(threads), key)

        def on_thread():
            th = threading.Thread(target=deliver, args=(8,))
            th.start()
            th.join()

        timed(on_thread, "deliver_from_own_thread")
        # the host half alone: the bounce buffer copied into each 32 MiB of the file in turn, on
        # the same 8 threads with the same stores, while no copy engine runs
        per = bounce_bytes >> 20

        def host_half():
            for at in range(0, payload - bounce_bytes + 1, bounce_bytes):
                ext.host_gather_ranges(bounce[0].data_ptr(), per, 1 << 20, [0], [per],
                                       addr + at, per, 8)

        timed(host_half, "host_copy_only")

        # the copy-engine half alone: the same batches into the two bounce buffers in turn
        def dma_half():
            with torch.cuda.stream(side):
                for k, at in enumerate(range(0, payload - bounce_bytes + 1, bounce_bytes)):
                    ext.copy_rows_async(bounce[k & 1].data_ptr(), staging.data_ptr() + at, 1,
                                        bounce_bytes, bounce_bytes, dev)
            side.synchronize()

        timed(dma_half, "copy_engine_only")
        out["host"]["bounce_numa_nodes"] = page_nodes([b.data_ptr() for b in bounce], bounce_bytes)
        out["host"]["file_numa_nodes"] = page_nodes([addr], payload)
        out["host"]["main_thread_cpu"] = current_cpu()
        sample = np.r_[0:1 << 20, payload - (1 << 20):payload]
        deliver(8)
        out["bytes_equal"] = bool(np.array_equal(view[sample],
                                                 staging.view(-1)[torch.from_numpy(sample).to(dev)]
                                                 .cpu().numpy()))
        # a pageable copy: the runtime stages it through its own buffers
        file_t = torch.frombuffer(mapping, dtype=torch.uint8)
        timed(lambda: file_t.copy_(staging.view(-1)), "pageable_copy")
        del file_t
    finally:
        del view
        mapping.close()
        path.unlink(missing_ok=True)
    return out


def page_nodes(ptrs, nbytes, every=1 << 20):
    """The NUMA nodes of host pages, sampled every MiB of each buffer (move_pages, which only
    reports), as {node: pages}; None where the call is unavailable."""
    import ctypes

    try:
        libc = ctypes.CDLL(None, use_errno=True)
        pages = [p + off for p in ptrs for off in range(0, nbytes, every)]
        arr = (ctypes.c_void_p * len(pages))(*pages)
        status = (ctypes.c_int * len(pages))()
        if libc.syscall(279, 0, ctypes.c_ulong(len(pages)), arr, None, status, 0) != 0:
            return None
        counts = {}
        for st in status:
            counts[str(st)] = counts.get(str(st), 0) + 1
        return counts
    except (OSError, AttributeError):
        return None


def current_cpu():
    import ctypes

    try:
        return int(ctypes.CDLL(None).sched_getcpu())
    except (OSError, AttributeError):
        return None


def host_numa():
    """The host's NUMA nodes with their CPUs, and the GPU's node, as sysfs reports them."""
    out = {}
    base = Path("/sys/devices/system/node")
    for node in sorted(base.glob("node[0-9]*")) if base.is_dir() else []:
        try:
            out[node.name] = (node / "cpulist").read_text().strip()
        except OSError:
            pass
    for card in sorted(Path("/sys/class/drm").glob("card[0-9]*/device/numa_node")):
        try:
            out[f"{card.parent.parent.name}_numa_node"] = card.read_text().strip()
        except OSError:
            pass
    return out


def c3_stager_round(ext, layers, blocks, dev):
    """C3's 2048 blocks as one notice round through the product's StepStager: the block gather,
    then the delivery into the stage's file. Timed from commit until the sink has the file,
    three rounds (the faster of the last two reported), after ``prepare`` made the round's file
    and buffers (timed apart); then one round of another size, whose file the first commit
    makes."""
    import torch

    from everserve_amd.state.staging import StepStager

    kv = {f"model.layers.{i}.self_attn.attn": t for i, t in enumerate(layers)}
    scales = torch.ones(len(layers), dtype=torch.float32, device=dev)
    times = []
    ids = blocks.tolist()
    bs = layers[0].shape[2]
    with StepStager(ext, kv, [0], lambda job: None, scales=scales) as st:
        t0 = time.perf_counter()
        st.prepare([len(ids) * bs])
        prepare_s = time.perf_counter() - t0
        for k in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            n = st.commit_blocks(1, k + 1, ids)
            st.flush()
            times.append(time.perf_counter() - t0)
        half = ids[:len(ids) // 2]  # another capacity: no file of its size in the pool
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st.commit_blocks(1, 4, half)
        st.flush()
        unprepared_s = time.perf_counter() - t0
        bounce_nodes = page_nodes([b.data_ptr() for b in st._bounce], st._bounce_bytes)
    payload = n * len(layers) * layers[0].shape[-1] * 2
    ms = sorted(times[1:])[0] * 1e3
    return {"prepare_ms": round(prepare_s * 1e3, 3), "first_ms": round(times[0] * 1e3, 3),
            "ms": round(ms, 3), "gbs": round(payload / ms / 1e6, 2),
            "repeats_ms": [round(t * 1e3, 2) for t in times],
            "half_round_unprepared_ms": round(unprepared_s * 1e3, 3),
            "bounce_numa_nodes": bounce_nodes}


# ------------------------------------------------------------------------------ C4 restore
def bench_c4(ext, steps, warmup):
    import torch

    L, NB, BS, H, D = 32, 16384, 16, 8, 128
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    n = NB * BS  # 64 seqs x 4096 tokens: a full permutation of the 16,384-block cache
    rows = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device=dev)
    rows.normal_(generator=torch.Generator(device=dev).manual_seed(4))
    caches = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    _, slots = block_table_slots(NB, NB, BS, seed=4)
    ptrs = torch.tensor([t.data_ptr() for t in caches], dtype=torch.long, device=dev)
    s = torch.from_numpy(slots).to(dev)
    heads = torch.arange(H, dtype=torch.long, device=dev)
    strides = layout_strides(caches[0])
    payload = L * H * n * 2 * D * 2

    def scatter():
        ext.scatter_rows(ptrs, s, heads, rows.data_ptr(), n, D, BS, strides, 2)

    per, _ = time_launches(scatter, steps, warmup, stream)
    # round trip on the device: gather the restored cache back and compare with the rows
    back = torch.empty_like(rows[:4])
    ext.gather_rows(ptrs[:4], s, heads, back.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    ok = bool(torch.equal(back.view(torch.int16), rows[:4].view(torch.int16)))

    # the same call in staged order (evs_scatter_rows alone)
    def staged():
        ext.scatter_rows(ptrs, s, heads, rows.data_ptr(), n, D, BS, strides, 2, ordered=False)

    for t in caches[:4]:
        t.zero_()
    per_s, _ = time_launches(staged, steps, warmup, stream)
    ext.gather_rows(ptrs[:4], s, heads, back.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    ok_s = bool(torch.equal(back.view(torch.int16), rows[:4].view(torch.int16)))

    # the same restore with its writes in cache order: the (slot, staged row) pairs sorted by slot
    # on the host from the block table, then scatter_pairs
    from everserve_amd.state.restore import destination_order

    t0 = time.perf_counter()
    o_slots, o_rows = destination_order(slots, block_size=BS)
    order_ms = (time.perf_counter() - t0) * 1e3
    os_dev, or_dev = torch.from_numpy(o_slots).to(dev), torch.from_numpy(o_rows).to(dev)

    def ordered():
        ext.scatter_pairs(ptrs, os_dev, or_dev, heads, rows.data_ptr(), n, D, BS, strides, 2)

    for t in caches[:4]:
        t.zero_()
    per_o, _ = time_launches(ordered, steps, warmup, stream)
    ext.gather_rows(ptrs[:4], s, heads, back.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    ok_o = bool(torch.equal(back.view(torch.int16), rows[:4].view(torch.int16)))

    # the same with the pairs ordered on the device (evs_order_pairs), the sort inside the timing
    pairs = (torch.empty_like(s), torch.empty_like(s))  # the sort writes here: nothing allocated

    def ordered_on_device():
        o_s, o_r = ext.order_pairs(s, NB * BS, out=pairs)
        ext.scatter_pairs(ptrs, o_s, o_r, heads, rows.data_ptr(), n, D, BS, strides, 2)

    for t in caches[:4]:
        t.zero_()
    per_d, _ = time_launches(ordered_on_device, steps, warmup, stream)
    ext.gather_rows(ptrs[:4], s, heads, back.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    ok_d = bool(torch.equal(back.view(torch.int16), rows[:4].view(torch.int16)))
    per_sort, _ = time_launches(lambda: ext.order_pairs(s, NB * BS, out=pairs), steps, warmup,
                                stream)

    # the same rows restored as a store's tables name them: one written range per layer, row t
    # to slot t (scatter_ranges, what the Restorer launches, here over the whole cache at once)
    starts = torch.zeros(1, dtype=torch.long, device=dev)
    first_rows = torch.tensor([0, n], dtype=torch.long, device=dev)

    def by_ranges():
        ext.scatter_ranges(ptrs, starts, first_rows, n, heads, rows.data_ptr(), n, D, BS,
                           strides, 2)

    for t in caches[:4]:
        t.zero_()
    per_r, _ = time_launches(by_ranges, steps, warmup, stream)
    in_order = torch.arange(n, dtype=torch.long, device=dev)
    ext.gather_rows(ptrs[:4], in_order, heads, back.data_ptr(), n, D, BS, strides, 2)
    torch.cuda.synchronize()
    ok_r = bool(torch.equal(back.view(torch.int16), rows[:4].view(torch.int16)))
    del rows, caches, back
    settle_device(ext)
    ms = sum(per) / len(per)
    ms_s = sum(per_s) / len(per_s)
    ms_o = sum(per_o) / len(per_o)
    ms_d = sum(per_d) / len(per_d)
    ms_r = sum(per_r) / len(per_r)
    return {
        "config": "C4 restore: [32,8,262144,2,128] bf16 rows into a fresh 16384-block cache, "
                  "random-permutation block table (64 seqs x 4096 tokens)",
        "paths": "scatter_* here: the loader's scatter_rows as it chooses, which at this size "
                 "sorts the (slot, row) pairs by slot on the device (evs_order_pairs) and writes "
                 "them through the pair scatter (evs_scatter_pairs), the sort inside each timed "
                 "call; staged_order: scatter_rows(ordered=False), evs_scatter_rows alone; the "
                 "Restorer (a restore from the store's tables) launches evs_scatter_ranges, "
                 "measured in by_ranges_in_slot_order",
        "scatter_ms": round(ms, 3),
        "scatter_gbs": round(2 * payload / ms / 1e6, 1),
        "scatter_frac_of_8tbs": round(2 * payload / ms / 1e6 / PEAK_HBM_GBS, 4),
        "round_trip_equal_first_4_layers": ok,
        "staged_order": {
            "how": "scatter_rows(ordered=False): evs_scatter_rows, one kernel, the rows read "
                   "in staged order, each half-row written at its slot",
            "scatter_ms": round(ms_s, 3),
            "scatter_gbs": round(2 * payload / ms_s / 1e6, 1),
            "scatter_frac_of_8tbs": round(2 * payload / ms_s / 1e6 / PEAK_HBM_GBS, 4),
            "round_trip_equal_first_4_layers": ok_s,
        },
        "ordered": {
            "how": "scatter_pairs with the pairs in slot order (destination_order on the host: "
                   "the block table's 16,384 blocks sorted)",
            "scatter_ms": round(ms_o, 3),
            "scatter_gbs": round(2 * payload / ms_o / 1e6, 1),
            "scatter_frac_of_8tbs": round(2 * payload / ms_o / 1e6 / PEAK_HBM_GBS, 4),
            "order_host_ms": round(order_ms, 2),
            "round_trip_equal_first_4_layers": ok_o,
        },
        "ordered_on_device": {
            "how": "order_pairs (a radix sort of the slot ids on the device) then scatter_pairs, "
                   "both inside each timed launch",
            "ms": round(ms_d, 3),
            "gbs": round(2 * payload / ms_d / 1e6, 1),
            "frac_of_8tbs": round(2 * payload / ms_d / 1e6 / PEAK_HBM_GBS, 4),
            "sort_ms": round(sum(per_sort) / len(per_sort), 4),
            "round_trip_equal_first_4_layers": ok_d,
        },
        "by_ranges_in_slot_order": {
            "how": "the same rows as a store's tables hold them, row t to slot t: one written "
                   "range per layer through scatter_ranges (each XCD a contiguous part)",
            "ms": round(ms_r, 3),
            "gbs": round(2 * payload / ms_r / 1e6, 1),
            "frac_of_8tbs": round(2 * payload / ms_r / 1e6 / PEAK_HBM_GBS, 4),
            "round_trip_equal_first_4_layers": ok_r,
        },
    }


# ------------------------------------------------------------------------------ restore host path
def bench_restore_host(ext, steps, warmup):
    """The restore from the store's table files: this build's Restorer against the reference's
    procedure (core/everserve/state/mirror.py:916-939: map, index_select into pinned memory,
    copy to the device, write_rows), on the same C4-shaped tables in /dev/shm."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    from everserve_amd.state.paged import PagedKV
    from everserve_amd.state.restore import Restorer, open_tables, release_later

    L, NB, BS, H, D = 4, 16384, 16, 8, 128
    n = NB * BS
    row_bytes = 2 * D * 2
    dev = torch.device("cuda", 0)
    need = L * H * n * row_bytes + (256 << 20)
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
    if shm is not None and shutil.disk_usage(shm).free < need:
        log(f"/dev/shm has {shutil.disk_usage(shm).free >> 20} MiB free, {need >> 20} needed: "
            f"the tables go to {tempfile.gettempdir()}")
        shm = None
    tmp = tempfile.mkdtemp(prefix="evs-restore-", dir=shm)
    try:
        base = np.random.default_rng(4).integers(0, 1 << 16, size=n * 2 * D, dtype=np.uint16)
        base &= 0xBFFF  # finite bf16 values (clears the top exponent bit: no inf or NaN)
        paths = {}
        for layer in range(L):
            for h in range(H):
                table = layer * 1000 + h
                paths[table] = os.path.join(tmp, f"table{table}.rows")
                base.tofile(paths[table])
        written = [(0, n)]
        caches = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
        head_map = {h: (h + 3) % H for h in range(H)}
        # The Restorer (its pinned and device buffers) is built when the spare starts, before
        # any failure, and timed apart. Then four restores, each opening (mapping) the tables
        # afresh inside its timing, as the reference's procedure maps each file in its loop. The
        # timing ends when the cache is written; the tables' mappings are then released on a
        # thread of their own (release_later), timed apart and finished before the next restore
        # starts. The first restore is cold; the other three are the steady state, reported by
        # their median.
        t0 = time.perf_counter()
        restorer = Restorer(ext, caches)
        build_s = time.perf_counter() - t0
        ours, release, opened, parts = [], [], [], []
        for _ in range(4):
            t0 = time.perf_counter()
            tables = open_tables((t, p, written) for t, p in paths.items())
            opened.append(time.perf_counter() - t0)
            rows = restorer.restore(tables, head_map)
            ours.append(time.perf_counter() - t0)
            parts.append({k: round(v * 1e3, 2) for k, v in restorer.timing.items()
                          if k.endswith("_s")})
            t0 = time.perf_counter()
            release_later(tables).join()
            release.append(time.perf_counter() - t0)
        ours_s = sorted(ours[1:])[1]
        release_s = sorted(release[1:])[1]
        payload = rows * row_bytes
        # a spare that mapped the tables ahead of the failure and keeps them mapped
        tables = open_tables((t, p, written) for t, p in paths.items())
        restorer.restore(tables, head_map)  # the pages' first touch
        ahead = []
        for _ in range(3):
            t0 = time.perf_counter()
            restorer.restore(tables, head_map)
            ahead.append(time.perf_counter() - t0)
        del tables
        # check: layer 2's new head slot of theirs 5, slot ids 0..15
        got = caches[2][:, 0, :, head_map[5]].permute(1, 0, 2).contiguous()  # [16, 2, D]
        want = torch.from_numpy(base[: 16 * 2 * D].view(np.int16).reshape(16, 2, D).copy())
        ok = bool(torch.equal(got.view(torch.int16).cpu(), want))

        launches = restorer.timing.get("launches")
        # the reference's procedure on the same files: torch's index_select (on torch's
        # intra-op threads) into pinned memory allocated per table, then write_rows, whose
        # kv_first case is t[:, block, offset, head] = x (core/everserve/state/kvcopy.py:118-128)
        paged = PagedKV.of(caches[0])
        idx = torch.cat([torch.arange(s, s + c, dtype=torch.long) for s, c in written])
        idx_dev = idx.to(dev)
        blk, off = idx_dev // paged.block_size, idx_dev % paged.block_size
        ref = []
        for _ in range(4):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for table, path in paths.items():
                layer, head = divmod(table, 1000)
                src = torch.from_file(path, shared=True, size=n * 2 * D, dtype=torch.bfloat16)
                src = src.view(n, 2, D)
                pinned = torch.empty((idx.numel(), 2, D), dtype=torch.bfloat16, pin_memory=True)
                torch.index_select(src, 0, idx, out=pinned)
                on_device = pinned.to(dev, non_blocking=True)
                caches[layer][:, blk, off, head_map[head]] = on_device.transpose(0, 1)
            torch.cuda.synchronize()
            ref.append(time.perf_counter() - t0)
        ref_s = sorted(ref[1:])[1]
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    del caches
    settle_device(ext)
    plain = pinned_copy_gbs(1 << 30, to_host=False)
    return {
        "config": f"restore of {L * H} store tables of C4 shape ([262144, 2, 128] bf16, 128 MiB "
                  f"each, every slot written) from /dev/shm files into a fresh 16384-block cache "
                  f"at other head slots",
        "payload_bytes": payload,
        "tables_dir": os.path.dirname(tmp),
        "timing": "4 restores each, every one opening the tables afresh inside its timing (ours "
                  "through open_tables, with Python's garbage collection paused as in the restore "
                  "itself): the first cold, the steady state the median of the other 3. Ours is built "
                  "(restorer_build_ms) when the spare starts, before the first restore. Ours ends "
                  "when the cache is written; its tables' release is timed apart "
                  "(release_later). The reference's procedure releases each table inside its "
                  "loop, as written.",
        "restorer_build_ms": round(build_s * 1e3, 1),
        "ours_open_ms": [round(x * 1e3, 2) for x in opened],
        "ours_parts_ms": parts,
        "ours_s": round(ours_s, 3),
        "ours_gbs": round(payload / ours_s / 1e9, 2),
        "reference_procedure_s": round(ref_s, 3),
        "reference_procedure_gbs": round(payload / ref_s / 1e9, 2),
        "speedup": round(ref_s / ours_s, 2),
        "ours_release_ms": round(release_s * 1e3, 1),
        "ours_with_release_inline_gbs": round(payload / (ours_s + release_s) / 1e9, 2),
        "ours_tables_mapped_ahead_gbs": round(payload / sorted(ahead)[1] / 1e9, 2),
        "first_restore": {
            "ours_gbs": round(payload / ours[0] / 1e9, 2),
            "ours_with_build_gbs": round(payload / (ours[0] + build_s) / 1e9, 2),
            "ours_release_ms": round(release[0] * 1e3, 1),
            "reference_procedure_gbs": round(payload / ref[0] / 1e9, 2),
            "speedup": round(ref[0] / ours[0], 2),
        },
        "h2d_plain_memcpy_gbs": round(plain, 2),
        "frac_of_plain_h2d": round(payload / ours_s / 1e9 / plain, 4),
        "rows_check": ok,
        "host_threads": restorer._threads,
        "scatter_launches_per_restore": launches,
    }


def catch_up_written(steps_since, seqs=64, num_blocks=16384, block_size=16, seed=6):
    """The slots a decode run writes after a watermark, as the store's sorted (start, count)
    ranges: ``seqs`` sequences, each holding ``num_blocks // seqs`` blocks of a seeded
    random-permutation block table, each appending ``steps_since`` tokens from a position near
    1024 (a different one per sequence, so the runs start inside blocks)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    table = rng.permutation(num_blocks).reshape(seqs, num_blocks // seqs)
    p0 = 1024 + rng.integers(0, block_size, seqs)
    pos = p0[:, None] + np.arange(steps_since)[None, :]
    slots = np.sort((table[np.arange(seqs)[:, None], pos // block_size] * block_size
                     + pos % block_size).reshape(-1))
    cut = np.flatnonzero(np.diff(slots) != 1) + 1
    first = slots[np.r_[0, cut]]
    last = slots[np.r_[cut - 1, slots.size - 1]]
    return slots, [(int(a), int(b - a + 1)) for a, b in zip(first, last)]


def bench_restore_catch_up(ext, steps, warmup):
    """The spare's catch-up restore at the swap (adapters/vllm/everserve_vllm/spare.py:163-192):
    only the slots written after the first restore's watermark
    (core/everserve/state/mirror.py:897-904), many short ranges per table. All 256 tables of a
    Llama-3-8B rank ([262144, 2, 128] bf16 each, sparse /dev/shm files holding the written rows)
    into a fresh 16384-block cache, ours against the reference's procedure on the same files."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    from everserve_amd.state.restore import Restorer, open_tables, release_later

    L, NB, BS, H, D = 32, 16384, 16, 8, 128
    n = NB * BS
    row_bytes = 2 * D * 2
    dev = torch.device("cuda", 0)
    head_map = {h: (h + 3) % H for h in range(H)}
    caches = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    restorer = Restorer(ext, caches)
    out = {"config": f"catch-up restore of {L * H} store tables ([262144, 2, 128] bf16) into a "
                     f"fresh 16384-block cache at other head slots: 64 sequences on a random "
                     f"block table, the slots written in the last S decode steps",
           "timing": "4 restores each, tables mapped afresh inside each timing (ours through "
                     "open_tables, with Python's garbage collection paused); cold = the first, "
                     "steady = the median of the other 3; ours ends when the cache is written (the "
                     "mappings are released after, apart)"}
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
    for since in (16, 256):
        slots, written = catch_up_written(since, num_blocks=NB, block_size=BS)
        rows_per_table = slots.size
        payload = rows_per_table * row_bytes * L * H
        if shm is not None and shutil.disk_usage(shm).free < payload + (256 << 20):
            shm = None
        tmp = tempfile.mkdtemp(prefix="evs-catchup-", dir=shm)
        try:
            blk = np.random.default_rng(since).integers(0, 1 << 16, size=(rows_per_table, 2 * D),
                                                        dtype=np.uint16) & 0xBFFF
            paths = {}
            for layer in range(L):
                for h in range(H):
                    t = layer * 1000 + h
                    paths[t] = os.path.join(tmp, f"table{t}.rows")
                    with open(paths[t], "wb") as f:
                        f.truncate(n * row_bytes)
                    mm = np.memmap(paths[t], dtype=np.uint16, mode="r+", shape=(n, 2 * D))
                    mm[slots] = blk ^ np.uint16(t & 0x3FFF)
                    mm.flush()
                    del mm
            ours, release, opened, parts = [], [], [], []
            for _ in range(4):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                tables = open_tables((t, p, written) for t, p in paths.items())
                opened.append(time.perf_counter() - t0)
                got = restorer.restore(tables, head_map)
                ours.append(time.perf_counter() - t0)
                parts.append({k: round(v * 1e3, 2) for k, v in restorer.timing.items()
                              if k.endswith("_s")})
                t0 = time.perf_counter()
                release_later(tables).join()
                release.append(time.perf_counter() - t0)
            launches = restorer.timing.get("launches")
            # a spare that keeps the tables mapped from its first restore to the swap: the
            # catch-up then opens nothing and faults no page in
            kept = open_tables((t, p, written) for t, p in paths.items())
            restorer.restore(kept, head_map)
            mapped = []
            for _ in range(3):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                restorer.restore(kept, head_map)
                mapped.append(time.perf_counter() - t0)
            release_later(kept).join()
            # check two tables' rows in their new head slots
            ok = got == rows_per_table * L * H
            s_dev = torch.from_numpy(slots).to(dev)
            for t in (0 * 1000 + 5, 17 * 1000 + 2):
                layer, h = divmod(t, 1000)
                c = caches[layer][:, s_dev // BS, s_dev % BS, head_map[h]]  # [2, rows, D]
                want = torch.from_numpy((blk ^ np.uint16(t & 0x3FFF)).view(np.int16)
                                        .reshape(rows_per_table, 2, D).copy())
                ok = ok and bool(torch.equal(c.transpose(0, 1).contiguous().view(torch.int16)
                                             .cpu(), want))
            # the reference's procedure (mirror.py:916-939) on the same files: per table,
            # index_select of the written ranges into pinned memory, the copy, write_rows
            idx = torch.cat([torch.arange(a, a + c, dtype=torch.long) for a, c in written])
            ref = []
            for _ in range(4):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for t, path in paths.items():
                    layer, h = divmod(t, 1000)
                    src = torch.from_file(path, shared=True, size=n * 2 * D,
                                          dtype=torch.bfloat16).view(n, 2, D)
                    pinned = torch.empty((idx.numel(), 2, D), dtype=torch.bfloat16,
                                         pin_memory=True)
                    torch.index_select(src, 0, idx, out=pinned)
                    on_device = pinned.to(dev, non_blocking=True)
                    i_dev = idx.to(dev)
                    caches[layer][:, i_dev // BS, i_dev % BS, head_map[h]] = \
                        on_device.transpose(0, 1)
                torch.cuda.synchronize()
                ref.append(time.perf_counter() - t0)
        finally:
            shutil.rmtree(tmp, ignore_errors=True)
        o_s, r_s = sorted(ours[1:])[1], sorted(ref[1:])[1]
        out[f"steps_{since}"] = {
            "rows_per_table": int(rows_per_table),
            "ranges_per_table": len(written),
            "payload_bytes": int(payload),
            "ours_ms": round(o_s * 1e3, 3),
            "ours_gbs": round(payload / o_s / 1e9, 2),
            "ours_first_ms": round(ours[0] * 1e3, 3),
            "ours_open_ms": [round(x * 1e3, 2) for x in opened],
        "ours_parts_ms": parts,
            "ours_release_ms": round(sorted(release[1:])[1] * 1e3, 2),
            "reference_procedure_ms": round(r_s * 1e3, 3),
            "reference_procedure_gbs": round(payload / r_s / 1e9, 2),
            "reference_procedure_first_ms": round(ref[0] * 1e3, 3),
            "speedup": round(r_s / o_s, 2),
            "first_speedup": round(ref[0] / ours[0], 2),
            "scatter_launches": launches,
            "ours_parts_ms": parts,
            "ours_tables_kept_mapped_ms": round(sorted(mapped)[1] * 1e3, 3),
            "rows_check": bool(ok),
        }
    del caches, restorer
    settle_device(ext)
    return out


# ------------------------------------------------------------------------------ slot collective
def bench_slot(ext, steps, warmup):
    """The slot collective's one-GPU cost per call at decode sizes (evs_slot_all_reduce).

    With one GPU there is no peer, so each listed member is this same row repeated: every call
    publishes its words and then reads real, published words once per member, and never waits
    for a peer. A HIP graph of 50 calls is replayed, with sequence numbers advancing on the
    device, so the figure is the kernel's, not the host's launch rate. The reference's published
    4.21 us at 16,384 elements (4 x A100) includes NVLink transport, which is not measured here.
    """
    import torch

    dev = torch.device("cuda", 0)
    maxn, per_graph = 65536, 50
    half = maxn // 2
    ctrl_host, ctrl_dev = ext.host_alloc_mapped(ext.MAX_ROWS * ext.CTRL_WORDS * 8)
    out = {}
    try:
        for push in (False, True):
            words_buf = torch.zeros((2 * ext.MAX_ROWS if push else 2) * half, dtype=torch.int64,
                                    device=dev)
            bufs = torch.tensor([words_buf.data_ptr()] * ext.MAX_ROWS, dtype=torch.long,
                                device=dev)
            for k in (1, 4, 8):
                order = torch.tensor([k] + [0] * ext.MAX_ROWS, dtype=torch.int32, device=dev)
                for n in (2048, 16384, 65536):
                    x = torch.randn(n, device=dev).to(torch.bfloat16)
                    y = torch.empty_like(x)
                    seqs = torch.zeros(ext.slot_blocks(maxn, 1) + 1, dtype=torch.long,
                                       device=dev)
                    side = torch.cuda.Stream(device=dev)
                    side.wait_stream(torch.cuda.current_stream(dev))
                    with torch.cuda.stream(side):
                        for _ in range(3):  # eager warmup on the capture stream
                            ext.slot_all_reduce(x, y, bufs, ctrl_dev, order, seqs, 0, maxn, 1,
                                                push)
                    torch.cuda.synchronize()
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=side):
                        for _ in range(per_graph):
                            ext.slot_all_reduce(x, y, bufs, ctrl_dev, order, seqs, 0, maxn, 1,
                                                push)
                    for _ in range(max(1, warmup)):
                        g.replay()
                    torch.cuda.synchronize()
                    reps = max(4, steps)
                    t0 = torch.cuda.Event(enable_timing=True)
                    t1 = torch.cuda.Event(enable_timing=True)
                    t0.record()
                    for _ in range(reps):
                        g.replay()
                    t1.record()
                    torch.cuda.synchronize()
                    us = t0.elapsed_time(t1) * 1e3 / (reps * per_graph)
                    # k copies of x summed in fp32 are k * x exactly; one rounding to bf16
                    exact = bool(torch.equal(y, (x.float() * k).to(torch.bfloat16)))
                    out[f"{'push' if push else 'pull'}_k{k}_n{n}"] = {"us": round(us, 2),
                                                                       "sum_exact": exact}
                    del g
    finally:
        torch.cuda.synchronize()
        ext.host_free(ctrl_host)
    return {"config": "one GPU, members = this row repeated k times, 1 word per thread, "
                      "graph of 50 calls replayed", "per_call": out}


# ------------------------------------------------------------------------------ C5 reduce
def bench_c5(ext, steps, warmup):
    import torch

    from everserve_amd.kernels import REDUCE_STATE_WORDS

    K, N, SETS = 8, 256 * 8192, 32
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    sets = []
    for j in range(SETS):  # 32 sets x 36 MiB = 1.1 GiB: over 4x what the Infinity Cache holds
        # buffer i of set j from manual_seed(5 + i + 8 j): set 0 is the config's 5 + i
        bufs = [torch.randn(N, generator=torch.Generator(device=dev).manual_seed(5 + i + K * j),
                            device=dev, dtype=torch.float32).to(torch.bfloat16)
                for i in range(K)]
        table = torch.tensor([t.data_ptr() for t in bufs], dtype=torch.long, device=dev)
        out = torch.empty(N, dtype=torch.bfloat16, device=dev)
        sets.append((bufs, table, out))
    flags = torch.full((8,), 1, dtype=torch.long, device=dev)
    order = torch.tensor([K, *range(K)], dtype=torch.int32, device=dev)
    state = torch.zeros(REDUCE_STATE_WORDS, dtype=torch.long, device=dev)
    it = [0]

    def reduce_once():
        _, table, out = sets[it[0] % SETS]
        it[0] += 1
        ext.local_reduce(table, flags, order, out, 1, 10**9, 0, state)

    eager, _ = time_launches(reduce_once, max(steps, 4 * SETS), warmup, stream)
    torch.cuda.synchronize()
    eager_out = [out.clone() for _, _, out in sets]
    for _, _, out in sets:
        out.zero_()
    # the kernel's own cost: the 32 calls captured in a HIP graph (the reduce is capturable: no
    # memset, its counters reset themselves) and replayed, so no host launch sits between calls
    side = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _, table, out in sets:
            ext.local_reduce(table, flags, order, out, 1, 10**9, 0, state)
    replays = 25
    per, _ = time_launches(graph.replay, replays, 3, stream)
    per = [p / SETS for p in per]
    torch.cuda.synchronize()
    graph_equal = all(torch.equal(out.view(torch.int16), e.view(torch.int16))
                      for (_, _, out), e in zip(sets, eager_out))
    ok = int(state[0].item()) == 1 << 16
    # the stalled flag: row 3 left at epoch - 1 with a 1 ms bound fires the timeout
    flags[3] = 0
    t0 = time.perf_counter()
    ext.local_reduce(sets[0][1], flags, order, sets[0][2], 1, 1_000_000, 0, state)
    torch.cuda.synchronize()
    abort_ms = (time.perf_counter() - t0) * 1e3
    st = int(state[0].item())
    flags[3] = 1
    del sets
    settle_device(ext)
    decode = reduce_decode_sizes(ext, flags, order, state, steps, dev)
    late = reduce_late_member(ext, dev)
    us = sum(per) / len(per) * 1e3
    algo = (K + 1) * N * 2
    return {
        "config": "C5 local reduce: 8 bf16 buffers of 256 x 8192, fp32 accumulation in order; "
                  "32 buffer sets rotating (1.1 GiB, over 4x the 256 MB Infinity Cache)",
        "us_per_call": round(us, 2),
        "us_per_call_eager_launches": round(sum(eager) / len(eager) * 1e3, 2),
        "gbs": round(algo / us / 1e3, 1),
        "frac_of_8tbs": round(algo / us / 1e3 / PEAK_HBM_GBS, 4),
        "completed_status_ok": ok,
        "graph_replays_equal_eager": graph_equal,
        "stalled_flag": {"timeout_ns": 1_000_000, "host_ms_to_return": round(abort_ms, 3),
                         "reason": (st >> 8) & 0xFF, "late_mask": st & 0xFF},
        "decode_sizes": decode,
        "late_member": late,
    }


def reduce_late_member(ext, dev, trials=15, spin_us=50):
    """A call whose member in order position 4 (row 1) is still out when it starts, as when a
    peer's push lands after the reduce is launched: the reduce runs on one stream; on another, a
    bounded spin kernel (``torch.cuda._sleep``) and then a fill write that member's flag. The
    figure is the time from the flag's write (an event after the fill) to the call's end (an
    event after the reduce), median of ``trials``; every output is checked against the call with
    every member in."""
    import torch

    from everserve_amd.kernels import REDUCE_STATE_WORDS

    a, b = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(b):
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
    torch.cuda.synchronize()
    cycles_per_us = 1_000_000 / (e0.elapsed_time(e1) * 1e3)
    rows, late_row = [5, 3, 7, 0, 1, 6, 2, 4], 1
    out = {"how": "order [5,3,7,0,1,6,2,4], row 1 late: its flag written by a fill on a second "
                  f"stream after a {spin_us} us spin; microseconds from that write to the call's "
                  "end"}
    for n in (2048, 65536, 256 * 8192):
        bufs = [torch.randn(n, device=dev).to(torch.bfloat16) for _ in range(8)]
        table = torch.tensor([t.data_ptr() for t in bufs], dtype=torch.long, device=dev)
        order = torch.tensor([8, *rows], dtype=torch.int32, device=dev)
        flags = torch.ones(8, dtype=torch.long, device=dev)
        state = torch.zeros(REDUCE_STATE_WORDS, dtype=torch.long, device=dev)
        ref, y = (torch.empty(n, dtype=torch.bfloat16, device=dev) for _ in range(2))
        ext.local_reduce(table, flags, order, ref, 1, 10**9, 0, state)
        torch.cuda.synchronize()
        us, equal, ok = [], True, True
        for t in range(trials + 2):
            epoch = 2 + t
            flags.fill_(epoch)
            flags[late_row] = epoch - 1
            y.zero_()
            torch.cuda.synchronize()
            written, ended = (torch.cuda.Event(enable_timing=True) for _ in range(2))
            with torch.cuda.stream(a):
                ext.local_reduce(table, flags, order, y, epoch, 100_000_000, 0, state)
                ended.record()
            with torch.cuda.stream(b):
                torch.cuda._sleep(int(spin_us * cycles_per_us))
                flags[late_row:late_row + 1].fill_(epoch)
                written.record()
            torch.cuda.synchronize()
            equal &= bool(torch.equal(y.view(torch.int16), ref.view(torch.int16)))
            ok &= int(state[0].item()) == epoch << 16
            if t >= 2:
                us.append(written.elapsed_time(ended) * 1e3)
        us.sort()
        out[f"n{n}"] = {"us_flag_to_end": round(us[len(us) // 2], 2),
                        "sum_equal_all_in": equal, "status_ok": ok}
        del bufs
    return out


def reduce_decode_sizes(ext, flags, order, state, steps, dev, per_graph=50):
    """``evs_local_reduce`` at decode sizes (2 Ki, 16 Ki and 64 Ki bf16 elements) over k = 1, 4
    and 8 members: a HIP graph of 50 calls replayed, so the figure is the kernel's per call with
    no host launch between calls. Each sum is checked against torch's fp32 sum in order, rounded
    once to bf16 (core/everserve/reference/arith/ops.py:63-73)."""
    import torch

    out = {}
    for n in (2048, 16384, 65536):
        bufs = [torch.randn(n, device=dev).to(torch.bfloat16) for _ in range(8)]
        table = torch.tensor([t.data_ptr() for t in bufs], dtype=torch.long, device=dev)
        y = torch.empty(n, dtype=torch.bfloat16, device=dev)
        for k in (1, 4, 8):
            ordk = torch.tensor([k, *range(8)], dtype=torch.int32, device=dev)
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                ext.local_reduce(table, flags, ordk, y, 1, 10**9, 0, state)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for _ in range(per_graph):
                    ext.local_reduce(table, flags, ordk, y, 1, 10**9, 0, state)
            g.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = max(4, steps // 2)
            t0.record()
            for _ in range(reps):
                g.replay()
            t1.record()
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) * 1e3 / (reps * per_graph)
            acc = torch.zeros(n, dtype=torch.float32, device=dev)
            for t in bufs[:k]:
                acc += t.float()
            exact = bool(torch.equal(y.view(torch.int16), acc.to(torch.bfloat16).view(torch.int16)))
            ok = int(state[0].item()) == 1 << 16
            out[f"k{k}_n{n}"] = {"us": round(us, 2), "gbs": round((k + 1) * n * 2 / us / 1e3, 1),
                                 "sum_exact": exact, "status_ok": ok}
            del g
    return out


# ------------------------------------------------------------------------------ decode overhead
def bench_decode_overhead(ext, steps, warmup):
    """µs a per-step snapshot adds to a Llama-3-8B decode-step proxy (batch 64).

    The proxy's forward (32 layers: QKV projection, attention of 32 query heads over 8 KV heads
    and 1024 cached tokens, output projection, gated MLP; bf16) is captured once in a HIP graph,
    so a step is its kernels with no host launch between them, as a serving engine's decode step
    is. Each step ends with the host reading a slice of the step's output, as a serving loop reads
    the sampled tokens, so the host never runs ahead of the device.

    The snapshot is the reference's per-step semantics: the step's 64 new slots, every layer and
    KV head (8 MiB), through StepStager (gather behind the forward, host-side wait, delivery into a
    staging file in shared memory). The reference's own pattern (a side stream that waits on the
    forward's event, then gathers and copies to pinned memory, core/everserve/state/mirror.py:
    682-706) is timed beside it. Modes run interleaved, in rounds, and the best round counts.
    """
    import torch

    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    Lyr, Hd, HQ, HKV, DH, FF, B, CTX = 32, 4096, 32, 8, 128, 14336, 64, 1024
    bf = torch.bfloat16
    F = torch.nn.functional
    w = []
    for _ in range(Lyr):
        # weights stored [out, in], as nn.Linear keeps them; K and V [seq x kv head, 1, ctx, d].
        # The proxy has no norms, so its MLP (quadratic in x) is scaled down to keep the
        # residual stream finite over 32 layers (largest |x| about 60); what a GEMM costs does
        # not depend on the values.
        w.append({
            "qkv": torch.randn((HQ + 2 * HKV) * DH, Hd, device=dev, dtype=bf) * 0.02,
            "o": torch.randn(Hd, HQ * DH, device=dev, dtype=bf) * 0.02,
            "up": torch.randn(2 * FF, Hd, device=dev, dtype=bf) * 0.02,
            "down": torch.randn(Hd, FF, device=dev, dtype=bf) * 2e-5,
            "k": torch.randn(B * HKV, 1, CTX, DH, device=dev, dtype=bf),
            "v": torch.randn(B * HKV, 1, CTX, DH, device=dev, dtype=bf),
        })
    x0 = torch.randn(B, Hd, device=dev, dtype=bf)
    step_bytes = sum(t.numel() * t.element_size() for p in w for t in p.values())

    def forward():
        x = x0
        for p in w:
            qkv = F.linear(x, p["qkv"])
            # each KV head's 4 query heads attend over its 1024 cached tokens
            q = qkv[:, : HQ * DH].reshape(B * HKV, 1, HQ // HKV, DH)
            a = F.scaled_dot_product_attention(q, p["k"], p["v"])  # [B x HKV, 1, 4, DH]
            x = torch.addmm(x, a.reshape(B, HQ * DH), p["o"].t())
            gu = F.linear(x, p["up"])
            x = torch.addmm(x, F.silu(gu[:, :FF]) * gu[:, FF:], p["down"].t())
        return x

    eager_out = forward()
    torch.cuda.synchronize()
    eager_ms = []
    for _ in range(3):
        t0 = time.perf_counter()
        forward()
        torch.cuda.synchronize()
        eager_ms.append((time.perf_counter() - t0) * 1e3)
    def capture(fwd):
        cap = torch.cuda.Stream(device=dev)
        cap.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cap):
            for _ in range(2):
                fwd()
        torch.cuda.current_stream(dev).wait_stream(cap)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            o = fwd()
        g.replay()
        torch.cuda.synchronize()
        return g, o

    graph, out = capture(forward)
    # the library GEMMs may pick other algorithms inside a capture, so the graph's output can
    # differ from the eager one in the last bits; a capture that went wrong differs by O(1)
    graph_rel = float((out.float() - eager_out.float()).abs().max()
                      / eager_out.float().abs().max().clamp_min(1e-30))
    # the same step with fp8-e4m3 weights (per-tensor scale 1), as an FP8 checkpoint is served;
    # the activations are cast to fp8 per GEMM and the KV cache stays bf16
    fp8 = torch.float8_e4m3fn
    one = torch.ones((), device=dev)
    w8 = [{k: p[k].to(fp8) for k in ("qkv", "o", "up", "down")} for p in w]
    step8_bytes = step_bytes - sum(t.numel() for p in w8 for t in p.values())

    def lin8(x, weight):
        return torch._scaled_mm(x.to(fp8), weight.t(), scale_a=one, scale_b=one, out_dtype=bf)

    def forward8():
        x = x0
        for p, p8 in zip(w, w8):
            qkv = lin8(x, p8["qkv"])
            q = qkv[:, : HQ * DH].reshape(B * HKV, 1, HQ // HKV, DH)
            a = F.scaled_dot_product_attention(q, p["k"], p["v"])
            x = x + lin8(a.reshape(B, HQ * DH), p8["o"])
            gu = lin8(x, p8["up"])
            x = x + lin8(F.silu(gu[:, :FF]) * gu[:, FF:], p8["down"])
        return x

    graph8, out8 = capture(forward8)

    # the same fp8 step at batch 32 (the first 32 sequences, their K and V), a step that fits in
    # 5 ms on MI355X: the snapshot's share of a shorter step
    B32 = 32
    x32 = x0[:B32].contiguous()

    def forward8_b32():
        x = x32
        for p, p8 in zip(w, w8):
            qkv = lin8(x, p8["qkv"])
            q = qkv[:, : HQ * DH].reshape(B32 * HKV, 1, HQ // HKV, DH)
            a = F.scaled_dot_product_attention(q, p["k"][: B32 * HKV], p["v"][: B32 * HKV])
            x = x + lin8(a.reshape(B32, HQ * DH), p8["o"])
            gu = lin8(x, p8["up"])
            x = x + lin8(F.silu(gu[:, :FF]) * gu[:, FF:], p8["down"])
        return x

    graph8_32, out8_32 = capture(forward8_b32)

    # the snapshot: the step's 64 new slots, every layer and head, into a staging file
    from everserve_amd.state.staging import StepStager

    NB, BS = 4096, 16
    cache = [torch.randn(2, NB, BS, HKV, DH, device=dev, dtype=bf) for _ in range(Lyr)]
    kv = {f"model.layers.{i}.self_attn.attn": t for i, t in enumerate(cache)}
    slot_sets_32 = [torch.arange(i * B32, (i + 1) * B32, dtype=torch.long, device=dev) * 7
                    % (NB * BS) for i in range(4)]
    slot_sets = [torch.arange(i * B, (i + 1) * B, dtype=torch.long, device=dev) * 7 % (NB * BS)
                 for i in range(4)]
    staged = {"steps": 0}

    def sink(job):
        if job.descriptor is not None:
            staged["steps"] += 1

    stager = StepStager(ext, kv, list(range(HKV)), sink, depth=2)
    ptrs = torch.tensor([t.data_ptr() for t in cache], dtype=torch.long, device=dev)
    heads = torch.arange(HKV, dtype=torch.long, device=dev)
    strides = layout_strides(cache[0])
    side_rows = torch.empty((Lyr, HKV, B, 2, DH), dtype=bf, device=dev)
    side_host = torch.empty((Lyr, HKV, B, 2, DH), dtype=bf, pin_memory=True)
    side = torch.cuda.Stream(device=dev)
    row_bytes = 2 * DH * 2
    step_no = [0]

    def step(mode: str, i: int):
        g, o = ((graph8_32, out8_32) if mode.endswith("_fp8_b32")
                else (graph8, out8) if mode.endswith("_fp8") else (graph, out))
        g.replay()
        if mode.startswith("stager"):
            step_no[0] += 1
            sl = (slot_sets_32 if mode.endswith("_b32") else slot_sets)[i % 4]
            for name, t in kv.items():
                stager.save(name, t, sl)
            stager.commit(0, step_no[0], {})
        elif mode == "side_stream":
            done = torch.cuda.current_stream(dev).record_event()
            side.wait_event(done)
            with torch.cuda.stream(side):
                ext.gather_rows(ptrs, slot_sets[i % 4], heads, side_rows.data_ptr(), B, DH, BS,
                                strides, 2)
                ext.copy_rows_async(side_host.data_ptr(), side_rows.data_ptr(), Lyr * HKV,
                                    B * row_bytes, B * row_bytes, dev)
        o[:, :8].cpu()  # the sampled tokens: the host waits for the step's forward

    def run(mode: str, k: int):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(k):
            step(mode, i)
        stager.flush()  # the last step's rows are in the file before the clock stops
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / k

    modes = ("none", "stager", "side_stream", "none_fp8", "stager_fp8", "none_fp8_b32",
             "stager_fp8_b32")
    for _ in range(max(2, warmup)):
        for m in modes:
            step(m, 0)
    stager.flush()
    base = dict(stager.stats)
    k = max(steps, 20)
    times = {m: [] for m in modes}
    for _ in range(5):  # interleaved, so the box's drift falls on every mode alike
        for m in modes:
            times[m].append(run(m, k))
    stager.flush()
    st = {key: stager.stats[key] - base.get(key, 0) for key in stager.stats}
    stager.close()
    best = {m: min(v) for m, v in times.items()}
    off, on = best["none"], best["stager"]
    off8, on8 = best["none_fp8"], best["stager_fp8"]
    off32, on32 = best["none_fp8_b32"], best["stager_fp8_b32"]
    # the step as it would run at 75 % of HBM peak: the time the proxy's bytes take there
    roof_s = step_bytes / (0.75 * PEAK_HBM_GBS * 1e9)
    # the batch-32 step reads half the K and V
    step8_32_bytes = step8_bytes - Lyr * (B - B32) * HKV * CTX * DH * 2 * 2
    del w, w8, cache, graph, graph8, graph8_32
    settle_device(ext)
    return {
        "config": "Llama-3-8B decode-step proxy: 32 layers, batch 64, ctx 1024, bf16 (nn.Linear "
                  "layout GEMMs, SDPA per KV head), the forward in one HIP graph, the host "
                  "reading the output each step; snapshot = 64 slots "
                  "x 32 layers x 8 heads (8 MiB) through StepStager: gather on the forward's "
                  "stream, host-side wait, delivery into a staging file in shared memory",
        "step_ms_without": round(off * 1e3, 4),
        "step_ms_with": round(on * 1e3, 4),
        "added_us_per_step": round((on - off) * 1e6, 2),
        "added_percent": round((on - off) / off * 100, 3),
        "proxy_bytes_per_step": step_bytes,
        "proxy_hbm_gbs": round(step_bytes / off / 1e9, 1),
        "eager_forward_ms": round(sorted(eager_ms)[1], 3),
        "graph_forward_max_rel_diff": round(graph_rel, 6),
        "graph_forward_close_ok": graph_rel < 5e-2,
        "step_thread_us_per_step": round((st["step_thread_s"] - st["backpressure_s"]) /
                                         max(1, st["steps"]) * 1e6, 2),
        "copy_thread_us_per_step": round(st["copy_s"] / max(1, st["steps"]) * 1e6, 2),
        "backpressure_waits": st["backpressure_waits"],
        "commits": st["steps"],
        "steps_staged": staged["steps"],
        "added_us_side_stream_pattern": round((best["side_stream"] - off) * 1e6, 2),
        "added_percent_of_a_step_at_75pct_hbm": round((on - off) / roof_s * 100, 3),
        "step_at_75pct_hbm_ms": round(roof_s * 1e3, 3),
        "fp8_weights": {
            "step_ms_without": round(off8 * 1e3, 4),
            "step_ms_with": round(on8 * 1e3, 4),
            "added_us_per_step": round((on8 - off8) * 1e6, 2),
            "added_percent": round((on8 - off8) / off8 * 100, 3),
            "proxy_bytes_per_step": step8_bytes,
            "proxy_hbm_gbs": round(step8_bytes / off8 / 1e9, 1),
        },
        "fp8_weights_batch32": {
            "how": "the fp8 step over the first 32 sequences; snapshot = their 32 slots (4 MiB)",
            "step_ms_without": round(off32 * 1e3, 4),
            "step_ms_with": round(on32 * 1e3, 4),
            "added_us_per_step": round((on32 - off32) * 1e6, 2),
            "added_percent": round((on32 - off32) / off32 * 100, 3),
            "proxy_bytes_per_step": step8_32_bytes,
            "proxy_hbm_gbs": round(step8_32_bytes / off32 / 1e9, 1),
        },
        "rounds_ms": {m: [round(x * 1e3, 4) for x in v] for m, v in times.items()},
    }


# ------------------------------------------------------------------------------ counter runs
def pcie_workload(ext, copies=5):
    """What a rocprofv3 memory-copy trace measures: the host copies of the path, each beside a
    plain copy of the same size (torch's copy of a contiguous tensor, one hipMemcpyAsync).

    D2H: C3's staged rows, 80 groups of 8 MiB (640 MiB), by ``evs_copy_rows_async`` into pinned
    memory, and by ``evs_deliver_rows`` into a staging file in shared memory (the step path: 32 MiB
    batches into two pinned bounce buffers). H2D: the restore's copies by ``evs_copy_rows_async``,
    1 GiB in 16 pieces of 64 MiB, each piece 8 head tables' runs of 8 MiB placed 32 MiB apart in
    a 256 MiB chunk, as the Restorer copies a layer's heads; and one plain 1 GiB copy. Prints one line of
    HIP-event (and, for the delivery, host clock) rates. Every buffer is released before it
    returns, torch's pinned-memory cache included, so nothing of the workload is left for the
    process's exit to tear down.
    """
    import tempfile

    import numpy as np
    import torch

    from everserve_amd.state.staging import _map_stage_file

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    group, groups = 32768 * 256, 80
    d = torch.empty(group * groups, dtype=torch.uint8, device=dev)
    h = torch.empty(group * groups, dtype=torch.uint8, pin_memory=True)
    chunk, chunks = 64 << 20, 16
    d2 = torch.empty(chunk * chunks, dtype=torch.uint8, device=dev)
    h2 = torch.empty(chunk * chunks, dtype=torch.uint8, pin_memory=True)
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    path = Path(shm) / f"everserve-bench-pcie-{os.getpid()}.rows"
    mapping = _map_stage_file(path, group * groups)
    bounce_bytes = 32 << 20
    bounce = [torch.empty(bounce_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    side = torch.cuda.Stream(device=dev)
    file_addr = np.frombuffer(mapping, dtype=np.uint8).ctypes.data

    def rows_d2h():
        ext.copy_rows_async(h.data_ptr(), d.data_ptr(), groups, group, group, dev)

    def plain_d2h():
        h.copy_(d, non_blocking=True)

    def chunks_h2d():
        # a piece is rows [p, p + 8 MiB) of each of 8 tables laid 32 MiB apart in a chunk
        tables, run = 8, (chunk * 4) // 8 // 4
        for c in range(chunks // 4):
            base = c * 4 * chunk
            for p in range(4):
                off = base + p * run
                ext.copy_rows_async(d2.data_ptr() + off, h2.data_ptr() + off, tables, run,
                                    4 * run, dev)

    def plain_h2d():
        d2.copy_(h2, non_blocking=True)

    out = {}
    try:
        for name, fn, nbytes in (("d2h_rows", rows_d2h, d.numel()),
                                 ("d2h_plain", plain_d2h, d.numel()),
                                 ("h2d_chunks", chunks_h2d, d2.numel()),
                                 ("h2d_plain", plain_h2d, d2.numel())):
            per, _ = time_launches(fn, copies, 1, stream)
            out[name + "_gbs"] = round(nbytes / (sum(per) / len(per)) / 1e6, 2)
        torch.cuda.synchronize()
        times = []
        for _ in range(copies):
            t0 = time.perf_counter()
            ext.deliver_rows(file_addr, group, d.data_ptr(), group, groups, group,
                             [b.data_ptr() for b in bounce], bounce_bytes, side, 8)
            times.append(time.perf_counter() - t0)
        out["d2h_deliver_to_file_gbs"] = round(d.numel() / (sum(times) / len(times)) / 1e9, 2)
        torch.cuda.synchronize()
    finally:
        mapping.close()
        path.unlink(missing_ok=True)
        del d, h, d2, h2, bounce, side
        release_device_memory()
    print(json.dumps({"pcie_workload": out}), flush=True)


def release_device_memory():
    """Synchronise, then hand torch's cached device memory and pinned host memory back to the
    runtime now rather than at the process's exit."""
    import gc

    import torch

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    torch.cuda.synchronize()


def pmc_workload(ext, which="gather", launches=5):
    """What the rocprofv3 counter runs measure: ``launches`` calls of one kernel, then
    ``launches`` copies of a 1 GiB bf16 tensor by an elementwise kernel (torch.neg) whose
    FETCH_SIZE and WRITE_SIZE are known to be 1 GiB each, the scale the kernel's counters are
    read against.

    gather: the C2 gather. scatter: the C4 restore scatter (32 layers, 64 GiB moved) through
    the loader's scatter_rows as it chooses (at this size: its pairs sorted on the device, then
    the pair scatter). staged: scatter_rows(ordered=False), one kernel in staged order. pairs: the same restore
    in cache order (scatter_pairs, the pairs sorted by slot on the host). ranges: the same rows
    restored as one written range per layer, slots 0..n-1 in order (scatter_ranges, as the
    Restorer launches it, at C4's size). reduce: the C5 local
    reduce, each call on another of 32 buffer sets (1.1 GiB in all, over 4x what the Infinity
    Cache holds).
    """
    import torch

    from everserve_amd.kernels import REDUCE_STATE_WORDS

    dev = torch.device("cuda", 0)
    if which == "gather":
        L, NB, BS, H, D = 32, 8192, 16, 8, 128
        layers = random_cache_layers(L, (2, NB, BS, H, D), torch.bfloat16, dev, seed=0)
        _, slots = block_table_slots(NB, 1024, BS, seed=2)
        n = len(slots)
        ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.long, device=dev)
        s = torch.from_numpy(slots).to(dev)
        heads = torch.arange(H, dtype=torch.long, device=dev)
        out = torch.empty((L, H, n, 2, D), dtype=torch.bfloat16, device=dev)
        strides = layout_strides(layers[0])
        for _ in range(launches):
            ext.gather_rows(ptrs, s, heads, out.data_ptr(), n, D, BS, strides, 2)
        algo = 2 * L * H * n * 2 * D * 2
        del layers, out
    elif which in ("scatter", "staged", "pairs", "ranges"):
        L, NB, BS, H, D = 32, 16384, 16, 8, 128
        n = NB * BS
        # the counters count bytes, whatever they hold: the rows are left uninitialised
        rows = torch.empty((L, H, n, 2, D), device=dev, dtype=torch.bfloat16)
        caches = [torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev)
                  for _ in range(L)]
        _, slots = block_table_slots(NB, NB, BS, seed=4)
        ptrs = torch.tensor([t.data_ptr() for t in caches], dtype=torch.long, device=dev)
        s = torch.from_numpy(slots).to(dev)
        heads = torch.arange(H, dtype=torch.long, device=dev)
        strides = layout_strides(caches[0])
        if which == "pairs":
            from everserve_amd.state.restore import destination_order

            o_slots, o_rows = destination_order(slots, block_size=BS)
            os_dev, or_dev = torch.from_numpy(o_slots).to(dev), torch.from_numpy(o_rows).to(dev)
        starts = torch.zeros(1, dtype=torch.long, device=dev)
        first_rows = torch.tensor([0, n], dtype=torch.long, device=dev)
        for _ in range(launches):
            if which == "ranges":
                ext.scatter_ranges(ptrs, starts, first_rows, n, heads, rows.data_ptr(), n, D, BS,
                                   strides, 2)
            elif which == "pairs":
                ext.scatter_pairs(ptrs, os_dev, or_dev, heads, rows.data_ptr(), n, D, BS, strides,
                                  2)
            else:
                ext.scatter_rows(ptrs, s, heads, rows.data_ptr(), n, D, BS, strides, 2,
                                 ordered=which != "staged")
        algo = 2 * L * H * n * 2 * D * 2
        del rows, caches
    elif which == "reduce":
        K, N, SETS = 8, 256 * 8192, 32
        sets = []
        for i in range(SETS):
            bufs = [torch.randn(N, device=dev).to(torch.bfloat16) for _ in range(K)]
            table = torch.tensor([t.data_ptr() for t in bufs], dtype=torch.long, device=dev)
            sets.append((bufs, table, torch.empty(N, dtype=torch.bfloat16, device=dev)))
        flags = torch.ones(8, dtype=torch.long, device=dev)
        order = torch.tensor([K, *range(K)], dtype=torch.int32, device=dev)
        state = torch.zeros(REDUCE_STATE_WORDS, dtype=torch.long, device=dev)
        for i in range(launches):
            _, table, out = sets[i % SETS]
            ext.local_reduce(table, flags, order, out, 1, 10**9, 0, state)
        algo = (K + 1) * N * 2
        del sets
    else:
        raise ValueError(f"no counter workload {which!r}")
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    a = torch.randn(GIB // 2, device=dev, dtype=torch.float32).to(torch.bfloat16)
    b = torch.empty_like(a)
    for _ in range(launches):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    print(f"pmc workload done: {launches} {which} calls of {algo} algorithmic bytes, "
          f"{launches} copies of {GIB} bytes", flush=True)


# ------------------------------------------------------------------------------ main
def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="the headline only, no other configs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--legs", default="",
                    help="comma-separated extra legs to run (default: all; --quick: none)")
    ap.add_argument("--pcie", action="store_true",
                    help="only the host copies of the path beside plain copies, for a "
                         "rocprofv3 memory-copy trace")
    ap.add_argument("--pmc", nargs="?", const="gather", default=None,
                    choices=("gather", "scatter", "staged", "pairs", "ranges", "reduce"),
                    help="only a counter run's workload: 5 calls of the named kernel (default "
                         "gather), then 5 calibration copies")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {a.gpus}); run it with --gpus 1", file=sys.stderr)
        return 2
    legs = (("c1_gather", bench_c1), ("c2_layouts", bench_c2_layouts),
            ("c3_fp8_gather_d2h", bench_c3),
            ("c4_restore", bench_c4),
            ("restore_host_path", bench_restore_host),
            ("restore_catch_up", bench_restore_catch_up), ("store_commit", bench_store_commit),
            ("c5_reduce", bench_c5),
            ("slot_all_reduce", bench_slot), ("decode_overhead", bench_decode_overhead))
    wanted = {x for x in a.legs.split(",") if x}
    unknown = wanted - {name for name, _ in legs}
    if unknown:
        print(f"unknown legs: {sorted(unknown)}", file=sys.stderr)
        return 2

    import torch

    from everserve_amd import kernels

    ext = kernels.load()
    torch.cuda.set_device(0)
    if a.pmc:
        pmc_workload(ext, a.pmc)
        return 0
    if a.pcie:
        pcie_workload(ext)
        return 0
    log(f"device {torch.cuda.get_device_name(0)}; library {ext.__file__}")
    settle_device(ext)  # the copy probe's idle time, on the device before any leg allocates

    c2 = bench_c2(ext, a.steps, a.warmup, blocks_too=not a.quick)
    per = c2["per_launch_ms"]
    ms = sum(per) / len(per)
    achieved = c2["algo_bytes"] / (ms * 1e-3) / 1e9
    torch.cuda.synchronize()
    result = {
        "metric": "KV gather/restore GB/s & % HBM peak; µs added per decode step",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) caches, seeded block tables",
        "config": {
            "workload": "C2 Llama-3-8B KV gather: 32 layers x [2, 8192, 16, 8, 128] bf16 "
                        "kv_first, 1024 blocks over 64 seqs (16,384 slots), 8 heads -> "
                        "[32, 8, 16384, 2, 128] staging in HBM",
            "bytes_per_step": c2["algo_bytes"],
            "parallelism": "1 GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": pmc_traffic(),
            "kernel": "move_rows<16-byte words, gather, by slots>",
            "launch_ms_min_max": [round(min(per), 4), round(max(per), 4)],
        },
        "cpu_baseline": None,
        "extra": {"c2_spot_check": c2["spot_check"]},
    }
    if "blocks_per_launch_ms" in c2:
        bms = sum(c2["blocks_per_launch_ms"]) / a.steps
        result["extra"]["c2_gather_blocks"] = {
            "ms": round(bms, 4), "gbs": round(c2["algo_bytes"] / bms / 1e6, 1),
            "rows_equal_gather_rows": c2["blocks_equal"]}
    failed = []
    if not a.quick:
        for name, fn in legs:
            if wanted and name not in wanted:
                continue
            log(f"{name} ...")
            # the headline is measured: a leg that fails is recorded, and the line still printed
            try:
                result["extra"][name] = fn(ext, a.steps, a.warmup)
            except Exception as e:  # noqa: BLE001
                log(f"{name} failed: {type(e).__name__}: {e}")
                result["extra"][name] = {"error": f"{type(e).__name__}: {e}"}
                failed.append(name)
    if not a.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline_c2()
        if not a.quick and not wanted:
            log("cpu baselines of the restore and the reduce ...")
            result["extra"]["cpu_baselines_more"] = cpu_baselines_more()
    result["extra"]["settle_s"] = round(_SETTLE["waited_s"], 3)
    if failed:
        result["extra"]["failed_legs"] = failed
    wrong = failed_checks(result)
    if wrong:
        result["extra"]["failed_checks"] = wrong
    # the line is printed either way (its headline is measured); the exit status says whether
    # every leg ran and every parity check in it held
    result["status"] = "failed" if failed or wrong else "ok"
    print(json.dumps(result), flush=True)
    return 1 if failed or wrong else 0


def failed_checks(tree, path: str = "") -> list[str]:
    """The parity flags in a result that came out False: every boolean whose key says it checks
    bytes or values (``*equal*``, ``*check*``, ``*exact*``, ``*_ok``)."""
    out = []
    if isinstance(tree, dict):
        for k, v in tree.items():
            name = f"{path}.{k}" if path else str(k)
            if isinstance(v, bool):
                if not v and any(w in k for w in ("equal", "check", "exact", "_ok")):
                    out.append(name)
            else:
                out += failed_checks(v, name)
    return out


if __name__ == "__main__":
    sys.exit(main())
