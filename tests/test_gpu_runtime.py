"""The library's runtime helpers on the GPU, each checked directly.

Device memory outside torch (zeroed at allocation, cleared by the fill kernel), pinned host memory
mapped for the device, the row copy in both directions and with a pitch, events with and without
the system fence, the stream handoff, the wall clock and an IPC handle. Registering existing host
memory (host_register_mapped) is not called: the GPU pool these tests run on refuses it, and the
error it leaves would be reported by the next GPU call.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def host_view(ptr: int, n: int) -> np.ndarray:
    """n bytes of host memory at ptr as a numpy array (no copy)."""
    return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(ptr))


def test_device_memory_is_zeroed_and_the_fill_clears_it(ext):
    n = (1 << 20) + 12  # not a multiple of the fill's 16-byte words
    dev = ext.device_alloc(n)
    host, _ = ext.host_alloc_mapped(n)
    try:
        h = host_view(host, n)
        ext.copy_rows_async(host, dev, 1, n, n, torch.device("cuda", 0))
        torch.cuda.synchronize()
        assert not h.any()
        h[:] = np.arange(n, dtype=np.uint64).astype(np.uint8) | 1
        ext.copy_rows_async(dev, host, 1, n, n, torch.device("cuda", 0))
        torch.cuda.synchronize()  # the copy has read the host bytes before they change
        h[:] = 0
        ext.copy_rows_async(host, dev, 1, n, n, torch.device("cuda", 0))
        torch.cuda.synchronize()
        assert (h == (np.arange(n, dtype=np.uint64).astype(np.uint8) | 1)).all()
        ext.memset_async(dev, n - 5)  # the last 5 bytes keep their values
        ext.copy_rows_async(host, dev, 1, n, n, torch.device("cuda", 0))
        torch.cuda.synchronize()
        assert not h[:n - 5].any() and h[n - 5:].all()
    finally:
        ext.host_free(host)
        ext.device_free(dev)


def test_mapped_host_memory_is_seen_by_the_device(ext):
    n = 4096
    host, dev_ptr = ext.host_alloc_mapped(n)
    try:
        host_view(host, n)[:] = 0x5A
        out = torch.zeros(n, dtype=torch.uint8, device="cuda")
        ext.copy_rows_async(out.data_ptr(), dev_ptr, 1, n, n, out.device)
        torch.cuda.synchronize()
        assert bool((out == 0x5A).all())
    finally:
        ext.host_free(host)


def test_the_row_copy_with_a_pitch_moves_only_the_rows(ext):
    groups, nbytes, pitch = 7, 96, 160
    src = torch.arange(groups * pitch, dtype=torch.int32, device="cuda").to(torch.uint8)
    dst = torch.full((groups * pitch,), 0xEE, dtype=torch.uint8, device="cuda")
    ext.copy_rows_async(dst.data_ptr(), src.data_ptr(), groups, nbytes, pitch, dst.device)
    torch.cuda.synchronize()
    s, d = src.view(groups, pitch).cpu(), dst.view(groups, pitch).cpu()
    assert torch.equal(d[:, :nbytes], s[:, :nbytes]) and bool((d[:, nbytes:] == 0xEE).all())


@pytest.mark.parametrize("system_fence", [False, True])
def test_an_event_orders_the_host_after_the_stream(ext, system_fence):
    ev = ext.event_create(system_fence)
    try:
        t = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
        t.fill_(9)
        ext.event_record(ev, torch.cuda.current_stream())
        ext.event_synchronize(ev)
        assert int(t[-1].item()) == 9
    finally:
        ext.event_destroy(ev)


def test_the_stream_handoff_orders_one_stream_after_another(ext):
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    ev = ext.event_create(False)
    try:
        big = torch.empty(1 << 28, dtype=torch.int32, device="cuda")
        with torch.cuda.stream(a):
            big.fill_(3)  # long enough that an unordered reader would see it half done
        ext.stream_handoff(a, b, ev)
        with torch.cuda.stream(b):
            total = big.sum(dtype=torch.int64)
        b.synchronize()
        assert int(total.item()) == 3 * big.numel()
    finally:
        torch.cuda.synchronize()
        ext.event_destroy(ev)


def test_the_wall_clock_runs_and_a_device_buffer_has_an_ipc_handle(ext):
    assert ext.wall_clock_khz() > 0
    p = ext.device_alloc(1 << 16)
    try:
        h = ext.ipc_handle(p)
        assert len(h) == 64 and any(h)
    finally:
        ext.device_free(p)
