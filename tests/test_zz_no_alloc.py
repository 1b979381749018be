"""The allocation-free ordering (evs_order_pairs_static) on the GPU, through the C ABI.

Its output must equal evs_order_pairs' (the entry point with a caller's workspace) bit for bit, on
two calls in a row, the second smaller than the first, so that the scratch array still holds the
first call's contents when the second runs. The slot lists hold padding ids and repeated slots,
whose listed order the stable sort keeps. A call past the scratch's maximum is refused before
anything is enqueued, and the first call on a device allocates no device memory.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_PAIRS = 1 << 20
SCRATCH_BYTES = 32 << 20


def slot_list(n, num_slots, seed):
    rng = np.random.default_rng(seed)
    s = rng.integers(0, num_slots, size=n, dtype=np.int64)
    s[rng.integers(0, n, size=max(1, n // 50))] = -1  # padding
    s[: n // 10] = s[n // 10: 2 * (n // 10)]  # repeated slots
    return torch.from_numpy(s).cuda()


def with_workspace(ext, slots, bits):
    need = ctypes.c_int64()
    assert ext._lib.evs_order_pairs_workspace(slots.numel(), bits, ctypes.byref(need)) == 0
    work = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    out_s, out_r = torch.empty_like(slots), torch.empty_like(slots)
    rc = ext._lib.evs_order_pairs(slots.data_ptr(), slots.numel(), bits, out_s.data_ptr(),
                                  out_r.data_ptr(), work.data_ptr(), work.numel(),
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ext._lib.evs_last_error()
    return out_s, out_r


def static(ext, slots, bits):
    out_s, out_r = torch.empty_like(slots), torch.empty_like(slots)
    rc = ext._lib.evs_order_pairs_static(slots.data_ptr(), slots.numel(), bits, out_s.data_ptr(),
                                         out_r.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ext._lib.evs_last_error()
    return out_s, out_r


def test_the_first_call_allocates_no_device_memory(ext):
    """The call's promise: no device memory is allocated, by it or lazily under it (the scratch
    address looked up on the first call on a device, rocPRIM's first sort of a size). The
    library's kernels are loaded first, by the workspace entry point; the free device memory and
    torch's reserved memory are then the same after the first allocation-free call."""
    slots = slot_list(300_000, 1 << 20, seed=5)
    want = with_workspace(ext, slots, 20)
    out_s, out_r = torch.empty_like(slots), torch.empty_like(slots)
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    reserved_before = torch.cuda.memory_reserved()
    rc = ext._lib.evs_order_pairs_static(slots.data_ptr(), slots.numel(), 20, out_s.data_ptr(),
                                         out_r.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert rc == 0, ext._lib.evs_last_error()
    assert torch.cuda.memory_reserved() == reserved_before
    assert free_after == free_before, free_before - free_after
    assert torch.equal(out_s, want[0]) and torch.equal(out_r, want[1])


def test_the_scratch_holds_the_largest_call_it_takes(ext):
    need = ctypes.c_int64()
    for bits in (1, 18, 32, 64):
        assert ext._lib.evs_order_pairs_workspace(MAX_PAIRS, bits, ctypes.byref(need)) == 0
        assert need.value <= SCRATCH_BYTES, (bits, need.value)


@pytest.mark.parametrize("sizes,num_slots", [((262144, 5000), 262144), ((MAX_PAIRS, 3), 1 << 40)])
def test_two_calls_in_a_row_equal_the_workspace_entry_point(ext, sizes, num_slots):
    bits = max(1, (num_slots - 1).bit_length())
    for k, n in enumerate(sizes):
        slots = slot_list(n, num_slots, seed=17 + k)
        want = with_workspace(ext, slots, bits)
        got = static(ext, slots, bits)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), n
        # and it is the stable order by slot
        order = np.argsort(slots.cpu().numpy().view(np.uint64) & np.uint64((1 << bits) - 1)
                           if bits < 64 else slots.cpu().numpy().view(np.uint64), kind="stable")
        assert np.array_equal(got[1].cpu().numpy(), order), n


def test_a_call_past_the_maximum_is_refused_before_launch(ext):
    slots = torch.zeros(1, dtype=torch.long, device="cuda")
    out = torch.zeros(2, dtype=torch.long, device="cuda")
    rc = ext._lib.evs_order_pairs_static(slots.data_ptr(), MAX_PAIRS + 1, 20, out.data_ptr(),
                                         out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 1
    assert b"at most" in ext._lib.evs_last_error()
    assert ext._lib.evs_order_pairs_static(slots.data_ptr(), 0, 20, out.data_ptr(),
                                           out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert not out.any()
