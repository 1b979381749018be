"""SlotKernel over a region in pinned host memory, one process holding every row, on the GPU.

The reference's REPLACE (core/tests/test_slot_kernel.py:64-147,163-235) with the other members'
words written by the host, as its host-memory variant's rows are: three ranks reduce in rank order;
a graph is captured; rank 1 stops, the kernel names it late and the abort releases it; every
member resumes and takes the new order with the spare's row in rank 1's place; the graph captured
before the change replays over the new order without recapture and gives the same sum, bit for bit,
as before the change. The inputs make the order of the sum show.
"""

import numpy as np
import pytest
import torch

import oracle
from everserve_amd.comm.slotkernel import MAXN, Region, SlotKernel
from tests.cases import bits

pytestmark = pytest.mark.gpu

N = 16384
RANKS, SPARE = [0, 1, 2], 3
AFTER = [0, SPARE, 2]


def graph_input(rank):
    g = torch.Generator().manual_seed(7)
    big = torch.randn(N, generator=g) * 2.0**20
    small = torch.randn(N, generator=g) * 2.0**-6
    return {0: big, 1: small, 2: -big}[rank].to(torch.bfloat16)


def put_words(region, row, x, seq):
    """Row `row`'s words for call `seq`, as that member's kernel writes them."""
    pairs = x.contiguous().view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
    at = (seq & 1) * (MAXN // 2)
    region.words[row, at:at + pairs.size] = (np.int64(seq) << 32) | pairs


def test_replace_keeps_the_sum_and_the_captured_graph(ext):
    region = Region.in_pinned_memory(ext, "host")
    try:
        region.set_members(RANKS, RANKS)
        k = SlotKernel(region, 0, 0, ext=ext)
        assert k.can_take(torch.empty(N, dtype=torch.bfloat16, device="cuda"))
        assert not k.can_take(torch.empty(N + 1, dtype=torch.bfloat16, device="cuda"))
        xs = {r: graph_input(r) for r in (0, 1, 2)}
        in_rank = oracle.member_sum([bits(xs[r]) for r in RANKS])
        in_rows_after = oracle.member_sum([bits(xs[r]) for r in (0, 2, 1)])
        assert not np.array_equal(in_rank, in_rows_after), "the inputs must make the order show"

        x0 = xs[0].cuda()
        out = torch.empty_like(x0)
        # an eager call, seq 1
        for r in (1, 2):
            put_words(region, r, xs[r], 1)
        k.all_reduce_into(x0, out)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), in_rank)

        side = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            k.all_reduce_into(x0, out)
        for r in (1, 2):
            put_words(region, r, xs[r], 2)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), in_rank)

        # rank 1 stops: only rank 2's words for call 3; the kernel names row 1, the abort releases
        region.set_bound([0], 0.02)
        put_words(region, 2, xs[2], 3)
        graph.replay()
        seen = set()
        import time
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.3:
            seen |= region.late(0)
            time.sleep(0.002)
        k.abort()
        torch.cuda.synchronize()
        assert seen == {1}, seen
        assert region.late(0) == set()

        # the boundary: the executor writes the new order, the member resumes and takes it
        region.set_members(AFTER, AFTER)
        k.resume()
        assert int(region.ctrl[0, 1]) == 0 and int(k.seq.sum().item()) == 0
        k.set_members(AFTER, 1)
        assert region.order(0) == AFTER
        # the spare holds rank 1's state and writes its words in row 3; the counters restart at 1
        put_words(region, SPARE, xs[1], 1)
        put_words(region, 2, xs[2], 1)
        out.zero_()
        graph.replay()  # captured before the change
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), in_rank)
        k.close()
    finally:
        region.close()


@pytest.mark.parametrize("n", [16384, 3000, 2])
def test_sums_at_the_reference_sizes_are_member_sum_over_both_word_halves(ext, n):
    """The reference's sizes (core/tests/test_slot_kernel.py:163-190) through the driver: three
    rows in rank order, members N(0,1) from torch's generator, two calls in a row so that both
    halves of the words (the sequence number's parity) carry a sum; each equals member_sum."""
    region = Region.in_pinned_memory(ext, "host")
    try:
        region.set_members(RANKS, RANKS)
        k = SlotKernel(region, 0, 0, ext=ext)
        for call in (1, 2):
            xs = {r: torch.randn(n, generator=torch.Generator().manual_seed(1000 * r + n + call))
                  .to(torch.bfloat16) for r in RANKS}
            for r in (1, 2):
                put_words(region, r, xs[r], call)
            x0 = xs[0].cuda()
            out = torch.full_like(x0, float("nan"))
            k.all_reduce_into(x0, out)
            torch.cuda.synchronize()
            assert np.array_equal(bits(out), oracle.member_sum([bits(xs[r]) for r in RANKS])), call
        assert not k.can_take(torch.empty(3, dtype=torch.bfloat16, device="cuda"))  # odd
        assert not k.can_take(torch.empty(4, dtype=torch.float16, device="cuda"))
        assert not k.can_take(torch.empty(MAXN + 2, dtype=torch.bfloat16, device="cuda"))
        k.close()
    finally:
        region.close()
