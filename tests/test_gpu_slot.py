"""The slot collective's kernel (evs_slot_all_reduce) on one GPU, against the oracle's ordered sum.

The reference runs three ranks on NVLink GPUs (core/tests/test_slot_kernel.py:162-235); on one GPU
the members' words are staged in HBM instead: written by the test with the call's sequence number
(as core/tests/test_slot_kernel.py:108-122 writes a cut-short push), or written by other members'
kernels running at the same time on other streams. Checked bit for bit against
core/everserve/reference/arith/ops.py:63-73 at the reference's sizes {16384, 3000, 2}, both
variants, 1 and 16 words per thread, the order-sensitive inputs, eight members polled in one batch
or two, an order entry out of range, a member that never arrives (named in LATE, released by
ABORT, LATE cleared after), and replays of a captured graph whose sequence numbers advance in
device memory. Every wait is bounded by the kernel's own timeout.
"""

import ctypes
import time

import numpy as np
import pytest
import torch

import oracle
from tests.cases import bf16_tensor, bits, special_members

pytestmark = pytest.mark.gpu

MAXW, MAXN = 8, 64 * 1024
ABORT, LATE, BOUND, CTRL_WORDS = 1, 11, 12, 16


def member_input(rank: int, n: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(1000 * rank + n)
    return torch.randn(n, generator=g).to(torch.bfloat16)


def ll_words_host(x: torch.Tensor, seq: int) -> np.ndarray:
    """A member's LL words for one call, (seq << 32) | two bf16, computed on the host."""
    pairs = x.detach().cpu().contiguous().view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
    return (np.int64(seq) << 32) | pairs


def ll_words(x: torch.Tensor, seq: int) -> torch.Tensor:
    """The same words as int64 on the device."""
    return torch.from_numpy(ll_words_host(x, seq)).cuda()


class Region:
    """Word buffers per row, the control rows (host-mapped), and one member's order and seqs."""

    def __init__(self, ext, push: bool, rows):
        self.ext, self.push = ext, push
        per_row = (2 * MAXW if push else 2) * (MAXN // 2)
        self.words = {r: torch.zeros(per_row, dtype=torch.int64, device="cuda") for r in rows}
        table = [0] * MAXW
        for r, t in self.words.items():
            table[r] = t.data_ptr()
        self.bufs = torch.tensor(table, dtype=torch.long, device="cuda")
        self.ctrl_host, self.ctrl_dev = ext.host_alloc_mapped(MAXW * CTRL_WORDS * 8)
        self.ctrl = (ctypes.c_int64 * (MAXW * CTRL_WORDS)).from_address(self.ctrl_host)

    def member(self, order):
        o = torch.tensor([len(order), *order] + [0] * (MAXW - len(order)), dtype=torch.int32,
                         device="cuda")
        seqs = torch.zeros(self.ext.slot_blocks(MAXN, 1) + 1, dtype=torch.int64, device="cuda")
        return o, seqs

    def stage(self, reader: int, sender: int, x: torch.Tensor, seq: int):
        """Put `sender`'s words for call `seq` where `reader` reads them."""
        half = MAXN // 2
        parity = seq & 1
        w = ll_words(x, seq)
        if self.push:
            at = (parity * MAXW + sender) * half
            self.words[reader][at:at + w.numel()] = w
        else:
            at = parity * half
            self.words[sender][at:at + w.numel()] = w

    def close(self):
        self.ext.host_free(self.ctrl_host)


def reduce(ext, reg, row, order, seqs, x, words):
    xin = x.cuda()
    out = torch.empty_like(xin)
    ext.slot_all_reduce(xin, out, reg.bufs, reg.ctrl_dev, order, seqs, row, MAXN, words, reg.push)
    return out


@pytest.mark.parametrize("push", [False, True])
@pytest.mark.parametrize("n", [16384, 3000, 2])
@pytest.mark.parametrize("words", [1, 16])
def test_the_sum_is_member_sum_in_rank_order(ext, push, n, words):
    rows = [0, 1, 2]
    reg = Region(ext, push, rows)
    try:
        order, seqs = reg.member(rows)
        xs = {r: member_input(r, n) for r in rows}
        for r in (1, 2):
            reg.stage(0, r, xs[r], seq=1)
        out = reduce(ext, reg, 0, order, seqs, xs[0], words)
        torch.cuda.synchronize()
        want = oracle.member_sum([bits(xs[r]) for r in rows])
        assert np.array_equal(bits(out), want)
        # this member's own words were published where the others read them
        half = MAXN // 2
        own = ll_words(xs[0], 1)
        if push:
            for r in rows:
                at = (1 * MAXW + 0) * half
                assert torch.equal(reg.words[r][at:at + own.numel()], own)
        else:
            assert torch.equal(reg.words[0][half:half + own.numel()], own)
        # the second call uses the other parity and sequence number 2
        ys = {r: member_input(10 + r, n) for r in rows}
        for r in (1, 2):
            reg.stage(0, r, ys[r], seq=2)
        out = reduce(ext, reg, 0, order, seqs, ys[0], words)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), oracle.member_sum([bits(ys[r]) for r in rows]))
    finally:
        reg.close()


@pytest.mark.parametrize("push", [False, True])
@pytest.mark.parametrize("words", [1, 2, 4, 16])
def test_eight_members_in_one_batch_or_two(ext, push, words):
    """Eight members in a shuffled order, this member (row 3) in the middle: at 1 or 2 words a
    thread a poll covers all eight, at 4 or 16 they come in two batches of four. Two calls, so
    both parity halves are used."""
    rows = [5, 2, 7, 3, 0, 6, 1, 4]
    n = 16384 if words < 16 else 2 * 16 * 256 * 2 + 6  # 16 words: several workgroups, a ragged end
    reg = Region(ext, push, range(MAXW))
    try:
        order, seqs = reg.member(rows)
        for seq in (1, 2):
            xs = {r: member_input(100 * seq + r, n) for r in rows}
            for r in rows:
                if r != 3:
                    reg.stage(3, r, xs[r], seq=seq)
            out = reduce(ext, reg, 3, order, seqs, xs[3], words)
            torch.cuda.synchronize()
            want = oracle.member_sum([bits(xs[r]) for r in rows])
            assert np.array_equal(bits(out), want), seq
    finally:
        reg.close()


def test_a_row_out_of_range_in_the_order_is_skipped(ext):
    """An order entry outside [0, 8) is never waited for and adds nothing; the members around it
    are summed in their order."""
    n, rows = 3000, [0, 1, 2]
    reg = Region(ext, False, rows)
    try:
        o = torch.tensor([4, 2, 11, 0, 1] + [0] * (MAXW - 4), dtype=torch.int32, device="cuda")
        seqs = torch.zeros(ext.slot_blocks(MAXN, 1) + 1, dtype=torch.int64, device="cuda")
        xs = {r: member_input(30 + r, n) for r in rows}
        for r in (1, 2):
            reg.stage(0, r, xs[r], seq=1)
        out = reduce(ext, reg, 0, o, seqs, xs[0], 1)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), oracle.member_sum([bits(xs[2]), None, bits(xs[0]),
                                                             bits(xs[1])]))
    finally:
        reg.close()


def test_the_listed_order_is_the_order_of_the_sum(ext):
    n = 16384
    g = torch.Generator().manual_seed(7)
    big = torch.randn(n, generator=g) * 2.0**20
    small = torch.randn(n, generator=g) * 2.0**-6
    xs = {0: big.to(torch.bfloat16), 1: small.to(torch.bfloat16), 2: (-big).to(torch.bfloat16)}
    reg = Region(ext, False, [0, 1, 2])
    try:
        for order_rows in ([0, 1, 2], [0, 2, 1]):
            order, seqs = reg.member(order_rows)
            for r in (1, 2):
                reg.stage(0, r, xs[r], seq=1)
            out = reduce(ext, reg, 0, order, seqs, xs[0], 1)
            torch.cuda.synchronize()
            assert np.array_equal(bits(out), oracle.member_sum([bits(xs[r]) for r in order_rows]))
    finally:
        reg.close()


@pytest.mark.parametrize("push", [False, True])
def test_words_that_arrive_while_the_member_waits_are_summed(ext, push):
    """The members' words arrive while the kernel polls. The buffers the member reads are pinned
    host memory, as in the reference's host-memory variant (core/everserve/comm/slotkernel.py:
    535-548), and the test writes the peers' words from the host after the launch, one peer at a
    time. (Kernels of several members on several streams of one process are not guaranteed to
    run at once: two streams can share a hardware queue, so they are not used here.)"""
    rows, n = [0, 1, 2], 16384
    half = MAXN // 2
    per_row = (2 * MAXW if push else 2) * half
    host = {r: ext.host_alloc_mapped(per_row * 8) for r in rows}
    ctrl_host, ctrl_dev = ext.host_alloc_mapped(MAXW * CTRL_WORDS * 8)
    try:
        views = {r: np.frombuffer((ctypes.c_int64 * per_row).from_address(h), dtype=np.int64)
                 for r, (h, _) in host.items()}
        table = [0] * MAXW
        for r, (_, d) in host.items():
            table[r] = d
        bufs = torch.tensor(table, dtype=torch.long, device="cuda")
        order = torch.tensor([3, *rows] + [0] * (MAXW - 3), dtype=torch.int32, device="cuda")
        seqs = torch.zeros(ext.slot_blocks(MAXN, 1) + 1, dtype=torch.int64, device="cuda")
        xs = {r: member_input(r, n) for r in rows}
        x0 = xs[0].cuda()
        out = torch.empty_like(x0)
        # made before the launch: no device work may queue behind the waiting kernel
        peer_words = {r: ll_words_host(xs[r], 1) for r in (1, 2)}
        own = ll_words_host(xs[0], 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ext.slot_all_reduce(x0, out, bufs, ctrl_dev, order, seqs, 0, MAXN, 1, push)
        for r in (1, 2):
            time.sleep(0.02)
            words = peer_words[r]
            at = ((1 * MAXW + r) * half) if push else half
            target = views[0] if push else views[r]
            target[at:at + words.size] = words
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        assert 0.04 <= elapsed < 10, elapsed  # it waited for the words, and no longer
        want = oracle.member_sum([bits(xs[r]) for r in rows])
        assert np.array_equal(bits(out), want)
        # its own words went where the others read them
        if push:
            for r in rows:
                assert np.array_equal(views[r][(MAXW + 0) * half:(MAXW + 0) * half + own.size], own)
        else:
            assert np.array_equal(views[0][half:half + own.size], own)
    finally:
        for h, _ in host.values():
            ext.host_free(h)
        ext.host_free(ctrl_host)


def test_a_member_that_never_comes_is_named_then_released(ext):
    rows, n = [0, 1], 16384
    reg = Region(ext, False, rows)
    try:
        order, seqs = reg.member(rows)
        x0 = member_input(0, n)
        reg.ctrl[0 * CTRL_WORDS + BOUND] = 1_000_000  # name after 1 ms
        out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        xin = x0.cuda()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ext.slot_all_reduce(xin, out, reg.bufs, reg.ctrl_dev, order, seqs, 0, MAXN, 1, False)
        seen = set()
        while time.perf_counter() - t0 < 0.2:
            seen.add(int(reg.ctrl[LATE]))
            time.sleep(0.001)
        reg.ctrl[ABORT] = 1
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        assert (1 << 1) in seen and seen <= {0, 1 << 1}, seen
        assert int(reg.ctrl[LATE]) == 0
        assert elapsed < 10, elapsed
        # the missing member's words sum as zeros
        assert np.array_equal(bits(out), oracle.member_sum([bits(x0), None]))
    finally:
        reg.close()


def test_a_captured_call_replays_with_advancing_sequence_numbers(ext):
    rows, n = [0, 1], 3000
    reg = Region(ext, True, rows)
    try:
        order, seqs = reg.member(rows)
        x0 = member_input(0, n).cuda()
        out = torch.empty_like(x0)
        side = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            ext.slot_all_reduce(x0, out, reg.bufs, reg.ctrl_dev, order, seqs, 0, MAXN, 1, True)
        for seq in (1, 2, 3, 4):
            y = member_input(20 + seq, n)
            reg.stage(0, 1, y, seq=seq)
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(out), oracle.member_sum([bits(x0), bits(y)])), seq
        assert int(seqs[0].item()) == 4
    finally:
        reg.close()


def test_bad_arguments_are_refused(ext):
    from everserve_amd.kernels import KernelError

    reg = Region(ext, False, [0])
    try:
        order, seqs = reg.member([0])
        x = torch.zeros(4, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(KernelError, match="words per thread"):
            ext.slot_all_reduce(x, x, reg.bufs, reg.ctrl_dev, order, seqs, 0, MAXN, 3, False)
        with pytest.raises(KernelError, match="even element count"):
            ext.slot_all_reduce(x[:3], x[:3], reg.bufs, reg.ctrl_dev, order, seqs, 0, MAXN, 1, False)
        with pytest.raises(KernelError, match="row out of range"):
            ext.slot_all_reduce(x, x, reg.bufs, reg.ctrl_dev, order, seqs, 8, MAXN, 1, False)
        with pytest.raises(KernelError, match="too few counters"):
            ext.slot_all_reduce(x, x, reg.bufs, reg.ctrl_dev, order, seqs[:5], 0, MAXN, 1, False)
    finally:
        reg.close()


@pytest.mark.parametrize("push", [False, True])
def test_special_values_round_as_the_oracle_does(ext, push):
    """The slot collective over every bf16 pattern, overflowing sums and exact ties
    (tests/cases.py:special_members): the same bits as the oracle's ordered sum."""
    members = special_members()
    rows = [0, 1, 2]
    xs = {0: bf16_tensor(members[0]), 1: bf16_tensor(members[1]), 2: bf16_tensor(members[3])}
    reg = Region(ext, push, rows)
    try:
        order, seqs = reg.member(rows)
        for r in (1, 2):
            reg.stage(0, r, xs[r], seq=1)
        out = reduce(ext, reg, 0, order, seqs, xs[0], 1)
        torch.cuda.synchronize()
        want = oracle.member_sum([members[0], members[1], members[3]])
        assert np.array_equal(bits(out), want)
    finally:
        reg.close()


@pytest.mark.parametrize("push", [False, True])
def test_a_push_cut_short_is_named_by_the_blocks_still_waiting(ext, push):
    """The dead member's last call delivered block 0's words and none after them
    (core/tests/test_slot_kernel.py:108-122): block 0 sums every member and finishes, the blocks
    still waiting name the member in LATE until ABORT releases them, LATE is cleared after, and
    the words that never came sum as zeros."""
    rows, n = [0, 1], 16384
    per_block = 256  # words of one block at 1 word per thread: 512 elements
    reg = Region(ext, push, rows)
    released = False
    try:
        order, seqs = reg.member(rows)
        x0, x1 = member_input(0, n), member_input(1, n)
        w = ll_words(x1, 1)[:per_block]
        half = MAXN // 2
        if push:
            at = (1 * MAXW + 1) * half  # parity 1, sender 1, in reader 0's buffer
            reg.words[0][at:at + per_block] = w
        else:
            reg.words[1][half:half + per_block] = w  # sender 1's own buffer, parity 1
        reg.ctrl[0 * CTRL_WORDS + BOUND] = 1_000_000  # name after 1 ms
        out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        xin = x0.cuda()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ext.slot_all_reduce(xin, out, reg.bufs, reg.ctrl_dev, order, seqs, 0, MAXN, 1, push)
        seen = set()
        while time.perf_counter() - t0 < 0.2:
            seen.add(int(reg.ctrl[LATE]))
            time.sleep(0.001)
        reg.ctrl[ABORT] = 1
        released = True
        torch.cuda.synchronize()
        assert (1 << 1) in seen and seen <= {0, 1 << 1}, seen
        assert int(reg.ctrl[LATE]) == 0
        got = bits(out)
        full = oracle.member_sum([bits(x0), bits(x1)])
        alone = oracle.member_sum([bits(x0), None])
        e = 2 * per_block
        assert np.array_equal(got[:e], full[:e])  # block 0 had every word
        assert np.array_equal(got[e:], alone[e:])  # the rest never came: zeros
    finally:
        if not released:
            reg.ctrl[ABORT] = 1
            torch.cuda.synchronize()
        reg.close()
