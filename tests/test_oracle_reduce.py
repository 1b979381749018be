"""Pins of the oracle's reduction (oracle.member_sum, oracle/oracle.c orc_member_sum_bf16).

The oracle sums in fp32 in the given order from 0.0f and rounds once to bf16 with an integer
round-to-nearest-even (core/everserve/reference/arith/ops.py:63-73). What pins it:

* torch's own float32 arithmetic and its own .to(torch.bfloat16) rounding, on random inputs at
  the reference's sizes {16384, 3000, 2} (core/tests/test_slot_kernel.py:40);
* closed forms: small integers sum exactly in any order; single members round-trip;
* the rounding's special cases (ties to even, overflow to infinity, NaN to 0x7FC0, signed zero,
  subnormals) against torch's conversion;
* the order-sensitive inputs of core/tests/test_slot_kernel.py:50-55 (big, small, -big);
* planted mistakes (reversed order, truncation, bf16 accumulation) that these checks catch.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.cases import bf16_tensor, special_members


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def member_input(rank: int, n: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(1000 * rank + n)
    return torch.randn(n, generator=g).to(torch.bfloat16)


def torch_sum(inputs):
    """torch's fp32 arithmetic and torch's own bf16 rounding (the library routine)."""
    acc = torch.zeros(inputs[0].shape, dtype=torch.float32)
    for x in inputs:
        acc = acc + x.float()
    return acc.to(torch.bfloat16)


@pytest.mark.parametrize("n", [16384, 3000, 2])
@pytest.mark.parametrize("k", [1, 2, 3, 8])
def test_the_sum_is_torchs_fp32_sum_rounded_by_torch(n, k):
    xs = [member_input(r, n) for r in range(k)]
    for order in (list(range(k)), list(range(k))[::-1]):
        got = oracle.member_sum([bf16_bits(xs[r]) for r in order])
        want = bf16_bits(torch_sum([xs[r] for r in order]))
        assert np.array_equal(got, want)


def test_small_integers_sum_exactly_in_any_order():
    rng = np.random.default_rng(0)
    ints = rng.integers(-50, 50, size=(5, 4096))  # |sum| < 256: every integer exact in bf16
    xs = [torch.tensor(row, dtype=torch.float32).to(torch.bfloat16) for row in ints]
    exact = ints.sum(axis=0)
    for order in ([0, 1, 2, 3, 4], [4, 2, 0, 3, 1]):
        got = oracle.member_sum([bf16_bits(xs[r]) for r in order])
        assert np.array_equal(oracle.bf16_to_float(got), exact.astype(np.float32))


def test_one_member_is_itself():
    x = member_input(3, 3000)
    assert np.array_equal(oracle.member_sum([bf16_bits(x)]), bf16_bits(x))


SPECIAL = np.array([
    0x3F808000,  # 1 + 2^-8: a tie, rounds down to the even 0x3F80
    0x3F818000,  # a tie above an odd bf16: rounds up to 0x3F82
    0x3F808001,  # just above a tie: up
    0x3F807FFF,  # just below a tie: down
    0x7F7FFFFF,  # the largest float: rounds to +inf
    0xFF7FFFFF,  # and its negation to -inf
    0x7F800000, 0xFF800000,  # infinities stay
    0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFFFFFFF,  # NaNs of both signs: 0x7FC0
    0x80000000, 0x00000000,  # signed zeros keep their sign
    0x00000001, 0x00400000, 0x807FFFFF,  # subnormals
    0x3F7FFFFF, 0x477FE000, 0x477FF000,  # carries across the exponent
], dtype=np.uint32)


def test_the_rounding_is_torchs_on_its_special_cases():
    f = SPECIAL.view(np.float32)
    nan = np.isnan(f)
    # finite values and infinities: torch's tensor conversion
    want = bf16_bits(torch.from_numpy(f.copy()).to(torch.bfloat16))
    got = oracle.float_to_bf16(f)
    assert np.array_equal(got[~nan], want[~nan])
    # NaNs: torch is not of one mind. c10's scalar rule, which a 0-dim conversion takes and which
    # torch's GPU conversion follows, writes 0x7FC0; its vectorized CPU path writes 0xFFFF; the
    # reference's own kernel has no NaN rule (core/csrc/slot.cu:219-223). The oracle and the HIP
    # kernel keep c10's 0x7FC0; N(0,1) inputs never reach this case.
    scalar = [torch.tensor(float(v)).to(torch.bfloat16).view(torch.int16).item() & 0xFFFF
              for v in f[nan]]
    assert scalar == [0x7FC0] * int(nan.sum())
    assert got[nan].tolist() == scalar
    lib = oracle.lib()
    assert [int(lib.orc_float_to_bf16(float(v))) for v in f] == got.tolist()
    # the C oracle's rounding, reached through a one-member sum
    nan_sum = oracle.member_sum([np.array([0x7FC0, 0xFFC1], dtype=np.uint16)])
    assert nan_sum.tolist() == [0x7FC0, 0x7FC0]


def order_inputs():
    n = 16384
    g = torch.Generator().manual_seed(7)
    big = torch.randn(n, generator=g) * 2.0**20
    small = torch.randn(n, generator=g) * 2.0**-6
    return {0: big.to(torch.bfloat16), 1: small.to(torch.bfloat16), 2: (-big).to(torch.bfloat16)}


def test_the_order_of_the_sum_shows():
    xs = order_inputs()
    in_rank = oracle.member_sum([bf16_bits(xs[r]) for r in (0, 1, 2)])
    in_rows = oracle.member_sum([bf16_bits(xs[r]) for r in (0, 2, 1)])
    assert not np.array_equal(in_rank, in_rows)
    assert np.array_equal(in_rank, bf16_bits(torch_sum([xs[0], xs[1], xs[2]])))
    assert np.array_equal(in_rows, bf16_bits(torch_sum([xs[0], xs[2], xs[1]])))
    # in rank order a small value is absorbed by its large one in fp32 wherever |big| >= 2^17
    # (most samples), and the large ones then cancel to zero
    assert (oracle.bf16_to_float(in_rank) == 0).mean() > 0.5
    # in row order big + (-big) is exactly zero, so the sum is the small member itself
    assert np.array_equal(in_rows, bf16_bits(xs[1]))


@pytest.mark.parametrize("mistake", ["reversed order", "truncation", "bf16 accumulation"])
def test_planted_mistakes_are_caught(mistake):
    xs = order_inputs()
    order = (0, 1, 2)
    want = bf16_bits(torch_sum([xs[r] for r in order]))
    bits = [bf16_bits(xs[r]) for r in order]
    if mistake == "reversed order":
        got = oracle.member_sum(bits[::-1])
    elif mistake == "truncation":
        acc = np.zeros(len(bits[0]), dtype=np.float32)
        for b in bits:
            acc += oracle.bf16_to_float(b)
        got = (acc.view(np.uint32) >> 16).astype(np.uint16)
        # truncation differs from rounding on random sums of mixed signs
        ys = [bf16_bits(member_input(r, 4096)) for r in range(3)]
        acc = np.zeros(4096, dtype=np.float32)
        for y in ys:
            acc += oracle.bf16_to_float(y)
        assert not np.array_equal((acc.view(np.uint32) >> 16).astype(np.uint16),
                                  oracle.member_sum(ys))
        return
    else:
        acc = np.zeros(len(bits[0]), dtype=np.uint16)
        for b in bits:
            acc = oracle.float_to_bf16(oracle.bf16_to_float(acc) + oracle.bf16_to_float(b))
        got = acc
        ys = [bf16_bits(member_input(r, 4096)) for r in range(8)]
        acc = np.zeros(4096, dtype=np.uint16)
        for y in ys:
            acc = oracle.float_to_bf16(oracle.bf16_to_float(acc) + oracle.bf16_to_float(y))
        assert not np.array_equal(acc, oracle.member_sum(ys))
        return
    assert not np.array_equal(got, want)


def test_the_protocol_sums_zeros_for_missing_members_and_names_them():
    xs = {r: bf16_bits(member_input(r, 3000)) for r in range(4)}
    out, reason, late = oracle.reduce_protocol(xs, {0: 5, 1: 5, 2: 4, 3: 5}, [3, 2, 1, 0], 5)
    assert (reason, late) == (oracle.REDUCE_TIMED_OUT, 1 << 2)
    assert np.array_equal(out, oracle.member_sum([xs[3], None, xs[1], xs[0]]))
    # +0.0 for the missing member: the same as leaving it out, except that -0.0 sums become +0.0
    assert np.array_equal(out, oracle.member_sum([xs[3], xs[1], xs[0], np.zeros(3000, np.uint16)]))
    out, reason, late = oracle.reduce_protocol(xs, {r: 5 for r in range(4)}, [0, 1, 2, 3], 5)
    assert (reason, late) == (oracle.REDUCE_DONE, 0)
    out, reason, late = oracle.reduce_protocol(xs, {0: 5}, [0, 1], 5, abort=True)
    assert (reason, late) == (oracle.REDUCE_ABORTED, 1 << 1)


@pytest.mark.parametrize("n", [16384, 3000, 2])
def test_the_cpu_path_member_sum_is_the_oracles(n):
    """oracle/cpu_path.member_sum is the reduce that bench.py times as the CPU baseline: it must
    be the same arithmetic, bit for bit, as the checker."""
    from oracle import cpu_path

    xs = [member_input(r, n) for r in range(8)]
    got = bf16_bits(cpu_path.member_sum(xs))
    assert np.array_equal(got, oracle.member_sum([bf16_bits(x) for x in xs]))


SPECIAL_ORDERS = [[0], [0, 1], [1, 0, 2], [0, 3], [3, 0], [2, 0, 1, 3]]


@pytest.mark.parametrize("order", SPECIAL_ORDERS)
def test_special_values_sum_as_torch_does(order):
    """Every bf16 pattern through the sum: torch's fp32 adds and bf16 rounding give the same bits
    except at NaN, where the oracle keeps c10's 0x7FC0 (see the rounding test above)."""
    members = special_members()
    got = oracle.member_sum([members[r] for r in order])
    want = bf16_bits(torch_sum([bf16_tensor(members[r]) for r in order]))
    nan = np.isnan(oracle.bf16_to_float(want))
    assert np.array_equal(got[~nan], want[~nan])
    assert (got[nan] == 0x7FC0).all()
    if order == [0, 3]:
        # the ties: half an ulp added to an odd mantissa rounds up, to an even one stays
        v = members[0]
        tie = (members[3] != 0) & ((v & 0x7F80) != 0x7F80)
        odd = (v & 1) == 1
        assert tie.sum() > 50_000
        assert np.array_equal(got[tie & ~odd], v[tie & ~odd])
        assert np.array_equal(got[tie & odd], v[tie & odd] + 1)
