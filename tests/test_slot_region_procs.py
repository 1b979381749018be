"""The slot region shared by separate processes, on the CPU: what the members and the watchdog see
of each other through the one file (core/everserve/comm/slotkernel.py:71-120,411-429,535-575).

A controller creates the region and starts two member processes, which open the same file. Each
member publishes a buffer handle and its pid. Member 0 waits for member 1's handle, reads the
order the controller set, and then writes a late mask into its own control row, as its kernel
would when it waits on member 1 past its bound. The controller reads that mask, then sets ABORT on
row 1 only. Member 1 sees it and exits, while member 0's abort word stays clear.
"""

import multiprocessing as mp
import os
import time

import pytest

from everserve_amd.comm.slotkernel import Region

TIMEOUT = 60.0


def member(path: str, row: int, q) -> None:
    reg = Region(path)
    reg.publish(row, bytes([row + 1]) * 64)
    reg.set_pid(row, os.getpid())
    if row == 0:
        other = reg.handle(1, TIMEOUT)
        deadline = time.monotonic() + TIMEOUT
        while reg.order(0) != [1, 0] and time.monotonic() < deadline:
            time.sleep(0.01)
        reg.ctrl[0, 11] = 1 << 1  # LATE: its kernel still waits for row 1
        q.put(("member0", other[0], reg.order(0), int(reg.ctrl[0, 1])))
    else:
        deadline = time.monotonic() + TIMEOUT
        while not int(reg.ctrl[1, 1]) and time.monotonic() < deadline:
            time.sleep(0.01)
        q.put(("member1", int(reg.ctrl[1, 1])))
    reg.close()


def test_two_member_processes_and_a_controller_share_one_region(tmp_path):
    path = str(tmp_path / "slot.region")
    ctl = Region(path, create=True, variant="host")
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    procs = [ctx.Process(target=member, args=(path, r, q)) for r in (0, 1)]
    for p in procs:
        p.start()
    try:
        for r in (0, 1):
            assert ctl.handle(r, TIMEOUT) == bytes([r + 1]) * 64
        ctl.set_members([0, 1], [1, 0])
        got = q.get(timeout=TIMEOUT)
        assert got == ("member0", 2, [1, 0], 0)
        assert ctl.late(0) == {1}
        assert {ctl.pid(0), ctl.pid(1)} == {p.pid for p in procs}
        ctl.set_abort([1])
        assert q.get(timeout=TIMEOUT) == ("member1", 1)
        assert int(ctl.ctrl[0, 1]) == 0  # the abort is row 1's alone
    finally:
        for p in procs:
            p.join(timeout=TIMEOUT)
            if p.is_alive():
                p.kill()
        ctl.close()
    assert [p.exitcode for p in procs] == [0, 0]
