"""The slot region's control path on the host (everserve_amd.comm.slotkernel.Region): what the
executor writes and every member reads, as core/tests/test_slot_region.py states it."""

import pytest

from everserve_amd.comm.slotkernel import MAXW, Region, check_layout


def test_the_region_records_its_variant_and_carries_control_words_between_mappings(tmp_path):
    r = Region(str(tmp_path / "slot"), create=True, variant="p2p")
    r.set_members(range(4), range(4))
    r.set_members([4], [4])
    assert [r.order(i) for i in range(5)] == [[0, 1, 2, 3]] * 4 + [[4]]
    r.set_members([0, 1, 3, 4], [0, 1, 4, 3])  # rank 2 replaced by the spare's row, in its place
    assert r.order(4) == [0, 1, 4, 3] and r.order(2) == [0, 1, 2, 3]
    r.set_abort(range(MAXW), 1)
    r.set_bound([1], 0.25)
    r.publish(3, bytes(range(64)))
    other = Region(str(tmp_path / "slot"))  # another process's mapping of the same file
    assert other.variant == "p2p"
    assert other.order(4) == [0, 1, 4, 3] and int(other.ctrl[0, 1]) == 1
    assert other.bound(1) == 0.25
    assert other.handle(3, timeout_s=1) == bytes(range(64))
    with pytest.raises(TimeoutError):
        other.handle(2, timeout_s=0.05)  # never published
    other.ctrl[2, 11] = 0b101  # a kernel's late mask, as the watchdog reads it
    assert r.late(2) == {0, 2}
    other.close()
    r.close()


def test_an_order_with_a_row_twice_or_out_of_range_is_refused(tmp_path):
    r = Region(str(tmp_path / "slot"), create=True, variant="host")
    for bad in ([0, 1, 1], [0, MAXW]):
        with pytest.raises(ValueError):
            r.set_members([0], bad)
    r.close()


def test_a_file_that_is_not_a_region_is_refused(tmp_path):
    r = Region(str(tmp_path / "slot"), create=True, variant="host")
    r.header[0] = 0x45565253_4C4F5431  # "EVRSLOT1": the member mask layout
    r.close()
    with pytest.raises(ValueError):
        Region(str(tmp_path / "slot"))
    with pytest.raises(ValueError):
        Region(str(tmp_path / "other"), create=True, variant="nvlink")


def test_the_layout_words_sit_where_the_reference_puts_them(tmp_path):
    # core/everserve/comm/slotkernel.py:71-95: header 16 words, control rows at byte 128, handles
    # after them, host word rows at byte 4096, two parities of 32768 words per row
    r = Region(str(tmp_path / "slot"), create=True, variant="host")
    r.set_abort([2], 7)
    r.set_members([3], [5, 6])
    r.words[1, 5] = 0x1234
    r.close()
    raw = (tmp_path / "slot").read_bytes()
    word = lambda off: int.from_bytes(raw[off:off + 8], "little")  # noqa: E731
    assert word(0) == 0x45565253_4C4F5432
    assert word(128 + (2 * 16 + 1) * 8) == 7
    assert word(128 + (3 * 16 + 2) * 8) == 2 and word(128 + (3 * 16 + 3) * 8) == 5
    assert word(4096 + 1 * 2 * 32768 * 8 + 5 * 8) == 0x1234
    assert len(raw) == 4096 + 8 * 2 * 32768 * 8


def test_the_library_layout_is_checked():
    class Lib:
        MAX_ROWS, CTRL_WORDS, ABORT, LATE, BOUND = 8, 16, 1, 11, 12

    check_layout(Lib())
    Lib.LATE = 10
    with pytest.raises(RuntimeError, match="LATE"):
        check_layout(Lib())
