"""The build's check of the LDS-copy waits (teco-ops_amd/build.py
check_copy_waits), on hand-written assembly: it must accept a wait that
leaves only younger loads in flight and reject a wait whose count could
include the copies, a barrier before the wait, and M0 written for anything
but a copy; in its M0-only mode (flash_attention.hip) it counts copies and
checks M0 alone."""
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "teco-ops_amd"))
import build  # noqa: E402

HEAD = "_Zkernel:\n"
TAIL = ".Lfunc_end0:\n"
COPY = "\ts_mov_b32 m0, s9\n\tglobal_load_lds_dwordx4 v[4:5], off\n"


def run(body):
    return build.check_copy_waits(HEAD + body + TAIL, "test.hip")


def test_wait_leaving_younger_loads_in_flight_passes():
    body = (COPY + COPY + "\ts_sleep 16\n\tglobal_load_dwordx4 v[0:3], v[6:7], off nt\n"
            "\tglobal_load_dwordx4 v[8:11], v[6:7], off nt\n\ts_waitcnt vmcnt(2)\n\ts_barrier\n")
    assert run(body) == 1


def test_over_wait_passes():
    body = COPY + "\tglobal_load_dwordx4 v[0:3], v[6:7], off nt\n\ts_waitcnt vmcnt(0)\n\ts_barrier\n"
    assert run(body) == 1


def test_loads_sunk_below_the_wait_are_rejected():
    # the failure the check exists for: the W loads moved after the wait
    body = (COPY + "\ts_waitcnt vmcnt(2)\n\ts_barrier\n"
            "\tglobal_load_dwordx4 v[0:3], v[6:7], off nt\n"
            "\tglobal_load_dwordx4 v[8:11], v[6:7], off nt\n")
    with pytest.raises(RuntimeError, match="copies may be in flight"):
        run(body)


def test_barrier_before_the_wait_is_rejected():
    with pytest.raises(RuntimeError, match="barrier before"):
        run(COPY + "\ts_barrier\n\ts_waitcnt vmcnt(0)\n")


def test_m0_outside_a_copy_is_rejected():
    with pytest.raises(RuntimeError, match="M0 used outside"):
        run("\ts_mov_b32 m0, -1\n\tds_read_b32 v0, v1\n" + COPY + "\ts_waitcnt vmcnt(0)\n")


def test_kernels_without_copies_are_skipped():
    assert build.check_copy_waits(HEAD + "\ts_waitcnt vmcnt(5)\n\ts_barrier\n" + TAIL) == 0


def test_m0_only_mode_counts_copies_and_ignores_waits():
    body = COPY + COPY + "\ts_waitcnt vmcnt(9)\n\ts_barrier\n"
    assert build.check_copy_waits(HEAD + body + TAIL, "fa.hip", waits=False) == 2
    with pytest.raises(RuntimeError, match="M0 used outside"):
        build.check_copy_waits(HEAD + "\ts_mov_b32 m0, 0\n" + body + TAIL, "fa.hip", waits=False)
