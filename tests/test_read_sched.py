"""The host contract's reader rules on the CPU (no GPU): which queued file read a free reader starts
(tsa_test_read_sched drives the executor's scheduler single-threaded) and how an unaligned range is covered by aligned
reads (tsa_test_cover_windows).

The scheduling rules are the reference's reader priority (src/stream_ctx.cpp:353-431): demand reads first, then
read-ahead reads on at most max(1, readers - 1) readers (any reader once the context stops), then a speculative read
while at most one demand read runs; a promoted guess and a read-ahead a landing waits for go to the head of the demand
reads. The covering windows are checked against what O_DIRECT requires of each read and against the range they cover."""
import ctypes as C

import numpy as np
import pytest

from tierstream_amd import ss

DEMAND, AHEAD, GUESS = 0, 1, 2
PUSH, RAISE, REMOVE, TAKE, END, HOLD, STOP = range(7)


def _run(ops, readers=2):
    L = ss._declare()
    f = L.tsa_test_read_sched
    f.restype = C.c_int
    i32p = C.POINTER(C.c_int32)
    f.argtypes = [i32p, C.c_size_t, C.c_int, i32p, C.POINTER(C.c_size_t)]
    a = np.ascontiguousarray(np.array(ops, dtype=np.int32).reshape(-1), dtype=np.int32)
    out = np.zeros(2 * max(len(ops), 1), dtype=np.int32)
    n = C.c_size_t()
    assert f(a.ctypes.data_as(i32p), len(ops), readers, out.ctypes.data_as(i32p), C.byref(n)) == 0
    return [(int(out[2 * k]), int(out[2 * k + 1])) for k in range(n.value)]


def _take():
    return (TAKE, 0, 0)


def test_priority_demand_then_read_ahead_then_guess():
    got = _run([(PUSH, GUESS, 1), (PUSH, AHEAD, 2), (PUSH, DEMAND, 3), _take(), _take(), _take(), _take()])
    assert got == [(3, DEMAND), (2, AHEAD), (1, GUESS), (-1, -1)]


def test_arrival_order_inside_a_class():
    got = _run([(PUSH, DEMAND, 5), (PUSH, DEMAND, 4), (PUSH, DEMAND, 6), _take(), _take(), _take()])
    assert [g[0] for g in got] == [5, 4, 6]


@pytest.mark.parametrize("readers,cap", [(1, 1), (2, 1), (3, 2), (4, 3), (8, 7)])
def test_read_ahead_leaves_a_reader_for_demands(readers, cap):
    ops = [(PUSH, AHEAD, i) for i in range(cap + 2)] + [_take() for _ in range(cap + 1)]
    got = _run(ops, readers)
    assert [g[0] for g in got] == list(range(cap)) + [-1]
    # one read-ahead ends: the next one starts
    got = _run(ops + [(END, AHEAD, 0), _take()], readers)
    assert got[-1] == (cap, AHEAD)


def test_a_guess_waits_while_two_demands_run():
    ops = [(PUSH, DEMAND, 1), (PUSH, DEMAND, 2), _take(), _take(), (PUSH, GUESS, 9), _take()]
    assert _run(ops, 4)[-1] == (-1, -1)
    assert _run(ops + [(END, DEMAND, 0), _take()], 4)[-1] == (9, GUESS)


def test_a_demand_is_never_held_back():
    ops = [(PUSH, DEMAND, i) for i in range(5)] + [_take() for _ in range(5)]
    assert [g[0] for g in _run(ops, 1)] == [0, 1, 2, 3, 4]


def test_raise_puts_a_read_at_the_head_of_the_demands():
    ops = [(PUSH, DEMAND, 1), (PUSH, GUESS, 7), (PUSH, AHEAD, 8), (RAISE, GUESS, 7), (RAISE, AHEAD, 8),
           _take(), _take(), _take(), _take()]
    assert _run(ops, 2) == [(8, DEMAND), (7, DEMAND), (1, DEMAND), (-1, -1)]


def test_raise_or_remove_of_a_read_not_queued_there_changes_nothing():
    ops = [(PUSH, AHEAD, 3), (RAISE, GUESS, 3), (REMOVE, DEMAND, 3), _take()]
    assert _run(ops, 2) == [(3, AHEAD)]
    assert _run([(PUSH, AHEAD, 3), (REMOVE, AHEAD, 3), _take()], 2) == [(-1, -1)]


def test_hold_and_stop():
    ops = [(HOLD, 0, 1), (PUSH, DEMAND, 1), _take(), (HOLD, 0, 0), _take()]
    assert _run(ops) == [(-1, -1), (1, DEMAND)]
    # a stop overrides a hold, and lets read-ahead reads drain past their cap
    ops = [(PUSH, AHEAD, 1), (PUSH, AHEAD, 2), _take(), (HOLD, 0, 1), _take(), (STOP, 0, 0), _take()]
    assert _run(ops, 2) == [(1, AHEAD), (-1, -1), (2, AHEAD)]


def _windows(off, n, al, cap):
    L = ss._declare()
    f = L.tsa_test_cover_windows
    f.restype = C.c_int
    f.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64), C.c_size_t,
                  C.POINTER(C.c_size_t)]
    mx = n // cap + 2
    out = np.zeros(5 * mx, dtype=np.uint64)
    k = C.c_size_t()
    assert f(off, n, al, cap, out.ctypes.data_as(C.POINTER(C.c_uint64)), mx, C.byref(k)) == 0
    return [tuple(int(x) for x in out[5 * i:5 * i + 5]) for i in range(k.value)]


@pytest.mark.parametrize("seed", range(200))
def test_cover_windows_tile_the_range_with_aligned_reads(seed):
    rng = np.random.default_rng(seed)
    al = int(rng.choice([1, 512, 4096]))
    cap = al * int(rng.integers(1, 40)) if al > 1 else int(rng.integers(1, 20000))
    off = int(rng.integers(0, 1 << 22))
    n = int(rng.integers(0, 8 * cap + 3))
    w = _windows(off, n, al, cap)
    pos = 0
    for at, ln, a0, span, lead in w:
        assert at == pos and 0 < ln <= cap
        assert a0 % al == 0 and span % al == 0  # what O_DIRECT needs of the read
        assert a0 + lead == off + at and lead < al  # the piece starts inside the first aligned block
        assert a0 + span >= off + at + ln and span < ln + 2 * al  # covers the piece, at most one block each side
        pos += ln
    assert pos == n
    assert len(w) == (n + cap - 1) // cap
