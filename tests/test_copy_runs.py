"""Host contract: which pinned-block copies go as one host-to-device copy (tsa_test_copy_runs, the rule the MI355X
executor applies when an engine call returns). A run is consecutive orders of one layer whose sources sit in one pinned
allocation and destinations in one device allocation, each exactly one slot and one block further on; the span it
copies must never cover a slot or block of another unit (the regression: two units two slots apart, with a live unit
in the slot between, were once merged and the copy overwrote the middle slot)."""
import ctypes as C

import numpy as np
import pytest

from tierstream_amd import ss

U = 9 * 1024 * 1024  # a unit of 9 MiB: slots and blocks one unit apart
SRC, DST = 1 << 40, 1 << 44  # allocation bases


def _runs(orders, unit=U, cap=64 << 20):
    L = ss._declare()
    f = L.tsa_test_copy_runs
    f.restype = C.c_int
    u64p, i32p = C.POINTER(C.c_uint64), C.POINTER(C.c_int32)
    f.argtypes = [i32p, i32p, i32p, u64p, u64p, C.c_size_t, C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
    n = len(orders)
    arr = lambda k, t: np.ascontiguousarray([o[k] for o in orders], dtype=t)
    layer, sa, da = arr(0, np.int32), arr(1, np.int32), arr(2, np.int32)
    src, dst = arr(3, np.uint64), arr(4, np.uint64)
    out = np.zeros(max(n, 1), dtype=np.uint32)
    st = f(layer.ctypes.data_as(i32p), sa.ctypes.data_as(i32p), da.ctypes.data_as(i32p), src.ctypes.data_as(u64p),
           dst.ctypes.data_as(u64p), n, unit, cap, out.ctypes.data_as(C.POINTER(C.c_uint32)))
    assert st == 0
    return out[:n].tolist()


def _o(block, slot, layer=0, sa=0, da=0, stride=U):
    return (layer, sa, da, SRC + block * stride, DST + slot * stride)


def test_neighbours_merge():
    assert _runs([_o(3, 10), _o(4, 11), _o(5, 12)]) == [0, 0, 0]


def test_a_slot_between_is_never_covered():
    # units two blocks and two slots apart: equal steps, but the slot between holds another unit
    assert _runs([_o(3, 10), _o(5, 12)]) == [0, 1]
    assert _runs([_o(3, 10), _o(4, 11), _o(6, 13), _o(7, 14)]) == [0, 0, 1, 1]


def test_steps_must_agree_on_both_sides():
    assert _runs([_o(3, 10), _o(4, 12)]) == [0, 1]  # next block, a slot further
    assert _runs([_o(3, 10), _o(2, 11)]) == [0, 1]  # a block behind
    assert _runs([_o(3, 10), _o(4, 9)]) == [0, 1]   # a slot behind


def test_allocations_and_layers_split_runs():
    assert _runs([_o(3, 10), _o(4, 11, sa=1)]) == [0, 1]  # another pinned chunk
    assert _runs([_o(3, 10), _o(4, 11, da=1)]) == [0, 1]  # another ring class / pool
    assert _runs([_o(3, 10), _o(4, 11, layer=1)]) == [0, 1]
    assert _runs([_o(3, 10, sa=-1), _o(4, 11, sa=-1)]) == [0, 1]  # not pinned blocks


def test_padded_strides():
    # a 5,000,000-byte unit: blocks 4 KiB-aligned (5,001,216), slots 256-aligned (5,000,192): steps never agree
    n = 5_000_000
    hs, st = (n + 4095) // 4096 * 4096, (n + 255) // 256 * 256
    orders = [(0, 0, 0, SRC + k * hs, DST + k * st) for k in range(4)]
    assert _runs(orders, unit=n) == [0, 1, 2, 3]
    # equal padded strides (both 4 KiB-aligned) merge
    orders = [(0, 0, 0, SRC + k * hs, DST + k * hs) for k in range(4)]
    assert _runs(orders, unit=n) == [0, 0, 0, 0]


@pytest.mark.parametrize("cap,want", [(64 << 20, [0] * 7 + [1] * 3), (U, list(range(10))), (3 * U, [0, 0, 0, 1, 1, 1,
                                                                                                    2, 2, 2, 3])])
def test_cap_bounds_the_span(cap, want):
    assert _runs([_o(k, k) for k in range(10)], cap=cap) == want


def test_random_orders_never_cover_a_foreign_slot():
    rng = np.random.default_rng(5)
    for _ in range(200):
        k = int(rng.integers(1, 40))
        blocks = rng.choice(64, size=k, replace=False)
        slots = rng.choice(64, size=k, replace=False)
        if rng.integers(0, 2):  # make neighbours likely
            blocks, slots = np.sort(blocks), np.sort(slots)
        orders = [_o(int(b), int(s)) for b, s in zip(blocks, slots)]
        run_of = _runs(orders)
        for r in set(run_of):
            mem = [i for i, x in enumerate(run_of) if x == r]
            assert mem == list(range(mem[0], mem[-1] + 1))  # runs are consecutive orders
            b = [int(blocks[i]) for i in mem]
            s = [int(slots[i]) for i in mem]
            # the run's span covers exactly its own blocks and slots
            assert b == list(range(b[0], b[0] + len(b))) and s == list(range(s[0], s[0] + len(s)))
