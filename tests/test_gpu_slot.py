"""ss_dg_slot and ts_dg_slot as an engine kernel calls them, on a synthetic view: the reference's own device vectors
(tests/test_ts_device.cu:38-41: two gated layers of 3 and 2 units, slot_of {4, -1, 2, 5, -1}, guard slot 7; a resident
id, an absent id, out-of-range ids, and an aborted view), and the absent_err rule of include/strix_stream/ss.h:950-960
(an absent entry without abort sets absent_err; an out-of-range id or an aborted view does not)."""
import ctypes as C

import numpy as np
import pytest

from tierstream_amd import check, ss

pytestmark = pytest.mark.gpu

SLOT_OF = [4, -1, 2, 5, -1]
UNIT_BASE = [0, 3, 5]
QUERIES = [(0, 0), (0, 1), (0, 2), (0, 3), (0, -1), (1, 0), (1, 1), (1, 2)]
WANT_LIVE = [4, 7, 2, 7, 7, 5, 7, 7]


def probe(queries, aborted, with_absent):
    E = ss.engine()
    E.tse_slot_probe.restype = C.c_int
    g = np.array([q[0] for q in queries], dtype=np.uint32)
    ids = np.array([q[1] for q in queries], dtype=np.int32)
    so = np.array(SLOT_OF, dtype=np.int32)
    ub = np.array(UNIT_BASE, dtype=np.uint32)
    out_ss = np.full(len(queries), -99, dtype=np.int32)
    out_ts = np.full(len(queries), -99, dtype=np.int32)
    absent = C.c_uint32(0)
    P = lambda a, t: a.ctypes.data_as(C.POINTER(t))  # noqa: E731
    check(E.tse_slot_probe(P(so, C.c_int32), C.c_uint32(len(so)), P(ub, C.c_uint32), C.c_uint32(2), C.c_uint32(7),
                           C.c_uint32(aborted), C.c_int(with_absent), P(g, C.c_uint32), P(ids, C.c_int32),
                           C.c_uint32(len(queries)), P(out_ss, C.c_int32), P(out_ts, C.c_int32), C.byref(absent)))
    return list(out_ss), list(out_ts), absent.value


@pytest.mark.parametrize("aborted", [0, 1])
def test_reference_vectors(gpu, aborted):
    got_ss, got_ts, _ = probe(QUERIES, aborted, with_absent=0)
    want = [7] * len(QUERIES) if aborted else WANT_LIVE
    assert got_ss == want and got_ts == want


def test_absent_err_rule(gpu):
    _, _, a = probe([(0, 0), (0, 2), (1, 0)], 0, with_absent=1)  # residents only
    assert a == 0
    _, _, a = probe([(0, 3), (0, -1), (1, 2)], 0, with_absent=1)  # out of range: guard, no absent_err
    assert a == 0
    _, _, a = probe([(0, 1)], 0, with_absent=1)  # absent without abort
    assert a == 1
    _, _, a = probe([(0, 1), (1, 1)], 1, with_absent=1)  # aborted: the guard, nothing reported
    assert a == 0
