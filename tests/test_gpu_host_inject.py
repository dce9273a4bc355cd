"""The reference's host test hooks on the MI355X (ss_test_inject, ss_test_check_exclusive), against the reference CPU
backend driven by the same calls (reference tests/test_readahead.cpp:190-260, tests/test_exclusive.cpp:530-560).

A one-shot injection makes one step of the read-ahead path fail; the forward must then end as the reference's does:
a read-ahead read that fails (5: at once, 8: after a part, 9: its bytes fail the hash) or cannot be queued (1) leaves
its unit to be read from the file (the fetch falls back, ss_end succeeds); a landing copy that fails before it starts
(3) or after its first piece (4: the buffer is quarantined, the other buffers keep serving) fails the acquire that
needs it with SS_E_IO and the forward; a landing that cannot be queued (2) fails with SS_E_NOMEM and poisons the
context. The copy mutations 6, 7 and 10 (a copy skipping a wait) are refused here with SS_E_UNSUPPORTED.
ss_test_check_exclusive holds between forwards of an exclusive context, also after a landing failure, and is refused
inside a forward or on an inclusive context."""
import ctypes as C
import json

import numpy as np
import pytest

from oracle import fixtures, ref
from tierstream_amd import ss
from tierstream_amd.ss import SsLayerView

pytestmark = pytest.mark.gpu

KiB = 1024
vp, i32 = C.c_void_p, C.c_int32
OK, E_INVALID, E_IO, E_NOMEM, E_BACKEND, E_UNSUPPORTED = 0, 1, 3, 4, 5, 8


def _libs():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    return [("ours", ss._declare(), None), ("reference", ref.lib(), 0)]


def _declare(L):
    for name, args in (("ss_test_inject", [vp, C.c_int]), ("ss_test_check_exclusive", [vp]),
                       ("ss_test_hold_readers", [vp, C.c_int]), ("ss_test_ra_quiesce", [vp]),
                       ("ss_host_prefetch_layer", [vp, C.c_int]), ("ss_check_unit", [vp, C.c_int, C.c_int]),
                       ("ss_host_prefetch", [vp, C.c_int, C.POINTER(i32), C.c_int]), ("ss_layer_all", [vp, C.c_int]),
                       ("ss_release", [vp, C.c_int, vp]), ("ss_stats_reset", [vp])):
        f = getattr(L, name)
        f.restype = C.c_int
        f.argtypes = args
    L.ss_stats_to_json.restype = C.c_int
    L.ss_stats_to_json.argtypes = [vp, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.ss_stats_exclusive_sized.restype = C.c_int
    L.ss_stats_exclusive_sized.argtypes = [vp, C.POINTER(ss.SsExclusiveStats), C.c_uint32]
    L.ss_free.argtypes = [C.c_void_p]


class _Run:
    def __init__(self, L, backend, desc_json, tiers, bkw, okw):
        self.L, self.d, self.p, self.c = L, vp(), vp(), vp()
        b = desc_json.encode()
        assert L.ss_desc_from_json(b, len(b), C.byref(self.d)) == OK
        self.b = ss.budget(**bkw)
        t = (C.c_uint8 * len(tiers))(*tiers)
        assert L.ss_plan_from_tiers(self.d, C.byref(self.b), t, len(tiers), C.byref(self.p)) == OK
        o = ss.options(**okw)
        if backend is not None:
            o.backend = backend
        assert L.ss_open(self.d, C.byref(self.b), self.p, C.byref(o), C.byref(self.c)) == OK, L.ss_last_error()

    def acquire(self, layer):
        v = SsLayerView()
        return self.L.ss_acquire(self.c, layer, None, C.byref(v))

    def routes(self, layer, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        return self.L.ss_layer_routes(self.c, layer, a.ctypes.data_as(C.POINTER(i32)), len(ids))

    def doc(self):
        txt, n = C.c_void_p(), C.c_size_t()
        assert self.L.ss_stats_to_json(self.c, C.byref(txt), C.byref(n)) == OK
        out = json.loads(C.string_at(txt, n.value).decode())
        self.L.ss_free(txt)
        return out

    def layer_major(self, layer, units):
        """A forward over `layer` with every unit routed, each landed unit checked against its file bytes."""
        L, c = self.L, self.c
        out = [L.ss_begin(c, None, 0), L.ss_host_prefetch_layer(c, layer), L.ss_layer_all(c, layer), self.acquire(layer)]
        out += [L.ss_check_unit(c, layer, u) for u in range(units)] if out[-1] == OK else []
        return out + [L.ss_release(c, layer, None), L.ss_end(c)]

    def close(self):
        if self.c:
            self.L.ss_close(self.c)
        self.L.ss_plan_free(self.p)
        self.L.ss_desc_free(self.d)


UNITS = 8


def _model(tmp_path, seed):
    """4 layers x 8 units of 2 x 4 KiB; layers 0-2 pinned, layer 3 read from its file (through the ring)."""
    m = fixtures.write_model(tmp_path, 4, UNITS, [4 * KiB, 4 * KiB], top_k=2, seed=seed, tiers="pinned|disk")
    return m, [1] * 24 + [2] * UNITS


BKW = dict(device_bytes=256 << 20, host_pinned_bytes=8 << 20, ring_slots=16)
OKW = dict(verify_hash=1, staging_bytes=64 * KiB, readahead_units=4)


def _scenario(L, r, what):
    """The reference's injection scenarios on layer 3 (tests/test_readahead.cpp:190-232); the statuses in order."""
    c = r.c
    if what in (5, 8, 9):  # an unattached read fails: the fetch reads the file
        return [L.ss_begin(c, None, 0), L.ss_test_inject(c, what), L.ss_host_prefetch_layer(c, 3),
                L.ss_test_ra_quiesce(c), L.ss_layer_all(c, 3), r.acquire(3)] + \
            [L.ss_check_unit(c, 3, u) for u in range(UNITS)] + [L.ss_release(c, 3, None), L.ss_end(c)]
    if what == 1:  # queueing a read fails: the same
        return [L.ss_begin(c, None, 0), L.ss_test_inject(c, 1), L.ss_host_prefetch_layer(c, 3), L.ss_layer_all(c, 3),
                r.acquire(3)] + [L.ss_check_unit(c, 3, u) for u in range(UNITS)] + \
            [L.ss_release(c, 3, None), L.ss_end(c)]
    if what in (3, 4):  # a landing's copy fails: the acquire and the forward fail; the context serves on
        out = [L.ss_begin(c, None, 0), L.ss_host_prefetch_layer(c, 3), L.ss_test_ra_quiesce(c),
               L.ss_test_inject(c, what), L.ss_layer_all(c, 3), r.acquire(3)]
        out.append(int(L.ss_end(c) != OK))
        for _ in range(2):  # the next forwards serve (4: three buffers left)
            out += r.layer_major(3, UNITS)
        return out
    raise AssertionError(what)


@pytest.mark.parametrize("what", [5, 8, 9, 1, 3, 4])
def test_injected_read_ahead_failures_end_as_the_reference(what, tmp_path, gpu):
    m, tiers = _model(tmp_path, 41)
    seen = {}
    for name, L, backend in _libs():
        _declare(L)
        r = _Run(L, backend, m.desc_json(), tiers, BKW, OKW)
        try:
            L.ss_stats_reset(r.c)
            out = _scenario(L, r, what)
            seen[name] = (out, r.doc()["readahead"])
        finally:
            r.close()
    ours, theirs = seen["ours"], seen["reference"]
    assert ours[0] == theirs[0], (what, ours[0], theirs[0])
    ra = ours[1]
    if what in (5, 8, 9, 1):
        assert all(s == OK for s in ours[0]) and ra["failed"] == 1 and ra["fallback"] == 1, (ours, ra)
        assert ra["failed"] == theirs[1]["failed"] and ra["fallback"] == theirs[1]["fallback"], (ra, theirs[1])
    else:
        assert ours[0][5] == E_IO and ours[0][6] == 1, ours[0]
        assert all(s == OK for s in ours[0][7:]), ours[0]


@pytest.mark.parametrize("order", ["ready", "reading"])
def test_injected_landing_queue_failure_poisons(order, tmp_path, gpu):
    """Reference tests/test_readahead.cpp:236-256: the landing of a read that has ended (Ready) or that is still held
    back (Reading) cannot be queued: SS_E_NOMEM at the acquire, and the context is poisoned (ss_end: SS_E_BACKEND)."""
    m, tiers = _model(tmp_path, 43)
    seen = {}
    for name, L, backend in _libs():
        _declare(L)
        r = _Run(L, backend, m.desc_json(), tiers, BKW, OKW)
        c = r.c
        try:
            out = [L.ss_begin(c, None, 0)]
            if order == "ready":
                out += [L.ss_host_prefetch_layer(c, 3), L.ss_test_ra_quiesce(c), L.ss_test_inject(c, 2),
                        L.ss_layer_all(c, 3)]
            else:
                out += [L.ss_test_hold_readers(c, 1), L.ss_host_prefetch_layer(c, 3), L.ss_layer_all(c, 3),
                        L.ss_test_inject(c, 2), L.ss_test_hold_readers(c, 0)]
            out += [r.acquire(3), L.ss_end(c)]
            seen[name] = out
        finally:
            r.close()
    assert seen["ours"] == seen["reference"], seen
    assert seen["ours"][-2:] == [E_NOMEM, E_BACKEND], seen


def test_copy_mutations_are_refused(tmp_path, gpu):
    m, tiers = _model(tmp_path, 45)
    L = ss._declare()
    _declare(L)
    r = _Run(L, None, m.desc_json(), tiers, BKW, OKW)
    try:
        for what in (6, 7, 10):
            assert L.ss_test_inject(r.c, what) == E_UNSUPPORTED, what
        assert L.ss_test_inject(r.c, 0) == OK
        assert r.layer_major(3, UNITS) == [OK] * (6 + UNITS)
    finally:
        r.close()


def test_check_exclusive(tmp_path, gpu):
    """Reference tests/test_exclusive.cpp:530-560: an exclusive context whose landing read fails (5, parked behind
    held readers) or whose landing copy fails (3) keeps every pinned block accounted for; ss_test_check_exclusive
    holds between forwards, and is SS_E_INVALID inside a forward and on an inclusive context."""
    m = fixtures.write_model(tmp_path, 5, 16, [4 * KiB, 4 * KiB], top_k=2, seed=47, tiers="pinned|disk")
    # layer 2: two residents, two dynamic units, four pinned, eight from the file; the others pinned
    tiers = [1] * 32 + [0, 0] + [2, 2] + [1] * 4 + [2] * 8 + [1] * 32
    bkw = dict(device_bytes=4 << 20, host_pinned_bytes=8 << 20, ring_slots=16, tier_mode=1, host_spare_units=2,
               dynamic_slots_per_layer=2)
    okw = dict(verify_hash=1, pin_planned=0, staging_bytes=64 * KiB, readahead_units=2)
    seen = {}
    for name, L, backend in _libs():
        _declare(L)
        r = _Run(L, backend, m.desc_json(), tiers, bkw, okw)
        c = r.c
        two = np.array([2], dtype=np.int32)
        p2 = two.ctypes.data_as(C.POINTER(i32))
        try:
            out = [L.ss_test_check_exclusive(c)]
            for inj in (5, 3):
                out.append(L.ss_begin(c, None, 0))
                out.append(L.ss_test_check_exclusive(c))  # inside a forward: refused
                if inj == 5:
                    out += [L.ss_test_hold_readers(c, 1), L.ss_host_prefetch(c, 2, p2, 1), L.ss_test_inject(c, 5),
                            r.routes(2, [2]), L.ss_test_hold_readers(c, 0)]
                else:
                    out += [L.ss_host_prefetch(c, 2, p2, 1), L.ss_test_ra_quiesce(c), L.ss_test_inject(c, 3),
                            r.routes(2, [2])]
                out += [r.acquire(2), int(L.ss_end(c) != OK), L.ss_test_check_exclusive(c)]
            # the next forwards serve, every block still accounted for
            for ids in ([0, 2], [2, 5, 6], [7, 8, 9, 10]):
                out += [L.ss_begin(c, None, 0), r.routes(2, ids), r.acquire(2)] + \
                    [L.ss_check_unit(c, 2, u) for u in ids] + [L.ss_release(c, 2, None), L.ss_end(c),
                                                               L.ss_test_check_exclusive(c)]
            x = ss.SsExclusiveStats()
            L.ss_stats_exclusive_sized(c, C.byref(x), C.sizeof(x))
            seen[name] = (out, x.writebacks, x.promoted, x.free_blocks)
        finally:
            r.close()
    assert seen["ours"] == seen["reference"], seen
    out = seen["ours"][0]
    assert out[0] == OK and out[2] == E_INVALID and out.count(E_IO) == 2, out
    # an inclusive context has no blocks to check
    L = ss._declare()
    r = _Run(L, None, m.desc_json(), tiers, dict(bkw, tier_mode=0), dict(okw, readahead_units=0))
    try:
        assert L.ss_test_check_exclusive(r.c) == E_INVALID
    finally:
        r.close()
