"""Host contract error paths and read-ahead states on the MI355X, against the reference CPU backend driven by the same
calls (reference tests/test_runtime.cpp:216-256, tests/test_readahead.cpp:387-476): a unit whose file bytes differ from
the descriptor hash fails the acquire that needs it with SS_E_HASH (verify_hash = 1), the forward's end reports it
again, and the next forward serves the healthy units; a stream ring too small for a layer's transient units is
SS_E_CAPACITY naming the ring, not a hang, and the forward still ends cleanly; read-ahead landings from reads that have
ended and from reads held back (the reference's ss_test_hold_readers / ss_test_ra_quiesce hooks); a close with reads in
flight. Both libraries see the same descriptor, plan tiers, budget and options; every status must be the reference's."""
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
OK, E_HASH, E_CAPACITY = 0, 7, 6


def _libs():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    return [("ours", ss._declare(), None), ("reference", ref.lib(), 0)]


class _Run:
    """One context of library L over (descriptor, tiers, budget, options); backend: the options' backend (None: the
    library's default)."""

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
        self.open_status = L.ss_open(self.d, C.byref(self.b), self.p, C.byref(o), C.byref(self.c))

    def routes(self, layer, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        return self.L.ss_layer_routes(self.c, layer, a.ctypes.data_as(C.POINTER(i32)), len(ids))

    def acquire(self, layer):
        v = SsLayerView()
        st = self.L.ss_acquire(self.c, layer, None, C.byref(v))
        return st, v

    def close(self):
        if self.c:
            self.L.ss_close(self.c)
        self.L.ss_plan_free(self.p)
        self.L.ss_desc_free(self.d)


def _model(tmp_path, corrupt=None):
    m = fixtures.write_model(tmp_path, 3, 8, [64 * KiB] * 3, top_k=2, seed=21, tiers="pinned|disk")
    d = json.loads(m.desc_json())
    if corrupt is not None:  # a descriptor hash the file bytes do not have
        L, u = corrupt
        h = int(d["layers"][L]["hash"][u], 16)
        d["layers"][L]["hash"][u] = f"{h ^ 0x5A5A5A5A5A5A5A5A:016x}"
    return m, json.dumps(d)


def test_hash_mismatch_is_reported(tmp_path, gpu):
    m, desc = _model(tmp_path, corrupt=(1, 3))
    st = (m.unit_bytes + 255) // 256 * 256
    tiers = [2] * (3 * 8)  # nothing resident or pinned: layer 1's units are read from the file at their first use
    bkw = dict(device_bytes=8 * st + st // 2, host_pinned_bytes=64 << 20, ring_slots=8)
    okw = dict(verify_hash=1, staging_buffers=2, staging_bytes=1 << 20)
    seen = {}
    for name, L, backend in _libs():
        r = _Run(L, backend, desc, tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            out = [L.ss_begin(r.c, None, 0), r.routes(1, [2, 3])]
            a, _ = r.acquire(1)
            out.append(a)
            msg = L.ss_last_error().decode()
            out.append(L.ss_end(r.c))
            # the next forward: the healthy unit only
            out += [L.ss_begin(r.c, None, 0), r.routes(1, [2])]
            a, v = r.acquire(1)
            out += [a, int(v.table_host[2] != 0) if a == OK else -1, L.ss_release(r.c, 1, None), L.ss_end(r.c)]
            seen[name] = (out, msg)
        finally:
            r.close()
    ours, theirs = seen["ours"], seen["reference"]
    assert ours[0] == theirs[0], (ours, theirs)
    assert ours[0][2] == E_HASH and ours[0][3] != OK and ours[0][4:] == [OK, OK, OK, 1, OK, OK], ours
    assert "(1, 3)" in ours[1] or "1, 3" in ours[1], ours[1]  # the message names the unit


def test_ring_too_small_is_an_error_not_a_hang(tmp_path, gpu):
    m, desc = _model(tmp_path)
    st = (m.unit_bytes + 255) // 256 * 256
    # layer 1: two residents, six units read from the file through a 4-slot ring; ss_layer_all needs six ring slots
    tiers = [2] * 8 + [0, 0] + [2] * 6 + [2] * 8
    bkw = dict(device_bytes=(2 + 4) * st + st // 2, host_pinned_bytes=64 << 20, ring_slots=4)
    okw = dict(staging_buffers=2, staging_bytes=1 << 20)
    seen = {}
    for name, L, backend in _libs():
        r = _Run(L, backend, desc, tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            out = [L.ss_begin(r.c, None, 0), L.ss_layer_all(r.c, 1)]
            a, _ = r.acquire(1)
            out.append(a)
            msg = L.ss_last_error().decode()
            out.append(L.ss_end(r.c))
            seen[name] = (out, msg)
        finally:
            r.close()
    ours, theirs = seen["ours"], seen["reference"]
    assert ours[0] == theirs[0] == [OK, OK, E_CAPACITY, OK], (ours, theirs)
    assert "ring" in ours[1] and "ring" in theirs[1], (ours[1], theirs[1])


def _declare_hooks(L):
    for name, args in (("ss_test_hold_readers", [vp, C.c_int]), ("ss_test_ra_quiesce", [vp]),
                       ("ss_host_prefetch", [vp, C.c_int, C.POINTER(i32), C.c_int]), ("ss_check_unit", [vp, C.c_int, C.c_int]),
                       ("ss_stats_reset", [vp])):
        f = getattr(L, name)
        f.restype = C.c_int
        f.argtypes = args
    L.ss_stats_exclusive_sized.restype = C.c_int
    L.ss_stats_exclusive_sized.argtypes = [vp, C.POINTER(ss.SsExclusiveStats), C.c_uint32]
    L.ss_stats_total.restype = C.c_int
    L.ss_stats_total.argtypes = [vp, C.POINTER(ss.SsLayerStats)]
    L.ss_stats_to_json.restype = C.c_int
    L.ss_stats_to_json.argtypes = [vp, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.ss_free.argtypes = [C.c_void_p]


def _doc(L, c):
    txt, n = C.c_void_p(), C.c_size_t()
    assert L.ss_stats_to_json(c, C.byref(txt), C.byref(n)) == OK
    out = json.loads(C.string_at(txt, n.value).decode())
    L.ss_free(txt)
    return out


@pytest.mark.parametrize("excl", [1, 0])
@pytest.mark.parametrize("reading", [0, 1])
def test_read_ahead_lands_in_admitted_slots(excl, reading, tmp_path, gpu):
    """Reference tests/test_readahead.cpp:410-476: two file-backed units asked for by ss_host_prefetch, then routed and
    admitted into the layer's pool (evicting two residents), land from their read-ahead buffers, whether the reads
    have ended (ss_test_ra_quiesce: Ready) or are still held back (ss_test_hold_readers: the landing waits for the
    read). Exclusive: the landings go into the victims' slots after their write-backs; inclusive: the victims just
    leave. Each unit's file bytes count once (its read), the landing copy nowhere; the evicted residents then come
    back from their blocks (exclusive) or their file. Statuses, stats, the read-ahead object and the exclusive
    counters must be the reference's."""
    m = fixtures.write_model(tmp_path, 3, 8, [4 * KiB, 4 * KiB], top_k=2, seed=23, tiers="pinned|disk")
    desc = m.desc_json()
    tiers = [1] * 8 + [0, 0, 0, 0, 2, 2, 2, 2] + [1] * 8
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=4 << 20, ring_slots=16, tier_mode=excl)
    okw = dict(verify_hash=1, pin_planned=0, staging_bytes=64 * KiB, readahead_units=2)
    seen = {}
    for name, L, backend in _libs():
        _declare_hooks(L)
        r = _Run(L, backend, desc, tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            L.ss_stats_reset(r.c)
            ids = np.array([5, 6], dtype=np.int32)
            out = [L.ss_begin(r.c, None, 0)]
            if reading:
                out.append(L.ss_test_hold_readers(r.c, 1))
            out.append(L.ss_host_prefetch(r.c, 1, ids.ctypes.data_as(C.POINTER(i32)), 2))
            if not reading:
                out.append(L.ss_test_ra_quiesce(r.c))
            out.append(r.routes(1, [5, 6]))
            if reading:
                out.append(L.ss_test_hold_readers(r.c, 0))
            a, v = r.acquire(1)
            out += [a, L.ss_check_unit(r.c, 1, 5), L.ss_check_unit(r.c, 1, 6), L.ss_release(r.c, 1, None),
                    L.ss_end(r.c)]
            doc = _doc(L, r.c)
            t = ss.SsLayerStats()
            L.ss_stats_total(r.c, C.byref(t))
            x = ss.SsExclusiveStats()
            L.ss_stats_exclusive_sized(r.c, C.byref(x), C.sizeof(x))
            first = (doc["readahead"], t.as_dict(), x.writebacks)
            # 5 and 6 are resident now; the evicted residents come back
            out += [L.ss_begin(r.c, None, 0), r.routes(1, [0, 1, 5, 6])]
            a, v = r.acquire(1)
            out += [a] + [L.ss_check_unit(r.c, 1, u) for u in (0, 1, 5, 6)] + [L.ss_release(r.c, 1, None),
                                                                               L.ss_end(r.c)]
            L.ss_stats_total(r.c, C.byref(t))
            seen[name] = (out, first, t.as_dict())
        finally:
            r.close()
    ours, theirs = seen["ours"], seen["reference"]
    assert all(s == OK for s in ours[0]), ours[0]
    assert ours[0] == theirs[0]
    ra, tot1, wb = ours[1]
    ub = m.unit_bytes
    assert ra["landed"] == 2 and ra["unused"] == 0 and ra["bytes"] == 2 * ub, ra
    assert tot1["bytes_disk"] == 2 * ub and tot1["admitted"] == 2 and tot1["bytes_pinned"] == 0, tot1
    assert wb == (2 if excl else 0)
    assert ours[2]["hits"] == 2 and ours[2]["bytes_disk"] == (2 if excl else 4) * ub, ours[2]
    drop = ("wait_ns",)
    assert {k: v for k, v in tot1.items() if k not in drop} == {k: v for k, v in theirs[1][1].items() if k not in drop}
    assert ra == theirs[1][0] and wb == theirs[1][2]
    assert {k: v for k, v in ours[2].items() if k not in drop} == {k: v for k, v in theirs[2].items() if k not in drop}


def test_close_with_reads_in_flight(tmp_path, gpu):
    """Reference tests/test_readahead.cpp:387-408: a context closed with read-ahead reads queued behind held readers
    (no ss_end) closes cleanly; a new context on the same files then serves."""
    m = fixtures.write_model(tmp_path, 4, 16, [4 * KiB, 4 * KiB], top_k=2, seed=29, tiers="pinned|disk")
    desc = m.desc_json()
    tiers = [1] * 16 + [2] * 48
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=8 << 20, ring_slots=16)
    okw = dict(verify_hash=1, staging_bytes=64 * KiB, readahead_units=2)
    L = ss._declare()
    _declare_hooks(L)
    r = _Run(L, None, desc, tiers, bkw, okw)
    try:
        assert r.open_status == OK, L.ss_last_error()
        assert L.ss_test_hold_readers(r.c, 1) == OK
        assert L.ss_begin(r.c, None, 0) == OK
        L.ss_host_prefetch_layer.restype = C.c_int
        L.ss_host_prefetch_layer.argtypes = [vp, C.c_int]
        assert L.ss_host_prefetch_layer(r.c, 3) == OK
        assert L.ss_layer_all(r.c, 3) == OK
        assert L.ss_test_hold_readers(r.c, 0) == OK
    finally:
        r.close()  # (the forward never ended)
    r = _Run(L, None, desc, tiers, bkw, okw)
    try:
        assert r.open_status == OK
        assert L.ss_begin(r.c, None, 0) == OK and r.routes(2, [1, 2]) == OK
        a, _ = r.acquire(2)
        assert a == OK and L.ss_check_unit(r.c, 2, 1) == OK and L.ss_check_unit(r.c, 2, 2) == OK
        assert L.ss_release(r.c, 2, None) == OK and L.ss_end(r.c) == OK
    finally:
        r.close()


def _declare_more(L):
    for name, res, args in (("ss_seed", C.c_int, [vp, C.c_int, C.POINTER(i32), C.c_int]),
                            ("ss_stats_layer", C.c_int, [vp, C.c_int, C.POINTER(ss.SsLayerStats)]),
                            ("ss_prefetch", C.c_int, [vp, C.c_int, C.POINTER(i32), C.c_int, C.c_int]),
                            ("ss_layer_all", C.c_int, [vp, C.c_int]),
                            ("ss_release", C.c_int, [vp, C.c_int, vp])):
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _ids(*xs):
    a = np.array(xs, dtype=np.int32)
    return a, a.ctypes.data_as(C.POINTER(i32))


def _streams():
    import tierstream_amd as tsa
    out = []
    for _ in range(2):
        s = C.c_void_p()
        tsa.check(tsa.lib().tsa_stream_create(C.byref(s)))
        out.append(s)
    return out


def test_call_order_errors(tmp_path, gpu):
    """Reference tests/test_runtime.cpp:291-311: calls out of order are SS_E_INVALID and leave the context usable."""
    m = fixtures.write_model(tmp_path, 3, 8, [4 * KiB, 4 * KiB], top_k=2, seed=31, tiers="pinned|disk")
    tiers = [2] * 24
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=0, ring_slots=8)
    seen = {}
    for name, L, backend in _libs():
        _declare_more(L)
        r = _Run(L, backend, m.desc_json(), tiers, bkw, dict(staging_bytes=64 * KiB))
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            bad, p = _ids(99)
            out = [r.acquire(1)[0], L.ss_begin(r.c, None, 0), L.ss_begin(r.c, None, 0), r.acquire(1)[0],
                   L.ss_layer_routes(r.c, 1, p, 1), L.ss_layer_all(r.c, 2), r.acquire(2)[0], L.ss_end(r.c),
                   L.ss_release(r.c, 2, None), L.ss_end(r.c), L.ss_release(r.c, 2, None)]
            seen[name] = out
        finally:
            r.close()
    E = 1  # SS_E_INVALID
    assert seen["ours"] == seen["reference"] == [E, OK, E, E, E, OK, OK, E, OK, OK, E], seen


def test_one_stream_per_forward_and_seed_rollback(tmp_path, gpu):
    """Reference tests/test_runtime.cpp:313-357: a seed with an invalid id is refused whole; a seed whose unit fails
    its hash is rolled back (SS_E_HASH) while the healthy one stays; a forward uses one engine stream (another one is
    SS_E_INVALID), the next forward may use another; the rolled-back unit is read again and fails again, not served
    as a hit on garbage."""
    m, desc = _model(tmp_path, corrupt=(1, 3))
    st = (m.unit_bytes + 255) // 256 * 256
    tiers = [2] * 24
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=0, ring_slots=4, dynamic_slots_per_layer=4)
    okw = dict(verify_hash=1, pin_planned=0, staging_buffers=2, staging_bytes=1 << 20)
    s1, s2 = _streams()
    seen = {}
    for name, L, backend in _libs():
        _declare_more(L)
        r = _Run(L, backend, desc, tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            mixed, pm = _ids(2, 99)
            seed, ps = _ids(2, 3)
            two, p2 = _ids(2)
            three, p3 = _ids(3)
            out = [L.ss_seed(r.c, 1, pm, 2), L.ss_seed(r.c, 1, ps, 2), L.ss_begin(r.c, None, 0),
                   L.ss_layer_routes(r.c, 1, p2, 1)]
            v = SsLayerView()
            out.append(L.ss_acquire(r.c, 1, s1, C.byref(v)))
            out.append(L.ss_check_unit(r.c, 1, 2) if name == "ours" else OK)
            out += [L.ss_release(r.c, 1, s2), L.ss_release(r.c, 1, s1), L.ss_end(r.c), L.ss_begin(r.c, None, 0),
                    L.ss_layer_routes(r.c, 1, p3, 1), L.ss_acquire(r.c, 1, s2, C.byref(v)), int(L.ss_end(r.c) != OK)]
            s = ss.SsLayerStats()
            L.ss_stats_layer(r.c, 1, C.byref(s))
            seen[name] = (out, s.hits)
        finally:
            r.close()
    import tierstream_amd as tsa
    for x in (s1, s2):
        tsa.lib().tsa_stream_destroy(x)
    E = 1
    assert seen["ours"] == seen["reference"], seen
    assert seen["ours"] == ([E, E_HASH, OK, OK, OK, OK, E, OK, OK, OK, OK, E_HASH, 1], 1), seen


def test_seed_and_prefetch_between_forwards(tmp_path, gpu):
    """Reference tests/test_runtime.cpp:258-289: units seeded between forwards are hits (one group of two, both
    resident before the forward); an idle CERTAIN prefetch of the next forward's layer 2 lands before its routes."""
    m = fixtures.write_model(tmp_path, 3, 16, [4 * KiB, 4 * KiB], top_k=2, seed=37, tiers="pinned|disk")
    tiers = [2] * 48
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=0, ring_slots=4, dynamic_slots_per_layer=4)
    okw = dict(pin_planned=0, staging_bytes=64 * KiB)
    seen = {}
    for name, L, backend in _libs():
        _declare_more(L)
        r = _Run(L, backend, m.desc_json(), tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            seed, ps = _ids(5, 9, 9)
            nxt, pn = _ids(1, 6)
            r1, p1 = _ids(5, 9)
            out = [L.ss_seed(r.c, 1, ps, 3), L.ss_prefetch(r.c, 2, pn, 2, 0), L.ss_begin(r.c, None, 0),
                   L.ss_layer_routes(r.c, 1, p1, 2)]
            v = SsLayerView()
            out.append(L.ss_acquire(r.c, 1, None, C.byref(v)))
            out.append(v.groups[0].n_units)
            out += [L.ss_release(r.c, 1, None), L.ss_layer_routes(r.c, 2, pn, 2), L.ss_acquire(r.c, 2, None, C.byref(v))]
            if name == "ours":
                out += [L.ss_check_unit(r.c, 2, 1), L.ss_check_unit(r.c, 2, 6)]
            else:
                out += [OK, OK]
            out += [L.ss_release(r.c, 2, None), L.ss_end(r.c)]
            stats = []
            for layer in (1, 2):
                s = ss.SsLayerStats()
                L.ss_stats_layer(r.c, layer, C.byref(s))
                stats.append({k: x for k, x in s.as_dict().items() if k != "wait_ns"})
            seen[name] = (out, stats)
        finally:
            r.close()
    assert seen["ours"] == seen["reference"], seen
    assert seen["ours"][0] == [OK, OK, OK, OK, OK, 2, OK, OK, OK, OK, OK, OK, OK] and seen["ours"][1][0]["hits"] == 2


def test_exclusive_evicted_then_routed_same_forward(tmp_path, gpu):
    """Reference tests/test_exclusive.cpp:610-633: a CERTAIN prefetch of layer 1 evicts resident 0 (LRU, lowest id)
    into a free block; the layer's routes then route 0, which is read back from the block its write-back of this same
    forward targets - the copy must wait for that write-back (ss_check_unit: the device bytes equal the file's). Two
    write-backs, no file bytes. rereads counts the read-back on this discrete device; the reference's unified CPU
    backend never counts it."""
    m = fixtures.write_model(tmp_path, 3, 8, [4 * KiB, 4 * KiB], top_k=2, seed=41, tiers="pinned|disk")
    tiers = [1] * 8 + [0, 0, 0, 0, 1, 1, 1, 1] + [1] * 8
    bkw = dict(device_bytes=256 << 20, host_pinned_bytes=4 << 20, ring_slots=4, tier_mode=1, host_spare_units=2)
    okw = dict(verify_hash=1, pin_planned=0, staging_bytes=64 * KiB)
    seen = {}
    for name, L, backend in _libs():
        _declare_more(L)
        _declare_hooks(L)
        r = _Run(L, backend, m.desc_json(), tiers, bkw, okw)
        try:
            assert r.open_status == OK, (name, L.ss_last_error())
            pre, pp = _ids(5)
            ids, pi = _ids(0, 5)
            out = [L.ss_begin(r.c, None, 0), L.ss_prefetch(r.c, 1, pp, 1, 0), L.ss_layer_routes(r.c, 1, pi, 2)]
            v = SsLayerView()
            out.append(L.ss_acquire(r.c, 1, None, C.byref(v)))
            out += [L.ss_check_unit(r.c, 1, 0), L.ss_check_unit(r.c, 1, 5), L.ss_release(r.c, 1, None), L.ss_end(r.c)]
            x = ss.SsExclusiveStats()
            L.ss_stats_exclusive_sized(r.c, C.byref(x), C.sizeof(x))
            t = ss.SsLayerStats()
            L.ss_stats_total(r.c, C.byref(t))
            seen[name] = (out, x.writebacks, x.rereads, t.bytes_disk,
                          {k: v for k, v in t.as_dict().items() if k != "wait_ns"})
        finally:
            r.close()
    ours, theirs = seen["ours"], seen["reference"]
    assert ours[0] == theirs[0] == [OK] * 8, (ours, theirs)
    assert ours[1] == theirs[1] == 2 and ours[3] == theirs[3] == 0 and ours[4] == theirs[4], (ours, theirs)
    assert theirs[2] == 0 and ours[2] == 1, (ours, theirs)
