"""Host contract error paths on the MI355X, against the reference CPU backend driven by the same calls (reference
tests/test_runtime.cpp:216-256): a unit whose file bytes differ from the descriptor hash fails the acquire that needs it
with SS_E_HASH (verify_hash = 1), the forward's end reports it again, and the next forward serves the healthy units; a
stream ring too small for a layer's transient units is SS_E_CAPACITY naming the ring, not a hang, and the forward still
ends cleanly. Both libraries see the same descriptor, plan tiers, budget and options; every status must be the
reference's."""
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
