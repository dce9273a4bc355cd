"""Device-gated calls between tokens on the MI355X, against the reference DgCore making the same calls (oracle/_ref):

* ss_dg_residency, then a new context seeded with it (dg_seed, reference src/dg_ctx.cpp:1908-1926): the list is the
  reference core's recency order, the seeded open places units as the reference core does with the same seed, and
  the tokens that follow match it;
* ss_dg_set_budgets (the spare target and the prefetch budgets, reference src/dg_ctx.cpp:892-899) changed between
  tokens of a decode with predictions;
* ss_dg_set_clean_evict switched between tokens of a three-tier decode (reference src/dg_ctx.cpp:595-605);
* ss_dg_gated_index over a descriptor with a layer that has no units;
* the reference's test hooks ss_test_dg_check and ss_test_dg_stop_service (dg_test_hooks = 1);
* the file tier read with O_DIRECT (ss_source_direct = 1): direct reads bounced past pinned staging.
Every token the slot table and the counters must equal the reference core's, and every routed unit the engine read
through ss_dg_slot must checksum to its file bytes."""
import json
import os
import tempfile

import numpy as np
import pytest

import test_gpu_dg_parity as base
from oracle import fixtures, ref
from tierstream_amd import ss

pytestmark = pytest.mark.gpu

KiB = 1024
E_INVALID, E_BACKEND = 1, 5


def _need_ref():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")


class _Shape:
    """The mixtral-shape test case at test size: its model, plan and the reference core's geometry."""

    def __init__(self, tmp_path, layers=4, units=8, parts=(64 * KiB,) * 3, n_res=12, dyn=1, spares=6, n_ids=2, seed=21):
        self.layers, self.units, self.n_ids = layers, units, n_ids
        self.parts = list(parts)
        self.m, self.bkw, self.okw = base._setup(tmp_path, layers, units, self.parts, n_res, dyn, spares, n_ids,
                                                 seed=seed)
        self.d = ss.Desc(self.m.desc_json())
        self.plan = ss.Plan(self.d, ss.budget(**self.bkw))
        tiers = self.plan.tiers()
        self.residents = [L * units + u for L in range(layers) for u in range(units) if tiers[L][u] == 0]
        self.P = sum(1 for L in range(layers) for u in range(units) if tiers[L][u] == 1)
        self.Q = self.plan.json()["spare_blocks"][0]["blocks"]
        self.D = sum(min(dyn, sum(1 for u in range(units) if tiers[L][u] != 0)) for L in range(layers))
        self.keys = layers * units
        self.expect = {(L, u): self.m.checksum(L, u) for L in range(layers) for u in range(units)}

    def refdg(self, seed_keys=()):
        return ref.RefDg([self.units] * self.layers, len(self.residents) + self.D, self.n_ids, self.P + self.Q, self.D,
                         self.parts, list(seed_keys) + self.residents + list(range(self.keys)))

    def ctx(self, **extra):
        return ss.Ctx(self.d, ss.budget(**self.bkw), self.plan, ss.options(**dict(self.okw, **extra)))

    def check(self, ctx, refdg, eng, routes, preds=None, counters=base.COUNTERS, tag=""):
        cks, _ = eng.token(routes, preds=preds)
        want_table, want = refdg.token(routes.astype(np.uint32), pred=preds.astype(np.uint32) if preds is not None
                                       else None)
        got = ctx.dg_stats()
        assert np.array_equal(ctx.dg_table(), want_table), tag
        for k in counters:
            assert got[k] == want[k], (tag, k, got[k], want[k])
        for L in range(self.layers):
            for i, u in enumerate(routes[L]):
                assert int(cks[L, i]) == self.expect[(L, int(u))], (tag, L, i)
        return got


def test_residency_reseeds_a_new_context(tmp_path, gpu):
    _need_ref()
    s = _Shape(tmp_path)
    routes = base._routes(s.layers, s.units, s.n_ids, 24, seed=5, zipf=True)
    ctx, refdg = s.ctx(), s.refdg()
    eng = ss.DgEngine(ctx, s.n_ids)
    try:
        for t in range(12):
            s.check(ctx, refdg, eng, routes[t], tag=("first", t))
        res = ctx.dg_residency()
        keys = [g * s.units + u for g, u in res]
        assert keys == refdg.residency(), (keys, refdg.residency())
        assert len(keys) == len(set(keys)) == int(np.sum(ctx.dg_table() >= 0))
    finally:
        eng.close()
        ctx.close()
        refdg.close()
    # the seed is the last tokens' recency order, not the plan's residents: it places differently
    plain, seeded = s.refdg(), s.refdg(keys)
    assert not np.array_equal(plain.table(), seeded.table())
    plain.close()
    seeded.close()
    arr, n = ss.dg_seed(res)
    ctx = s.ctx(dg_seed=ss.C.cast(arr, ss.vp), dg_seed_n=n)
    refdg = s.refdg(keys)
    eng = ss.DgEngine(ctx, s.n_ids)
    try:
        assert np.array_equal(ctx.dg_table(), refdg.table()), "the seeded open's placement"
        for t in range(12, 24):
            got = s.check(ctx, refdg, eng, routes[t], tag=("seeded", t))
        assert got["tokens"] == 12 and ctx.verify_failures() == 0
    finally:
        eng.close()
        ctx.close()
        refdg.close()
    # a seed entry out of range refuses the open
    bad, nb = ss.dg_seed([(0, s.units)])
    with pytest.raises(ss.SsError):
        s.ctx(dg_seed=ss.C.cast(bad, ss.vp), dg_seed_n=nb)


def test_set_budgets_between_tokens(tmp_path, gpu):
    _need_ref()
    s = _Shape(tmp_path, layers=4, units=16, n_res=24, dyn=2, spares=12, n_ids=4)
    predict = 3
    routes = base._routes(s.layers, s.units, s.n_ids, 24, seed=5, zipf=True)
    preds = base._preds(routes, s.units, predict)
    ctx, refdg = s.ctx(), s.refdg()
    eng = ss.DgEngine(ctx, s.n_ids, n_pred=predict)
    changes = {4: (s.D - 1, 1, 3), 9: (0, 2, 5), 14: (s.D, 0, 0), 19: (2, 4, 48)}
    counters = base.COUNTERS + base.PRED_COUNTERS
    try:
        for t in range(routes.shape[0]):
            if t in changes:
                ctx.dg_set_budgets(*changes[t])
                refdg.set_budgets(*changes[t])
            got = s.check(ctx, refdg, eng, routes[t], preds=preds[t], counters=counters, tag=t)
        assert got["prefetched"] > 0 and got["evicted"] > 0, got
        with pytest.raises(ss.SsError):
            ctx.dg_set_budgets(s.D + 1, 4, 48)  # above the billed spares
    finally:
        eng.close()
        ctx.close()
        refdg.close()


def test_gated_index_skips_layers_without_units(tmp_path, gpu):
    s = _Shape(tmp_path)
    doc = json.loads(s.m.desc_json())
    moe = doc["layers"]
    layers = [moe[0], {"index": 1, "kind": "dense", "fixed_bytes": 4096}] + moe[1:]
    for i, l in enumerate(layers):
        l["index"] = i
    doc["layers"] = layers
    d = ss.Desc(json.dumps(doc))
    b = ss.budget(**dict(s.bkw, device_bytes=s.bkw["device_bytes"] + 4096))
    plan = ss.Plan(d, b)
    ctx = ss.Ctx(d, b, plan, ss.options(**s.okw))
    try:
        assert [ctx.dg_gated_index(L) for L in range(-1, len(layers) + 1)] == [-1, 0, -1, 1, 2, 3, -1]
        assert ctx.dg_view().n_gated == 4
        eng = ss.DgEngine(ctx, s.n_ids)
        try:
            routes = base._routes(s.layers, s.units, s.n_ids, 4, seed=7, zipf=True)
            for t in range(4):
                cks, _ = eng.token(routes[t])
                for g in range(s.layers):
                    for i, u in enumerate(routes[t, g]):
                        assert int(cks[g, i]) == s.expect[(g, int(u))]
        finally:
            eng.close()
    finally:
        ctx.close()


def test_clean_evict_switched_between_tokens(tmp_path, gpu):
    _need_ref()
    layers, units, n_ids, staging, dyn = 4, 8, 2, 4, 1
    m, tiers, bkw = base._three_tier(tmp_path, extra_blocks=staging)
    parts = [64 * KiB] * 3
    keys = layers * units
    d = ss.Desc(m.desc_json())
    plan = ss.Plan(d, ss.budget(**bkw), tiers=tiers)
    Q = plan.json()["spare_blocks"][0]["blocks"]
    D = sum(min(dyn, sum(1 for u in range(units) if tiers[L * units + u] != 0)) for L in range(layers))
    flags = [1 if t == 2 else 0 for t in tiers]
    refdg = ref.RefDg([units] * layers, 12 + D, n_ids, 10 + Q, D, parts, list(range(12)) + list(range(keys)),
                      disk=dict(flags=flags, home_blocks=10, disk_staging=staging, clean_evict=0))
    ctx = ss.Ctx(d, ss.budget(**bkw), plan, ss.options(forward_mode=1, dg_max_ids=n_ids, pin_planned=0, verify_hash=2,
                                                      dg_disk_tier=1, dg_disk_staging=staging, dg_disk_queue=4,
                                                      dg_wait_timeout_ms=5000))
    eng = ss.DgEngine(ctx, n_ids)
    routes = base._routes(layers, units, n_ids, 30, seed=9, zipf=True)
    expect = {(L, u): fixtures.engine_checksum(m.unit_data(L, u)) for L in range(layers) for u in range(units)}
    counters = base.COUNTERS + ["disk_reads", "disk_drops", "disk_discards", "clean_drops"]
    switch = {6: 1, 14: 0, 20: 1}
    try:
        for t in range(routes.shape[0]):
            if t in switch:
                ctx.dg_set_clean_evict(switch[t])
                refdg.set_clean_evict(switch[t])
                assert json.loads(ctx.stats_json())["device_gated"]["three_tier"]["clean_evict"] == switch[t]
            cks, _ = eng.token(routes[t])
            want_table, want = refdg.token(routes[t].astype(np.uint32))
            got = ctx.dg_stats()
            assert np.array_equal(ctx.dg_table(), want_table), t
            for k in counters:
                assert got[k] == want[k], (t, k, got[k], want[k])
            for g in range(layers):
                for i, u in enumerate(routes[t, g]):
                    assert int(cks[g, i]) == expect[(g, int(u))], (t, g, i)
        assert got["clean_drops"] > 0 and got["disk_reads"] > 0, got
        with pytest.raises(ss.SsError):
            ctx.dg_set_clean_evict(2)
    finally:
        eng.close()
        ctx.close()
        refdg.close()


def test_check_and_stop_service_hooks(tmp_path, gpu):
    """ss_test_dg_check: the core's ownership invariants hold between tokens; refused without dg_test_hooks.
    ss_test_dg_stop_service: the next token fails closed - every kernel of it ends on the host's abort word, ss_end
    reports SS_E_BACKEND and the context refuses further tokens - and the context closes."""
    s = _Shape(tmp_path)
    routes = base._routes(s.layers, s.units, s.n_ids, 6, seed=3, zipf=True)
    ctx = s.ctx()
    try:
        assert ctx.test_dg_check() == E_INVALID and ctx.test_dg_stop_service() == E_INVALID  # no dg_test_hooks
    finally:
        ctx.close()
    ctx = s.ctx(dg_test_hooks=1, dg_wait_timeout_ms=3000)
    eng = ss.DgEngine(ctx, s.n_ids)
    try:
        for t in range(4):
            eng.token(routes[t])
            assert ctx.test_dg_check() == 0, t
        assert ctx.test_dg_stop_service() == 0
        st, _, _ = eng.token_status(routes[4])
        assert st == E_BACKEND, st
        st, _, _ = eng.token_status(routes[5])
        assert st == E_BACKEND, st  # poisoned
    finally:
        eng.close()
        ctx.close()


def _direct_dir():
    """A directory whose file system takes O_DIRECT reads (the temp directory, then the working directory)."""
    for cand in (tempfile.gettempdir(), os.getcwd(), os.path.expanduser("~")):
        try:
            d = tempfile.mkdtemp(dir=cand)
        except OSError:
            continue
        p = os.path.join(d, "probe")
        with open(p, "wb") as f:
            f.write(b"\0" * 8192)
        try:
            fd = os.open(p, os.O_RDONLY | os.O_DIRECT)
            os.close(fd)
            os.remove(p)
            return d
        except OSError:
            os.remove(p)
            os.rmdir(d)
    return None


@pytest.mark.parametrize("queue", [0, 4])
def test_three_tier_direct_io(queue, gpu):
    """The file tier on a file system that takes O_DIRECT: ss_source_direct is 1 and every read is direct (into
    pinned staging, which the kernel cannot pin for the read: each piece bounces through the reader's pageable buffer);
    placement, counters and checksums equal the reference's."""
    _need_ref()
    d0 = _direct_dir()
    if d0 is None:
        pytest.skip("no writable file system here takes O_DIRECT")
    import pathlib
    import shutil
    try:
        layers, units, n_ids, staging, dyn = 4, 8, 2, 4, 1
        m, tiers, bkw = base._three_tier(pathlib.Path(d0), extra_blocks=staging)
        parts = [64 * KiB] * 3
        keys = layers * units
        d = ss.Desc(m.desc_json())
        plan = ss.Plan(d, ss.budget(**bkw), tiers=tiers)
        Q = plan.json()["spare_blocks"][0]["blocks"]
        D = sum(min(dyn, sum(1 for u in range(units) if tiers[L * units + u] != 0)) for L in range(layers))
        flags = [1 if t == 2 else 0 for t in tiers]
        refdg = ref.RefDg([units] * layers, 12 + D, n_ids, 10 + Q, D, parts, list(range(12)) + list(range(keys)),
                          disk=dict(flags=flags, home_blocks=10, disk_staging=staging))
        ctx = ss.Ctx(d, ss.budget(**bkw), plan, ss.options(forward_mode=1, dg_max_ids=n_ids, pin_planned=0,
                                                          verify_hash=2, dg_disk_tier=1, dg_disk_staging=staging,
                                                          dg_disk_queue=queue, direct_io=1, dg_wait_timeout_ms=5000))
        eng = ss.DgEngine(ctx, n_ids)
        try:
            assert ctx.source_direct(0) == 1
            routes = base._routes(layers, units, n_ids, 16, seed=9, zipf=True)
            for t in range(routes.shape[0]):
                cks, _ = eng.token(routes[t])
                want_table, want = refdg.token(routes[t].astype(np.uint32))
                got = ctx.dg_stats()
                assert np.array_equal(ctx.dg_table(), want_table), t
                for k in base.COUNTERS + ["disk_reads", "disk_drops", "disk_discards"]:
                    assert got[k] == want[k], (t, k, got[k], want[k])
                for g in range(layers):
                    for i, u in enumerate(routes[t, g]):
                        assert int(cks[g, i]) == fixtures.engine_checksum(m.unit_data(g, int(u))), (t, g, i)
            assert got["disk_reads"] > 0 and ctx.verify_failures() == 0, got
        finally:
            eng.close()
            ctx.close()
            refdg.close()
    finally:
        shutil.rmtree(d0, ignore_errors=True)


def test_legacy_null_stream_is_refused(tmp_path, gpu):
    """The library's streams are CU-masked (a hardware queue each), which the HIP runtime creates as blocking
    streams: work on the legacy null stream and theirs wait for each other, so a layer's wait kernel there would hold
    the checks and ready words it waits for until dg_wait_timeout_ms. Every ss_dg_enqueue_* call refuses that stream
    (nullptr and hipStreamLegacy) with SS_E_INVALID, launches nothing and leaves the context usable: the tokens that
    follow on the engine's own stream match the reference core. (The reference's streams are non-blocking and take
    the null stream, src/dg_ctx.cpp:71-73.)"""
    import ctypes as C
    import tierstream_amd as tsa
    _need_ref()
    s = _Shape(tmp_path)
    routes = base._routes(s.layers, s.units, s.n_ids, 6, seed=9, zipf=True)
    ctx, refdg = s.ctx(), s.refdg()
    L = tsa.lib()
    vp, i32 = C.c_void_p, C.c_int
    for name, types in [("ss_dg_enqueue_begin", [vp, vp]), ("ss_dg_enqueue_end", [vp, vp]),
                        ("ss_dg_enqueue_wait", [vp, i32, vp]), ("ss_dg_enqueue_predict", [vp, i32, vp, i32, vp]),
                        ("ss_dg_enqueue_export", [vp, i32, vp, i32, i32, vp])]:
        getattr(L, name).argtypes = types
        getattr(L, name).restype = i32
    ids = tsa.DeviceBuffer(4 * 64)
    ids.upload(np.zeros(64, dtype=np.int32))
    calls = {
        "ss_dg_enqueue_begin": lambda st: L.ss_dg_enqueue_begin(ctx.h, st),
        "ss_dg_enqueue_export": lambda st: L.ss_dg_enqueue_export(ctx.h, 0, ids.ptr, 1, 0, st),
        "ss_dg_enqueue_predict": lambda st: L.ss_dg_enqueue_predict(ctx.h, 0, ids.ptr, 1, st),
        "ss_dg_enqueue_wait": lambda st: L.ss_dg_enqueue_wait(ctx.h, 0, st),
        "ss_dg_enqueue_end": lambda st: L.ss_dg_enqueue_end(ctx.h, st),
    }
    try:
        for name, call in calls.items():
            for st in (None, 1):  # nullptr, hipStreamLegacy
                assert call(st) == E_INVALID, (name, st)
                msg = L.ss_last_error().decode()
                assert name in msg and "legacy null stream" in msg, msg
        eng = ss.DgEngine(ctx, s.n_ids)
        try:
            for t in range(6):
                s.check(ctx, refdg, eng, routes[t], tag=("after refusals", t))
        finally:
            eng.close()
    finally:
        ids.close()
        ctx.close()
        refdg.close()
