"""The host contract's MI355X executor on random configurations, against the reference CPU backend: the shapes of the
CPU placement parity (tests/test_host_placement.py: pools, rings, exclusive write-backs and discards, LRU and scored
eviction, ss_layer_all and hits-first groups, next-layer prefetch) run through the real executor - deferred and merged
pinned copies, file reads through staging, the device check of every landed unit (verify_hash = 2). Per step the
stats and every layer's table equal the reference's, and every routed unit's checksum, read on the device through the
table, equals the file's; a refusal (a ring too small) is the reference's status."""
import numpy as np
import pytest

from oracle import fixtures, ref
from tierstream_amd import ss

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(120))
def test_random_host_configuration_matches_reference(seed, tmp_path, gpu):
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    from test_host_placement import _case
    m, bkw, okw, routes, prefetch, mode = _case(seed, tmp_path)
    okw = dict(okw, verify_hash=2)
    try:
        want = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(**okw), routes, mode, prefetch=prefetch)
        want_status = 0
    except RuntimeError as e:
        want, want_status = None, int(str(e).split("reference status ")[1].split(":")[0])
    d = ss.Desc(m.desc_json())
    try:
        ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options(**okw))
    except ss.SsError as e:
        assert want_status == e.status, (seed, want_status, str(e))
        return
    try:
        if want is None:
            with pytest.raises(ss.SsError) as err:
                ctx.host_run(routes, mode, prefetch=prefetch)
            assert err.value.status == want_status, (seed, str(err.value))
            return
        cks, tabs, stats, _ = ctx.host_run(routes, mode, prefetch=prefetch)
        units = m.units
        for s in range(routes.shape[0]):
            assert {k: v for k, v in stats[s].items() if k != "wait_ns"} == \
                {k: v for k, v in want[s]["stats"].items() if k != "wait_ns"}, (seed, s)
            for l in range(m.layers):
                got = [ctx.region_of(int(a)) if a else (0, -1, 0) for a in tabs[s, l, :units]]
                assert got == want[s]["tables"][l], (seed, s, l)
                # (ss_layer_all: the engine reads the first route-width units of the layer, the reference all of them)
                ids = list(range(min(units, routes.shape[2]))) if mode == 1 else \
                    [int(x) for x in routes[s, l] if x >= 0]
                exp = [m.checksum(l, u) for u in ids]
                assert [int(x) for x in cks[s, l, :len(ids)]] == exp == want[s]["checksums"][l][:len(ids)], (seed, s, l)
        assert ctx.verify_failures() == 0
        n_units, n_copies = ctx.host_copies()
        assert n_copies <= n_units
    finally:
        ctx.close()


def _ra_case(seed, tmp_path):
    """A host configuration with file-backed units and read-ahead: random tiers per unit (resident, pinned, file),
    dynamic slots, ring, exclusive mode now and then, readahead_units 1-4, ss_host_prefetch_layer of the next 0-2
    layers after each layer's routes, next-layer ss_prefetch now and then."""
    rng = np.random.default_rng(7000 + seed)
    layers, units = int(rng.integers(2, 6)), int(rng.integers(4, 13))
    parts = [int(rng.choice([4, 8, 16])) * 1024 for _ in range(int(rng.integers(1, 4)))]
    top_k = int(rng.integers(1, min(3, units) + 1))
    m = fixtures.write_model(tmp_path, layers, units, parts, top_k=top_k, seed=seed % 1000, tiers="pinned|disk")
    tiers = [int(rng.choice([0, 1, 2, 2])) for _ in range(layers * units)]
    st = (m.unit_bytes + 255) // 256 * 256
    hs = (m.unit_bytes + 4095) // 4096 * 4096
    n_res = sum(1 for t in tiers if t == 0)
    ring = 2 * top_k + int(rng.integers(1, 3))
    dyn = int(rng.integers(0, 3))
    ra = int(rng.integers(1, 5))
    excl = bool(rng.integers(0, 3) == 0)
    bkw = dict(device_bytes=n_res * st + ring * st + dyn * layers * st + st // 2,
               host_pinned_bytes=(layers * units + ra + 8) * hs + (64 << 20), dynamic_slots_per_layer=dyn,
               ring_slots=ring)
    if excl:
        bkw.update(tier_mode=1, host_spare_units=int(rng.integers(1, 6)))
    okw = dict(readahead_units=ra, pin_planned=int(rng.integers(0, 2)), verify_hash=int(rng.choice([1, 2])),
               staging_bytes=64 * 1024)
    routes = fixtures.uniform_routes(layers, units, top_k, int(rng.integers(6, 14)), seed=seed + 3)
    prefetch = None
    if rng.integers(0, 3) == 0:
        prefetch = fixtures.uniform_routes(layers, units, top_k, routes.shape[0], seed=seed + 5)
    return m, tiers, bkw, okw, routes, prefetch, int(rng.integers(0, 3))


@pytest.mark.parametrize("seed", range(40))
def test_random_read_ahead_configuration_matches_reference(seed, tmp_path, gpu):
    """Host read-ahead on random configurations: tables, per-step stats but bytes_disk and checksums equal the
    reference's; the read-ahead requests equal its, reads = landed + unused on both sides, and without next-layer
    prefetch the file fetches ((file bytes - read-ahead bytes) / unit bytes + landed) are the same. (With a prefetch, a
    CERTAIN prefetch of a unit the next routes leave out releases its ring slot, and its landing from a read-ahead
    buffer runs or is cancelled depending on when the read ends: in either library, so the fetch count follows
    timing.)"""
    import json
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    m, tiers, bkw, okw, routes, prefetch, lookahead = _ra_case(seed, tmp_path)
    try:
        want = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(**okw), routes, 0, prefetch=prefetch,
                            host_lookahead=lookahead, tiers=tiers)
        want_status = 0
    except RuntimeError as e:
        want, want_status = None, int(str(e).split("reference status ")[1].split(":")[0])
    d = ss.Desc(m.desc_json())
    plan = ss.Plan(d, ss.budget(**bkw), tiers=tiers)
    try:
        ctx = ss.Ctx(d, ss.budget(**bkw), plan, ss.options(**okw))
    except ss.SsError as e:
        plan.close()
        assert want_status == e.status, (seed, want_status, str(e))
        return
    try:
        if want is None:
            with pytest.raises(ss.SsError) as err:
                ctx.host_run(routes, 0, host_lookahead=lookahead, prefetch=prefetch)
            assert err.value.status == want_status, (seed, str(err.value))
            return
        cks, tabs, stats, _ = ctx.host_run(routes, 0, host_lookahead=lookahead, prefetch=prefetch)
        drop = ("wait_ns", "bytes_disk")
        for s in range(routes.shape[0]):
            assert {k: v for k, v in stats[s].items() if k not in drop} == \
                {k: v for k, v in want[s]["stats"].items() if k not in drop}, (seed, s)
            for l in range(m.layers):
                got = [ctx.region_of(int(a)) if a else (0, -1, 0) for a in tabs[s, l, :m.units]]
                assert got == want[s]["tables"][l], (seed, s, l)
                ids = [int(x) for x in routes[s, l] if x >= 0]
                exp = [m.checksum(l, u) for u in ids]
                assert [int(x) for x in cks[s, l, :len(ids)]] == exp == want[s]["checksums"][l], (seed, s, l)
        ours, theirs = json.loads(ctx.stats_json()), json.loads(want[-1]["stats_json"])
        if "readahead" in theirs:
            ra, ra_ref = ours["readahead"], theirs["readahead"]
            assert ra["requested"] == ra_ref["requested"], (seed, ra, ra_ref)
            for r in (ra, ra_ref):
                assert r["read"] == r["landed"] + r["unused"] and r["failed"] == 0, (seed, r)
            fetches = [(doc["total"]["bytes_disk"] - r["bytes"]) // m.unit_bytes + r["landed"]
                       for doc, r in ((ours, ra), (theirs, ra_ref))]
            assert prefetch is not None or fetches[0] == fetches[1], (seed, fetches)
        else:
            assert "readahead" not in ours
        assert ctx.verify_failures() == 0
    finally:
        ctx.close()
        plan.close()
