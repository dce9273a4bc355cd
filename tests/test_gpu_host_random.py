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
