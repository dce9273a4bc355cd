"""Host contract on the MI355X against the reference CPU backend (bit-exact): the same descriptor, budget, options and
route stream through both; per step the stats, every layer's table (region + offset: identical up to base), and the
checksum of every routed unit's bytes as the engine reads them through table_dev on the device. The reference's
checksums are of the bytes its own table entries point at, and both must equal the oracle's checksum of the file.
Shapes follow the benchmark workloads at test size (reference tests/test_runtime.cpp:58-83 check the same things:
table bytes == file bytes, stats balance)."""
import json

import numpy as np
import pytest

from oracle import fixtures, ref
from tierstream_amd import ss

pytestmark = pytest.mark.gpu

KiB = 1024
MiB = 1024 * KiB


def _budget(m, n_res, ring_slots, dyn=0, **kw):
    st = (m.unit_bytes + 255) // 256 * 256
    ring = ring_slots * st
    dev = n_res * st + ring + dyn * m.layers * st + st // 2
    host = (m.layers * m.units) * ((m.unit_bytes + 4095) // 4096 * 4096) + (64 << 20)
    return dict(device_bytes=dev, host_pinned_bytes=host, dynamic_slots_per_layer=dyn, ring_slots=ring_slots, **kw)


CASES = {
    # moe-small shape: ranked, half resident, inclusive, planned residents pinned (no eviction)
    "moe-small": dict(layers=4, units=8, parts=[64 * KiB] * 3, n_res=16, ring=8, steps=16, top_k=2, mode=0,
                      opts={}),
    # decode with a dynamic LRU set: residents are a warm start, 2 spare slots per layer, evictions every step
    "decode-lru": dict(layers=4, units=8, parts=[32 * KiB, 32 * KiB, 16 * KiB], n_res=8, ring=16, dyn=2, steps=24,
                       top_k=2, mode=0, opts=dict(pin_planned=0)),
    # dense-prefix shape: blob layers, prefix order, a 2-slot blob ring, ss_layer_all on every layer
    "dense-prefix": dict(layers=8, units=1, parts=[256 * KiB], kind="blob", order="prefix", n_res=3, ring=2, steps=4,
                         top_k=1, mode=1, opts={}),
    # qwen3-moe shape: a union of 4 tokens x top-4, exclusive with write-backs, hits-first groups
    "qwen-exclusive": dict(layers=6, units=16, parts=[32 * KiB] * 3, n_res=24, ring=32, dyn=2, steps=20, top_k=4,
                           tokens=4, mode=2, opts=dict(pin_planned=0, group_units=2),
                           budget=dict(tier_mode=1, host_spare_units=6)),
    # the SCORED policy (reference src/resident_set.cpp:52-68: 0.7 transition + 0.2 window frequency + 0.1 recency)
    "decode-scored": dict(layers=4, units=8, parts=[32 * KiB, 32 * KiB, 16 * KiB], n_res=8, ring=16, dyn=2, steps=24,
                          top_k=2, mode=0, opts=dict(pin_planned=0, policy=1, score_window=6)),
    # the reference's CPU-runnable config at full size: 4 x 8 experts of 3 x 1 MiB, top-2 uniform, half resident
    # (layers 0-1), the other half served from the pinned tier through an 8-slot ring, 64 steps
    "c1-full": dict(layers=4, units=8, parts=[1 * MiB] * 3, n_res=16, ring=8, steps=64, top_k=2, mode=0, opts={}),
    # pinned copies in several pieces (copy_piece_bytes below the unit): 256 KiB units in 64 KiB pieces, and the
    # exclusive shape's 96 KiB units in 40 KiB pieces (a short last piece)
    "multi-piece": dict(layers=4, units=8, parts=[96 * KiB, 96 * KiB, 64 * KiB], n_res=8, ring=16, dyn=2, steps=24,
                        top_k=2, mode=0, opts=dict(pin_planned=0, copy_piece_bytes=64 * KiB)),
    "multi-piece-exclusive": dict(layers=6, units=16, parts=[32 * KiB] * 3, n_res=24, ring=32, dyn=2, steps=20,
                                  top_k=4, tokens=4, mode=2,
                                  opts=dict(pin_planned=0, group_units=2, copy_piece_bytes=40 * KiB),
                                  budget=dict(tier_mode=1, host_spare_units=6)),
    "qwen-exclusive-scored": dict(layers=6, units=16, parts=[32 * KiB] * 3, n_res=24, ring=32, dyn=2, steps=20,
                                  top_k=4, tokens=4, mode=2, opts=dict(pin_planned=0, group_units=2, policy=1),
                                  budget=dict(tier_mode=1, host_spare_units=6)),
}


def _run_case(name, tmp_path, gpu):
    c = CASES[name]
    m = fixtures.write_model(tmp_path, c["layers"], c["units"], c["parts"], kind=c.get("kind", "moe"),
                             top_k=c["top_k"], order=c.get("order", "ranked"), seed=7)
    routes = fixtures.uniform_routes(c["layers"], c["units"], c["top_k"], c["steps"], seed=11,
                                     tokens=c.get("tokens", 1))
    bkw = _budget(m, c["n_res"], c["ring"], c.get("dyn", 0), **c.get("budget", {}))
    desc_json = m.desc_json()
    # the reference (CPU backend)
    want = ref.host_run(desc_json, ss.budget(**bkw), ss.options(**c["opts"]), routes, c["mode"])
    # the product (MI355X)
    d = ss.Desc(desc_json)
    ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options(**c["opts"]))
    try:
        cks, tabs, stats, _ = ctx.host_run(routes, c["mode"])
        for s in range(c["steps"]):
            w = want[s]
            got_stats = {k: v for k, v in stats[s].items() if k != "wait_ns"}
            want_stats = {k: v for k, v in w["stats"].items() if k != "wait_ns"}
            assert got_stats == want_stats, (name, s)
            for l in range(c["layers"]):
                got_tab = [ctx.region_of(int(a)) if a else (0, -1, 0) for a in tabs[s, l, :c["units"]]]
                assert got_tab == w["tables"][l], (name, s, l)
                ids = list(range(c["units"])) if c["mode"] == 1 else [int(x) for x in routes[s, l] if x >= 0]
                exp = [m.checksum(l, u) for u in ids]
                assert [int(x) for x in cks[s, l, :len(ids)]] == exp == w["checksums"][l], (name, s, l)
        return ctx, want
    except Exception:
        ctx.close()
        raise


def _stats_doc(text):
    """A stats-v1 document with what legitimately differs between the two backends taken out: the backend name and
    the host wait times. The text itself must be canonical (sorted keys, no whitespace), as the reference writes it."""
    doc = json.loads(text)
    assert text == json.dumps(doc, sort_keys=True, separators=(",", ":"))
    doc["backend"] = None
    for st in [doc["total"]] + doc["layers"]:
        st["wait_ns"] = 0
    return doc


@pytest.mark.parametrize("name", list(CASES))
def test_host_contract_matches_reference(name, tmp_path, gpu):
    ctx, want = _run_case(name, tmp_path, gpu)
    # the stats-v1 document (reference src/stream_ctx.cpp:1827-1885) after the same forwards
    assert _stats_doc(ctx.stats_json()) == _stats_doc(want[-1]["stats_json"]), name
    assert json.loads(ctx.stats_json())["backend"] == "hip"
    tot = ctx.stats_total()
    # the stats balance of reference tests/test_runtime.cpp:78-83
    assert tot["hits"] + tot["admitted"] + tot["transient"] + tot["prefetched"] + tot["spec_used"] == tot["routed"]
    if name == "qwen-exclusive":
        x = ctx.exclusive_stats()
        assert x["writebacks"] > 0  # the shape exercises write-backs
    ctx.close()


@pytest.mark.parametrize("name", ["decode-lru", "dense-prefix", "qwen-exclusive", "c1-full", "multi-piece"])
def test_device_verify_of_landed_units(name, tmp_path, gpu):
    """verify_hash = 2: every landed unit re-hashed in HBM (checkpoint-parallel) against the descriptor; none fails.
    The checks run in batches on their own stream, so a slot reused inside a forward (dense-prefix: 5 layers through a
    2-slot ring per forward) must not take its next unit before its previous one was checked."""
    c = CASES[name]
    m = fixtures.write_model(tmp_path, c["layers"], c["units"], c["parts"], kind=c.get("kind", "moe"),
                             top_k=c["top_k"], order=c.get("order", "ranked"), seed=3)
    routes = fixtures.uniform_routes(c["layers"], c["units"], c["top_k"], 12, seed=5, tokens=c.get("tokens", 1))
    bkw = _budget(m, c["n_res"], c["ring"], c.get("dyn", 0), **c.get("budget", {}))
    d = ss.Desc(m.desc_json())
    ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options(**c["opts"], verify_hash=2))
    try:
        cks, _, stats, _ = ctx.host_run(routes, c["mode"])
        import tierstream_amd as tsa
        assert tsa.ss._declare().tsa_test_verify_failures(ctx.h) == 0
        assert sum(s["admitted"] + s["transient"] for s in stats) > 0
    finally:
        ctx.close()


@pytest.mark.parametrize("name", ["moe-small", "qwen-exclusive"])
def test_stats_snapshot(name, tmp_path, gpu):
    """ss_stats_snapshot (reference include/strix_stream/ss.h:573-615): the first call arms and fails; each ss_end
    then publishes the counters as ss_stats_total / ss_stats_exclusive / ss_stats_to_json gave them, and so does a
    reset between forwards."""
    c = CASES[name]
    m = fixtures.write_model(tmp_path, c["layers"], c["units"], c["parts"], top_k=c["top_k"], seed=7)
    routes = fixtures.uniform_routes(c["layers"], c["units"], c["top_k"], 3, seed=11, tokens=c.get("tokens", 1))
    bkw = _budget(m, c["n_res"], c["ring"], c.get("dyn", 0), **c.get("budget", {}))
    d = ss.Desc(m.desc_json())
    ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options(**c["opts"]))
    try:
        with pytest.raises(ss.SsError):
            ctx.snapshot()
        with pytest.raises(ss.SsError):
            ctx.snapshot_json()
        ctx.host_run(routes[:2], c["mode"])
        tot, info = ctx.snapshot()
        assert tot == ctx.stats_total() and info["sequence"] == 2 and info["forwards"] == 2
        assert ctx.snapshot_json() == ctx.stats_json()
        excl = bkw.get("tier_mode", 0) == 1
        assert info["flags"] == (2 if excl else 0)
        if excl:
            x = ctx.exclusive_stats()
            for k in ("writebacks", "writeback_bytes", "deferred", "promoted", "free_blocks", "min_free_blocks",
                      "rereads", "discards"):
                assert info["exclusive_" + k] == x[k], k
            assert info["exclusive_blocks"] == json.loads(ctx.stats_json())["exclusive"]["blocks"] > 0
        ctx.stats_reset()
        tot, info = ctx.snapshot()
        assert info["sequence"] == 3 and tot["routed"] == 0 and ctx.snapshot_json() == ctx.stats_json()
    finally:
        ctx.close()


def test_host_prefetch_is_a_checked_no_op_without_read_ahead(tmp_path, gpu):
    """ss_host_prefetch / ss_host_prefetch_layer with readahead_units 0 (reference src/stream_ctx.cpp:1441-1449,
    src/capi.cpp:698-710): a no-op that still refuses a layer out of range and a negative count; the forwards after it
    match the reference."""
    import tierstream_amd as tsa
    c = CASES["decode-lru"]
    m = fixtures.write_model(tmp_path, c["layers"], c["units"], c["parts"], top_k=c["top_k"], seed=7)
    routes = fixtures.uniform_routes(c["layers"], c["units"], c["top_k"], 4, seed=11)
    bkw = _budget(m, c["n_res"], c["ring"], c.get("dyn", 0))
    want = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(**c["opts"]), routes, c["mode"])
    d = ss.Desc(m.desc_json())
    ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options(**c["opts"]))
    L = ss._declare()
    try:
        assert ctx.host_prefetch(0, [1, 2]) == tsa.SS_OK
        assert ctx.host_prefetch(c["layers"], [1]) == tsa.SS_E_INVALID
        assert L.ss_host_prefetch(ctx.h, 0, None, -1) == tsa.SS_E_INVALID
        assert L.ss_host_prefetch_layer(ctx.h, 1) == tsa.SS_OK
        assert L.ss_host_prefetch_layer(ctx.h, -1) == tsa.SS_E_INVALID
        _, _, stats, _ = ctx.host_run(routes, c["mode"])
        for s in range(4):
            assert {k: v for k, v in stats[s].items() if k != "wait_ns"} == \
                {k: v for k, v in want[s]["stats"].items() if k != "wait_ns"}, s
    finally:
        ctx.close()
