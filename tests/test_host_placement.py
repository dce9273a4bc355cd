"""The host contract's placement on the CPU (no GPU) against the reference CPU backend (oracle/_ref, compiled from its
sources): this library's HostPlacement alone (tsa_test_hostplace_run: the product's placement state machine with every
copy complete when issued) and the reference runtime on the same descriptor, budget, options and forward loop. Every
forward the address tables (pool slot or ring slot, as region + offset), the groups and the counters must be equal.

Configurations are drawn per seed: 2-6 layers of 3-16 units (MoE, sometimes a blob layer), unit sizes of one to three
parts, 1-4 routed ids per layer (sometimes a union of several tokens with repeats), budgets that leave a part of the
units resident, dynamic slots per layer, the ring size, pin_planned, LRU or SCORED (with its window), inclusive or
exclusive tiers (spare blocks, exclusive_discard), ss_layer_all or hits-first groups, and next-layer prefetch (CERTAIN
and SPECULATIVE, spec_persistent). The reference's own runtime tests check the same things (tests/test_runtime.cpp,
tests/test_exclusive.cpp)."""
import ctypes as C

import numpy as np
import pytest

from oracle import fixtures, ref
from tierstream_amd import ss

KiB = 1024
i32 = C.c_int32


def _lib():
    import tierstream_amd as tsa
    L = tsa.lib()
    L.tsa_test_hostplace_run.restype = C.c_int
    L.tsa_test_hostplace_run.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(ss.SsBudget), C.POINTER(ss.SsOptions),
                                         C.c_int, C.POINTER(i32), C.POINTER(i32), C.c_int, C.c_int, C.c_int,
                                         C.POINTER(i32), C.POINTER(i32), C.POINTER(i32),
                                         C.POINTER(ss.SsLayerStats)]
    L.tsa_test_hostplace_exclusive.restype = C.c_int
    L.tsa_test_hostplace_exclusive.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(ss.SsBudget),
                                               C.POINTER(ss.SsOptions), C.c_int, C.POINTER(i32), C.POINTER(i32),
                                               C.c_int, C.c_int, C.POINTER(ss.SsExclusiveStats)]
    return tsa, L


def _case(seed, tmp_path):
    rng = np.random.default_rng(seed)
    layers = int(rng.integers(2, 7))
    units = int(rng.integers(3, 17))
    parts = [int(rng.choice([4, 8, 12])) * KiB for _ in range(int(rng.integers(1, 4)))]
    mode = int(rng.choice([0, 0, 1, 2]))
    kind = "blob" if mode == 1 and rng.integers(0, 2) else "moe"
    if kind == "blob":
        units = 1
    top_k = int(rng.integers(1, min(4, units) + 1))
    tokens = int(rng.integers(1, 4)) if mode == 2 else 1
    m = fixtures.write_model(tmp_path, layers, units, parts, kind=kind, top_k=top_k,
                             order=str(rng.choice(["ranked", "prefix"])), seed=seed % 1000)
    st = (m.unit_bytes + 255) // 256 * 256
    hs = (m.unit_bytes + 4095) // 4096 * 4096
    total = layers * units
    n_res = int(rng.integers(0, total // 2 + 1))
    # mostly enough ring slots for a layer's transients plus the next layer's prefetches; now and then too few (the
    # acquire's SS_E_CAPACITY must then be the reference's too)
    ring = 2 * top_k * tokens + int(rng.integers(0, 3)) if kind == "moe" else int(rng.integers(1, 4))
    if rng.integers(0, 6) == 0:
        ring = max(1, ring // 3)
    dyn = int(rng.integers(0, 3))
    excl = bool(rng.integers(0, 3) == 0) and kind == "moe"
    bkw = dict(device_bytes=n_res * st + ring * st + dyn * layers * st + st // 2,
               host_pinned_bytes=total * hs + (64 << 20), dynamic_slots_per_layer=dyn, ring_slots=ring)
    if excl:
        bkw.update(tier_mode=1, host_spare_units=int(rng.integers(1, 8)))
    okw = dict(pin_planned=int(rng.integers(0, 2)), group_units=int(rng.integers(0, 3)))
    if rng.integers(0, 3) == 0:
        okw.update(policy=1, score_window=int(rng.integers(1, 20)))
    if excl and rng.integers(0, 3) == 0:
        okw.update(exclusive_discard=1)
        m.tiers = "pinned|disk"  # (a discarded victim is file-homed: the descriptor's tiers must allow it)
    if rng.integers(0, 3) == 0:
        okw.update(spec_persistent=0, lookahead_budget=int(rng.integers(1, 4)))
    steps = int(rng.integers(6, 16))
    routes = fixtures.uniform_routes(layers, units, top_k, steps, seed=seed + 3, tokens=tokens)
    if tokens > 1 and rng.integers(0, 2):  # repeats inside a union
        routes[:, :, -1] = routes[:, :, 0]
    prefetch = None
    if mode != 1 and rng.integers(0, 2):
        guess = fixtures.uniform_routes(layers, units, top_k, steps, seed=seed + 7, tokens=1)
        guess[:, :, 0] = np.where(rng.random((steps, layers)) < 0.6, routes[:, :, 0], guess[:, :, 0])
        prefetch = np.full_like(routes, -1)  # (rows as wide as the routes', -1 padded)
        prefetch[:, :, :guess.shape[2]] = guess
    return m, bkw, okw, routes, prefetch, mode


def _ours(m, bkw, okw, routes, prefetch, mode):
    tsa, L = _lib()
    steps, layers, max_ids = routes.shape
    mu = m.units
    kind = np.zeros((steps, layers, mu), np.int32)
    index = np.zeros_like(kind)
    group = np.zeros_like(kind)
    stats = (ss.SsLayerStats * steps)()
    r = np.ascontiguousarray(routes, dtype=np.int32)
    pf = np.ascontiguousarray(prefetch, dtype=np.int32) if prefetch is not None else None
    js = m.desc_json().encode()
    tsa.check(L.tsa_test_hostplace_run(js, len(js), C.byref(ss.budget(**bkw)), C.byref(ss.options(**okw)), steps,
                                       r.ctypes.data_as(C.POINTER(i32)),
                                       pf.ctypes.data_as(C.POINTER(i32)) if pf is not None else None, max_ids, mode,
                                       mu, kind.ctypes.data_as(C.POINTER(i32)), index.ctypes.data_as(C.POINTER(i32)),
                                       group.ctypes.data_as(C.POINTER(i32)), stats))
    return kind, index, group, [stats[s].as_dict() for s in range(steps)]


def _region(m, d, plan_json, kind, index, layer):
    """Our (kind, index) as the reference's (region kind, region index, offset)."""
    if kind == 0:
        return (0, -1, 0)
    st = (m.unit_bytes + 255) // 256 * 256  # (every layer of a fixture has the same unit bytes)
    if kind == 1:
        return (1, layer, index * st)
    first = 0
    for k, rc in enumerate(c for c in plan_json["rings"] if c["slots"]):
        if index < first + rc["slots"]:
            return (2, k, (index - first) * rc["slot_bytes"])
        first += rc["slots"]
    raise AssertionError("ring slot out of range")


def _compare(seed, tmp_path):
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    m, bkw, okw, routes, prefetch, mode = _case(seed, tmp_path)
    try:
        want = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(**okw), routes, mode, prefetch=prefetch,
                            checksums=False)
    except RuntimeError as e:  # a refusal (an open the reference refuses, a ring too small): ours refuses it too
        status = int(str(e).split("reference status ")[1].split(":")[0])
        with pytest.raises(ss.SsError) as ours:
            _ours(m, bkw, okw, routes, prefetch, mode)
        assert ours.value.status == status, (seed, str(e), str(ours.value))
        return []
    kind, index, group, stats = _ours(m, bkw, okw, routes, prefetch, mode)
    d = ss.Desc(m.desc_json())
    pj = ss.Plan(d, ss.budget(**bkw)).json()
    for s, w in enumerate(want):
        assert {k: v for k, v in stats[s].items() if k != "wait_ns"} == \
            {k: v for k, v in w["stats"].items() if k != "wait_ns"}, (seed, s, "stats")
        for l in range(m.layers):
            got = [_region(m, d, pj, int(kind[s, l, u]), int(index[s, l, u]), l) for u in range(m.units)]
            assert got == [tuple(t) for t in w["tables"][l]], (seed, s, l, "table")
            groups = [[] for _ in w["groups"][l]]
            for u in range(m.units):
                if group[s, l, u] >= 0:
                    assert group[s, l, u] < len(groups), (seed, s, l, u, "group")
                    groups[group[s, l, u]].append(u)
            assert groups == [sorted(g) for g in w["groups"][l]], (seed, s, l, "groups")
    d.close()
    return want


@pytest.mark.parametrize("seed", range(160))
def test_host_placement_matches_reference(seed, tmp_path):
    _compare(seed, tmp_path)


def test_cases_exercise_the_paths(tmp_path):
    """The random configurations together reach every decision the parity relies on: hits, admissions, evictions,
    ring transients, prefetches (certain and speculative, used and dropped), groups of several units."""
    tot = {}
    multi_group = 0
    for seed in range(60):
        d = tmp_path / str(seed)
        d.mkdir()
        for w in _compare(seed, d):
            for k, v in w["stats"].items():
                tot[k] = tot.get(k, 0) + v
            multi_group += sum(1 for g in w["groups"] if len(g) > 2)
    for k in ("hits", "admitted", "transient", "evicted", "prefetched", "spec_issued", "spec_used", "spec_dropped",
              "bytes_pinned"):
        assert tot[k] > 0, (k, tot)
    assert multi_group > 0


@pytest.mark.parametrize("seed", range(60))
def test_exclusive_counters_match_reference(seed, tmp_path):
    """Exclusive tier mode: write-backs, discards, deferrals, rereads, promotions and free blocks after the same
    forwards (the reference's ss_stats_exclusive); on every third seed with next-layer prefetch (certain and
    speculative) of guesses, and on every fourth with hits-first groups. rereads (a pinned read of a block whose
    write-back this forward issued) is a discrete device's count: the reference counts it only where a write-back
    leaves an event to wait for (src/stream_ctx.cpp:672-676, :1064-1100), never on its unified CPU backend. Only a
    prefetch makes one (a victim of the next layer's admission routed in the same forward), so without prefetch both
    are 0; with it, ours counts what the reference's discrete backend would."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference CPU backend) is not built")
    rng = np.random.default_rng(500 + seed)
    layers, units = int(rng.integers(2, 6)), int(rng.integers(4, 16))
    top_k = int(rng.integers(1, 4))
    m = fixtures.write_model(tmp_path, layers, units, [8 * KiB, 4 * KiB], top_k=top_k, seed=seed)
    st = (m.unit_bytes + 255) // 256 * 256
    hs = (m.unit_bytes + 4095) // 4096 * 4096
    n_res = int(rng.integers(1, layers * units // 2 + 1))
    ring = 2 * top_k + 1
    dyn = int(rng.integers(1, 3))
    bkw = dict(device_bytes=n_res * st + ring * st + dyn * layers * st + st // 2,
               host_pinned_bytes=layers * units * hs + (64 << 20), dynamic_slots_per_layer=dyn, ring_slots=ring,
               tier_mode=1, host_spare_units=int(rng.integers(1, 6)))
    okw = dict(pin_planned=0, exclusive_discard=int(rng.integers(0, 2)))
    if okw["exclusive_discard"]:
        m.tiers = "pinned|disk"
    routes = fixtures.uniform_routes(layers, units, top_k, 12, seed=seed + 1)
    prefetch = None
    if seed % 3 == 2:
        guess = fixtures.uniform_routes(layers, units, top_k, 12, seed=seed + 2)
        guess[:, :, 0] = np.where(rng.random((12, layers)) < 0.6, routes[:, :, 0], guess[:, :, 0])
        prefetch = guess
    mode = 2 if seed % 4 == 3 else 0
    if mode == 2:
        okw.update(group_units=2)
    want = ref.host_exclusive(m.desc_json(), ss.budget(**bkw), ss.options(**okw), routes, prefetch=prefetch,
                              mode=mode)
    tsa, L = _lib()
    x = ss.SsExclusiveStats()
    js = m.desc_json().encode()
    r = np.ascontiguousarray(routes, dtype=np.int32)
    pf = np.ascontiguousarray(prefetch, dtype=np.int32) if prefetch is not None else None
    tsa.check(L.tsa_test_hostplace_exclusive(js, len(js), C.byref(ss.budget(**bkw)), C.byref(ss.options(**okw)),
                                             routes.shape[0], r.ctypes.data_as(C.POINTER(i32)),
                                             pf.ctypes.data_as(C.POINTER(i32)) if pf is not None else None,
                                             routes.shape[2], mode, C.byref(x)))
    got = {k: getattr(x, k) for k, _ in ss.SsExclusiveStats._fields_ if k != "struct_size"}
    assert want["rereads"] == 0
    if prefetch is not None:
        want["rereads"] = got["rereads"]
    assert got == want, seed
