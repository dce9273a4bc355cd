"""The device-gated cache state machine against the reference's own, on the CPU (no GPU): this library's DgCore
(tsa_test_dgcore_*: the product's core on an eager transport) and the reference DgCore compiled from its sources
(oracle/_ref, refdg_*), on the same configuration, open-time priority and token route stream. After every token the
slot table, the counters and (three-tier) the pinned homes' recency order must be identical.

Configurations are drawn at random per seed: 2-6 gated layers of 4-16 units, 1-4 ids per layer (sometimes repeated,
the batch-union case), residents, spare slots and spare blocks, clean copies (dg_inclusive_blocks), deferred or
boundary write-backs; three-tier adds a file tier (a random share of the non-resident units), clean_evict and
disk prefetch off. Scored eviction (SCORED / SCORED_AUTO, weights, verify rows, starting counts), policy switches and
tokens that export only some layers are drawn the same way. Routes are skewed (Zipf-like over a per-layer permutation) so that hits, misses, bank serves,
resurrections and write-backs all occur. The reference's own CPU tests drive its core the same way
(tests/test_dg.cpp:201)."""
import ctypes as C

import numpy as np
import pytest

from oracle import ref

u32, u64 = C.c_uint32, C.c_uint64


class DgCoreConfig(C.Structure):
    _fields_ = [("n_units", C.POINTER(u32)), ("n_gated", u32), ("persistent_slots", u32), ("bank_slots", u32),
                ("blocks", u32), ("spare_target", u32), ("prefetch_reserve", u32), ("prefetch_per_layer", u32),
                ("prefetch_per_token", u32), ("wb_defer", u32), ("wb_on_d2h", u32), ("inclusive", u32),
                ("part_bytes", C.POINTER(u64)), ("n_parts", u32), ("disk_tier", u32), ("home_blocks", u32),
                ("disk_staging", u32), ("clean_evict", u32), ("disk_prefetch", u32),
                ("disk", C.POINTER(C.c_uint8)), ("policy", u32), ("w_trans", u32), ("w_freq", u32), ("w_rec", u32),
                ("rows", u32), ("score_cells", C.POINTER(u32)), ("bank_keep", u32), ("landing_blocks", u32),
                ("landing_ttl", u32)]


def _lib():
    import tierstream_amd as tsa
    L = tsa.lib()
    L.tsa_test_dgcore_open.argtypes = [C.POINTER(DgCoreConfig), C.POINTER(u32), u32, C.POINTER(C.c_void_p)]
    L.tsa_test_dgcore_open.restype = C.c_int
    L.tsa_test_dgcore_token.argtypes = [C.c_void_p, C.POINTER(u32), u32, C.POINTER(C.c_int32), C.POINTER(u64), u32]
    L.tsa_test_dgcore_token.restype = C.c_int
    L.tsa_test_dgcore_counter_names.restype = C.c_char_p
    L.tsa_test_dgcore_host_order.argtypes = [C.c_void_p, C.POINTER(u32), u32]
    L.tsa_test_dgcore_host_order.restype = u32
    L.tsa_test_dgcore_land_owner.argtypes = [C.c_void_p, C.POINTER(u32), u32]
    L.tsa_test_dgcore_land_owner.restype = u32
    L.tsa_test_dgcore_close.argtypes = [C.c_void_p]
    L.tsa_test_dgcore_close.restype = None
    L.tsa_test_dgcore_token_run.argtypes = [C.c_void_p, C.POINTER(u32), u32, C.POINTER(C.c_uint8),
                                            C.POINTER(C.c_int32), C.POINTER(u64), u32]
    L.tsa_test_dgcore_token_run.restype = C.c_int
    L.tsa_test_dgcore_token_pred.argtypes = [C.c_void_p, C.POINTER(u32), u32, C.POINTER(u32), u32,
                                             C.POINTER(C.c_uint8), C.POINTER(C.c_int32), C.POINTER(u64), u32]
    L.tsa_test_dgcore_token_pred.restype = C.c_int
    L.tsa_test_dgcore_set_policy.argtypes = [C.c_void_p, u32]
    L.tsa_test_dgcore_set_policy.restype = C.c_int
    L.tsa_test_dgcore_set_keep.argtypes = [C.c_void_p, C.POINTER(u32), u32]
    L.tsa_test_dgcore_set_keep.restype = C.c_int
    L.tsa_test_dgcore_set_wb_defer.argtypes = [C.c_void_p, u32]
    L.tsa_test_dgcore_set_wb_defer.restype = C.c_int
    L.tsa_test_dgcore_check_order.argtypes = [C.c_void_p, C.c_int]
    L.tsa_test_dgcore_check_order.restype = C.c_int
    return tsa, L


class OurCore:
    def __init__(self, n_units, persistent, bank, blocks, spare_target, part_bytes, order, wb_defer, inclusive,
                 disk=None, score=None):
        self.tsa, self.L = _lib()
        self._keep = []
        nu = (u32 * len(n_units))(*n_units)
        pb = (u64 * len(part_bytes))(*part_bytes)
        od = (u32 * len(order))(*order)
        c = DgCoreConfig()
        c.n_units, c.n_gated = nu, len(n_units)
        c.persistent_slots, c.bank_slots, c.blocks, c.spare_target = persistent, bank, blocks, spare_target
        c.prefetch_reserve, c.prefetch_per_layer, c.prefetch_per_token = 0xFFFFFFFF, 4, 48
        c.wb_defer, c.wb_on_d2h, c.inclusive = wb_defer, 1, inclusive
        c.part_bytes, c.n_parts = pb, len(part_bytes)
        if disk:
            fl = (C.c_uint8 * sum(n_units))(*disk["flags"])
            c.disk_tier, c.home_blocks, c.disk_staging = 1, disk["home_blocks"], disk["disk_staging"]
            c.clean_evict, c.disk_prefetch, c.disk = disk.get("clean_evict", 0), disk.get("disk_prefetch", 0), fl
            c.bank_keep = disk.get("bank_keep", 0)
            c.landing_blocks, c.landing_ttl = disk.get("landing_blocks", 0), disk.get("landing_ttl", 0)
            self._keep.append(fl)
        c.w_trans, c.w_freq, c.w_rec, c.rows = 700, 200, 100, 1
        if score:
            c.policy, c.rows = score["policy"], score.get("rows", 1)
            c.w_trans, c.w_freq, c.w_rec = score.get("w", (700, 200, 100))
            if score.get("cells") is not None:
                cp = (u32 * len(score["cells"]))(*score["cells"])
                c.score_cells = cp
                self._keep.append(cp)
        self._keep += [nu, pb, od, c]
        self.h = C.c_void_p()
        self.tsa.check(self.L.tsa_test_dgcore_open(C.byref(c), od, len(order), C.byref(self.h)))
        # every token also checks the copies' order (tsa_test_dgcore_check_order, tests/test_dgcore_order.py)
        self.tsa.check(self.L.tsa_test_dgcore_check_order(self.h, 1))
        self.keys = sum(n_units)
        self.names = self.L.tsa_test_dgcore_counter_names().decode().split()

    def token(self, ids, run=None, pred=None):
        x = np.ascontiguousarray(ids, dtype=np.uint32)
        table = np.zeros(self.keys, dtype=np.int32)
        counts = np.zeros(len(self.names), dtype=np.uint64)
        rv = (C.c_uint8 * x.shape[0])(*run) if run is not None else None
        p = np.ascontiguousarray(pred, dtype=np.uint32) if pred is not None else np.zeros((1, 1), np.uint32)
        self.tsa.check(self.L.tsa_test_dgcore_token_pred(self.h, x.ctypes.data_as(C.POINTER(u32)), x.shape[1],
                                                         p.ctypes.data_as(C.POINTER(u32)),
                                                         p.shape[1] if pred is not None else 0, rv,
                                                         table.ctypes.data_as(C.POINTER(C.c_int32)),
                                                         counts.ctypes.data_as(C.POINTER(u64)), len(self.names)))
        return table, {k: int(v) for k, v in zip(self.names, counts)}

    def set_policy(self, policy):
        self.tsa.check(self.L.tsa_test_dgcore_set_policy(self.h, policy))

    def set_keep(self, keys):
        k = np.ascontiguousarray(np.asarray(keys, dtype=np.uint32))
        self.tsa.check(self.L.tsa_test_dgcore_set_keep(self.h, k.ctypes.data_as(C.POINTER(u32)), len(k)))

    def set_wb_defer(self, on):
        self.tsa.check(self.L.tsa_test_dgcore_set_wb_defer(self.h, int(on)))

    def host_order(self):
        out = np.zeros(self.keys, dtype=np.uint32)
        n = self.L.tsa_test_dgcore_host_order(self.h, out.ctypes.data_as(C.POINTER(u32)), self.keys)
        return [int(v) for v in out[:n]]

    def land_owner(self):
        out = np.zeros(4096, dtype=np.uint32)
        n = self.L.tsa_test_dgcore_land_owner(self.h, out.ctypes.data_as(C.POINTER(u32)), 4096)
        return [int(v) for v in out[:n]]

    def close(self):
        if self.h:
            self.L.tsa_test_dgcore_close(self.h)
            self.h = None


def _case(seed, three):
    rng = np.random.default_rng(seed)
    G = int(rng.integers(2, 7))
    n_units = [int(rng.integers(4, 17)) for _ in range(G)]
    keys = sum(n_units)
    B = int(rng.integers(1, 5))
    repeats = bool(rng.integers(0, 4) == 0)
    prio = [int(k) for k in rng.permutation(keys)]
    R = int(rng.integers(0, keys // 2 + 1))
    D = int(rng.integers(1, 5))
    non_res = keys - R
    D = min(D, max(non_res, 1))
    persistent = R + D
    spare_target = int(rng.integers(max(0, D - 1), D + 1))
    order = prio[:R] + list(range(keys))  # the residents by priority, then key order (as the context builds it)
    residents = set(prio[:R])
    Q = int(rng.integers(1, 7))
    inclusive = int(rng.integers(0, Q)) if rng.integers(0, 2) else 0
    wb_defer = int(rng.integers(0, 2))
    parts = [int(p) for p in rng.choice([256, 512, 1024], size=int(rng.integers(1, 4)))]
    disk = None
    if three:
        cand = [k for k in range(keys) if k not in residents]
        f = int(rng.integers(1, max(2, len(cand))))
        file_keys = set(int(k) for k in rng.choice(cand, size=min(f, len(cand)), replace=False))
        flags = [1 if k in file_keys else 0 for k in range(keys)]
        P = non_res - len(file_keys)
        blocks = P + Q
        disk = dict(flags=flags, home_blocks=P, disk_staging=int(rng.integers(1, 9)),
                    clean_evict=int(rng.integers(0, 2)))
    else:
        blocks = non_res + Q
    tokens = int(rng.integers(16, 33))
    routes = np.zeros((tokens, G, B), dtype=np.uint32)
    perms = [rng.permutation(n) for n in n_units]
    for t in range(tokens):
        for g in range(G):
            w = 1.0 / np.arange(1, n_units[g] + 1) ** 1.1
            w /= w.sum()
            if repeats:
                ids = rng.choice(n_units[g], size=B, replace=True, p=w)
            else:
                ids = rng.choice(n_units[g], size=min(B, n_units[g]), replace=False, p=w)
                ids = np.resize(ids, B)
            routes[t, g] = perms[g][ids]
    return dict(n_units=n_units, persistent=persistent, bank=B, blocks=blocks, spare_target=spare_target,
                parts=parts, order=order, wb_defer=wb_defer, inclusive=inclusive, disk=disk, routes=routes)


def _score(seed, n_units, policy=None):
    """Scored eviction options drawn per seed: SCORED or SCORED_AUTO, default or random weights (summing to 1000),
    1-3 verify rows per boundary (AUTO ranks only above one), and sometimes starting counts, a few cells saturated so
    that increments are dropped."""
    rng = np.random.default_rng(seed + 77)
    pol = policy if policy is not None else int(rng.integers(1, 3))
    if rng.integers(0, 2):
        a, b = sorted(int(x) for x in rng.integers(0, 1001, size=2))
        w = (a, b - a, 1000 - b)
    else:
        w = (700, 200, 100)
    rows = int(rng.integers(1, 4))
    cells = None
    if rng.integers(0, 3) == 0:
        cells = []
        for n in n_units:
            t = rng.integers(0, 50, size=n * n).astype(np.uint64)
            hot = rng.random(n * n) < 0.05
            t[hot] = 0xFFFFFFFF
            cells += [int(v) for v in t]
    return dict(policy=pol, w=w, rows=rows, cells=cells)


def _preds(rng, routes, n_units, k):
    """Per token [G][k]: for layer g the ids predicted for layer g + 1 - mostly its true next ids, some random, a few
    out of range (pred_invalid); the last row is unused."""
    T, G, _ = routes.shape
    out = np.zeros((T, G, k), dtype=np.uint32)
    for t in range(T):
        for g in range(G - 1):
            nu = n_units[g + 1]
            for i in range(k):
                r = rng.random()
                if r < 0.6 and i < routes.shape[2]:
                    out[t, g, i] = routes[t, g + 1, i]
                elif r < 0.95:
                    out[t, g, i] = rng.integers(0, nu)
                else:
                    out[t, g, i] = nu + int(rng.integers(0, 3))
    return out


def _run(seed, three, score=None, switch=None, partial=False, predict=0, disk_prefetch=0, keep=False, sched=False,
         bank_keep=0, landing=None):
    """switch: (token, policy) - both cores switch policy between tokens there. partial: each token exports a random
    nonempty subset of the gated layers (ss_begin's rows), the others keep their state. keep: now and then, between
    tokens, a new keep list (ss_dg_keep: units no boundary may evict; sometimes empty, sometimes with keys off the
    device). sched: now and then write-back deferral is switched (ss_dg_set_sched)."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    c = _case(seed, three)
    if disk_prefetch and c["disk"]:
        c["disk"]["disk_prefetch"] = 1
    if bank_keep and c["disk"]:
        c["disk"]["bank_keep"] = bank_keep
    if landing and c["disk"]:
        c["disk"]["landing_blocks"], c["disk"]["landing_ttl"] = landing
    kw = dict(wb_defer=c["wb_defer"], inclusive=c["inclusive"])
    ours = OurCore(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"], c["order"],
                   disk=c["disk"], score=score, **kw)
    theirs = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                       c["order"], disk=c["disk"], score=score, **kw)
    seen = {}
    rng = np.random.default_rng(seed + 5)
    preds = _preds(np.random.default_rng(seed + 9), c["routes"], c["n_units"], predict) if predict else None
    keys = sum(c["n_units"])
    defer = c["wb_defer"]
    try:
        for t, ids in enumerate(c["routes"]):
            if switch and t == switch[0]:
                ours.set_policy(switch[1])
                theirs.set_policy(switch[1])
            if keep and rng.random() < 0.3:
                kk = [int(k) for k in rng.choice(keys, size=int(rng.integers(0, max(2, keys // 3))), replace=False)]
                ours.set_keep(kk)
                theirs.set_keep(kk)
            if sched and rng.random() < 0.25:
                defer = 1 - defer
                ours.set_wb_defer(defer)
                theirs.set_wb_defer(defer)
            run = None
            if partial:
                run = [int(v) for v in rng.integers(0, 2, size=ids.shape[0])]
                run[int(rng.integers(0, ids.shape[0]))] = 1
            pr = preds[t] if predict else None
            got_t, got = ours.token(ids, run, pr)
            want_t, want = theirs.token(ids, pred=pr, run=run)
            assert np.array_equal(got_t, want_t), (seed, t, "table")
            for k, v in got.items():
                assert v == want[k], (seed, t, k, v, want[k])
            if three:
                assert ours.host_order() == theirs.host_order(), (seed, t, "pinned recency order")
            if landing:
                assert ours.land_owner() == theirs.land_owner(), (seed, t, "landing blocks")
            for k in got:
                seen[k] = seen.get(k, 0) + got[k]
        return seen
    finally:
        ours.close()
        theirs.close()


@pytest.mark.parametrize("seed", range(150))
def test_two_tier_placement_matches_reference(seed):
    _run(seed, False)


@pytest.mark.parametrize("seed", range(150))
def test_three_tier_placement_matches_reference(seed):
    _run(1000 + seed, True)


def test_cases_exercise_the_paths():
    """The random cases together reach every path the parity relies on (a case generator that stopped producing
    misses, write-backs or file reads would pass vacuously)."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    tot2, tot3 = {}, {}
    for s in range(40):
        for k, v in _run(s, False).items():
            tot2[k] = tot2.get(k, 0) + v
        for k, v in _run(1000 + s, True).items():
            tot3[k] = tot3.get(k, 0) + v
    for k in ("misses", "bank_serves", "evicted", "writebacks_done", "resurrected", "inclusive_drops", "wb_forced"):
        assert tot2[k] > 0, k
    tp = {}
    for s in range(24):
        for k, v in _run(7000 + s, s % 2 == 1, predict=int(1 + s % 4), disk_prefetch=int(s % 4 == 1)).items():
            tp[k] = tp.get(k, 0) + v
    for k in ("prefetched", "prefetch_used", "pred_invalid", "predicted_true", "disk_reads"):
        assert tp[k] > 0, k
    for k in ("disk_reads", "disk_drops", "disk_discards", "clean_drops", "writebacks_done", "bank_serves"):
        assert tot3[k] > 0, k


@pytest.mark.parametrize("seed", range(120))
def test_scored_two_tier_matches_reference(seed):
    """Scored eviction (SCORED / SCORED_AUTO): victims lowest (score, demand epoch, recency stamp) first from the
    transition counts, the 16-union window and the recency term, through the same acceptance loop as LRU."""
    c = _case(2000 + seed, False)
    _run(2000 + seed, False, score=_score(seed, c["n_units"]))


@pytest.mark.parametrize("seed", range(60))
def test_scored_three_tier_matches_reference(seed):
    c = _case(3000 + seed, True)
    _run(3000 + seed, True, score=_score(seed, c["n_units"]))


@pytest.mark.parametrize("seed", range(30))
def test_policy_switch_matches_reference(seed):
    """ss_dg_set_policy between tokens: drained, the learning reset to the open counts, stamps renumbered in recency
    order; placement and recency kept. Both directions and AUTO."""
    c = _case(4000 + seed, bool(seed % 2))
    rng = np.random.default_rng(seed)
    sc = _score(seed, c["n_units"])
    _run(4000 + seed, bool(seed % 2), score=sc, switch=(int(rng.integers(3, 12)), int(rng.integers(0, 3))))


@pytest.mark.parametrize("seed", range(40))
def test_partial_exports_match_reference(seed):
    """Tokens that export only some gated layers (ss_begin's rows): LRU, and scored, where a layer left out scores
    from its older history at the boundary."""
    c = _case(6000 + seed, bool(seed % 3 == 0))
    score = _score(seed, c["n_units"]) if seed % 2 else None
    _run(6000 + seed, bool(seed % 3 == 0), score=score, partial=True)


@pytest.mark.parametrize("seed", range(60))
def test_prefetch_matches_reference(seed):
    """Predictions for the next layer (serve_prediction): prefetches within the per-layer and per-token budgets and
    the reserve, their use, resurrection from banks, invalid ids; three-tier cases read file-homed units ahead
    (dg_disk_prefetch) in half of them; some cases export only some layers."""
    three = seed % 2 == 1
    _run(7000 + seed, three, predict=int(1 + seed % 4), disk_prefetch=int(seed % 4 == 1), partial=seed % 5 == 0)


@pytest.mark.parametrize("seed", range(20))
def test_scored_prefetch_matches_reference(seed):
    c = _case(8000 + seed, False)
    _run(8000 + seed, False, score=_score(seed, c["n_units"]), predict=int(1 + seed % 3))


@pytest.mark.parametrize("seed", range(60))
def test_keep_lists_match_reference(seed):
    """ss_dg_keep: between tokens a keep list (every gated layer's set) that the next boundaries must not evict, under
    LRU and scored victims, two and three tiers, with predictions in some cases."""
    three = seed % 3 == 0
    c = _case(9000 + seed, three)
    score = _score(seed, c["n_units"]) if seed % 4 == 1 else None
    _run(9000 + seed, three, score=score, keep=True, predict=int(seed % 5 == 2) * 2)


@pytest.mark.parametrize("seed", range(40))
def test_wb_defer_switch_matches_reference(seed):
    """ss_dg_set_sched's wb_defer between tokens: off submits every deferred write-back first; on again restarts the
    per-layer credit and carry as after open."""
    three = seed % 2 == 1
    _run(9500 + seed, three, sched=True, keep=seed % 3 == 0)


def test_keep_lists_protect_units():
    """The keep cases are not vacuous: over the seeds, some boundaries would have evicted a kept unit (the tables with
    and without the keep lists differ)."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    differ = 0
    for seed in range(20):
        c = _case(9000 + seed, False)
        kw = dict(wb_defer=c["wb_defer"], inclusive=c["inclusive"])
        a = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                      c["order"], **kw)
        b = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                      c["order"], **kw)
        try:
            a.set_keep(list(range(0, sum(c["n_units"]), 2)))
            for ids in c["routes"]:
                ta, _ = a.token(ids)
                tb, _ = b.token(ids)
                differ += int(not np.array_equal(ta, tb))
        finally:
            a.close()
            b.close()
    assert differ > 0


def test_lru_open_refuses_a_switch_to_scoring():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    c = _case(5, False)
    ours = OurCore(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"], c["order"],
                   wb_defer=1, inclusive=0)
    theirs = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                       c["order"])
    try:
        with pytest.raises(Exception):
            ours.set_policy(1)
        with pytest.raises(RuntimeError):
            theirs.set_policy(1)
        ours.set_policy(0)  # LRU to LRU is allowed
        theirs.set_policy(0)
    finally:
        ours.close()
        theirs.close()


def test_scored_cases_choose_other_victims_than_lru():
    """The scored runs are not LRU in disguise: over the seeds, scored victims are taken, some transition cells
    saturate, and for some seeds the slot tables after a token differ from the same run under LRU (with AUTO at one
    row they never do)."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    differ = victims = saturated = 0
    for seed in range(30):
        c = _case(2000 + seed, False)
        sc = _score(seed, c["n_units"], policy=1)
        kw = dict(wb_defer=c["wb_defer"], inclusive=c["inclusive"])
        a = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                      c["order"], score=sc, **kw)
        b = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                      c["order"], **kw)
        auto = ref.RefDg(c["n_units"], c["persistent"], c["bank"], c["blocks"], c["spare_target"], c["parts"],
                         c["order"], score=dict(sc, policy=2, rows=1), **kw)
        try:
            for ids in c["routes"]:
                ta, ca = a.token(ids)
                tb, _ = b.token(ids)
                tc, cc = auto.token(ids)
                differ += int(not np.array_equal(ta, tb))
                assert np.array_equal(tb, tc)
                assert cc["scored_victims"] == 0
            victims += ca["scored_victims"]
            saturated += ca["score_saturated"]
        finally:
            a.close()
            b.close()
            auto.close()
    assert victims > 0 and differ > 0 and saturated > 0


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("seed", range(60))
def test_bank_keep_matches_reference(seed, mode):
    """dg_bank_keep: a bank-served demand file miss read into a pinned block (a free one, else the longest-homed
    unit's), which becomes its home at the bank's release - at the front of the pinned order (1) or behind its front
    half (2); tables, counters (bank_kept, bank_keep_drops, bank_keep_rereads) and the pinned order every token
    (reference src/dg_core.cpp keep_block / hpush_mid, docs/design.md 3.16)."""
    _run(3000 + seed, True, bank_keep=mode, predict=int(seed % 3), disk_prefetch=int(seed % 4 == 1))


def test_bank_keep_cases_exercise_the_paths():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    tot = {}
    for s in range(30):
        for k, v in _run(3000 + s, True, bank_keep=1 + s % 2).items():
            tot[k] = tot.get(k, 0) + v
    for k in ("bank_kept", "bank_keep_drops", "bank_keep_rereads", "bank_serves", "disk_drops"):
        assert tot[k] > 0, k


@pytest.mark.parametrize("ttl", [0, 1, 3])
@pytest.mark.parametrize("seed", range(40))
def test_landings_match_reference(seed, ttl):
    """dg_landing_blocks: a prediction of a file-homed unit reads it into a landing block (no slot, outside the
    prefetch budgets; none free: dropped), a demand copies it from there into the slot a file miss would have taken,
    and a landing goes back to its file after its target layer (TTL 0) or after TTL boundaries undemanded; tables,
    counters (landing_issued / promoted / expired / expired_layer / dropped_full / read_bytes, the landed units and
    free blocks) and every landing block's key every token (reference src/dg_core.cpp:501-610, :1146-1330, :1650-1663,
    docs/design.md 3.15)."""
    blocks = 1 + seed % 6
    _run(5000 + seed, True, predict=1 + seed % 4, disk_prefetch=int(seed % 5 == 2), bank_keep=int(seed % 7 == 3),
         landing=(blocks, ttl), keep=seed % 4 == 1, sched=seed % 6 == 5)


def test_landing_cases_exercise_the_paths():
    if not ref.available():
        pytest.skip("oracle/_ref (the reference core) is not built")
    tot = {}
    for s in range(24):
        for ttl in (0, 2):
            for k, v in _run(5000 + s, True, predict=1 + s % 4, landing=(1 + s % 6, ttl)).items():
                tot[k] = tot.get(k, 0) + v
    for k in ("landing_issued", "landing_promoted", "landing_expired", "landing_expired_layer", "landing_dropped_full",
              "disk_reads"):
        assert tot[k] > 0, k
