"""ORACLE (test infrastructure only): the reference's own CPU library (oracle/_ref/libtsref_harness.so, compiled from its
sources by oracle/Makefile) driven through its C ABI, and its DgCore on an immediate transport. The library is loaded
privately (RTLD_LOCAL) so its ss_* symbols never meet the product's."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import HERE

HARNESS = HERE / "_ref" / "libtsref_harness.so"
u32, u64, i32, vp = C.c_uint32, C.c_uint64, C.c_int32, C.c_void_p

_lib = None


def available() -> bool:
    return HARNESS.exists()


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not HARNESS.exists():
            raise RuntimeError(f"{HARNESS} is not built (make -C oracle ref, where the reference sources exist)")
        from tierstream_amd.ss import SsBudget, SsLayerStats, SsLayerView, SsOptions
        L = C.CDLL(str(HARNESS), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        st = C.c_int
        sigs = {
            "ss_last_error": (C.c_char_p, []),
            "ss_desc_from_json": (st, [C.c_char_p, C.c_size_t, C.POINTER(vp)]),
            "ss_desc_free": (None, [vp]),
            "ss_desc_to_json": (st, [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]),
            "ss_desc_n_layers": (C.c_int, [vp]),
            "ss_desc_layer_units": (C.c_int, [vp, C.c_int]),
            "ss_desc_unit_bytes": (u64, [vp, C.c_int]),
            "ss_budget_defaults_sized": (None, [C.POINTER(SsBudget), u32]),
            "ss_options_defaults_sized": (None, [C.POINTER(SsOptions), u32]),
            "ss_plan_make": (st, [vp, C.POINTER(SsBudget), C.POINTER(C.c_double), C.c_size_t, C.POINTER(vp)]),
            "ss_plan_free": (None, [vp]),
            "ss_plan_from_tiers": (st, [vp, C.POINTER(SsBudget), C.POINTER(C.c_uint8), C.c_size_t, C.POINTER(vp)]),
            "ss_plan_unit_tier": (C.c_int, [vp, C.c_int, C.c_int]),
            "ss_plan_to_json": (st, [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]),
            "ss_plan_from_json": (st, [vp, C.POINTER(SsBudget), C.c_char_p, C.c_size_t, C.POINTER(vp)]),
            "ss_free": (None, [vp]),
            "ss_open": (st, [vp, C.POINTER(SsBudget), vp, C.POINTER(SsOptions), C.POINTER(vp)]),
            "ss_close": (None, [vp]),
            "ss_begin": (st, [vp, vp, C.c_int]),
            "ss_layer_routes": (st, [vp, C.c_int, C.POINTER(i32), C.c_int]),
            "ss_layer_all": (st, [vp, C.c_int]),
            "ss_prefetch": (st, [vp, C.c_int, C.POINTER(i32), C.c_int, C.c_int]),
            "ss_acquire": (st, [vp, C.c_int, vp, C.POINTER(SsLayerView)]),
            "ss_acquire_groups": (st, [vp, C.c_int, vp, C.POINTER(SsLayerView)]),
            "ss_group_wait": (st, [vp, C.c_int, C.c_int, vp]),
            "ss_release": (st, [vp, C.c_int, vp]),
            "ss_end": (st, [vp]),
            "ss_host_prefetch_layer": (st, [vp, C.c_int]),
            "ss_stats_total": (st, [vp, C.POINTER(SsLayerStats)]),
            "ss_stats_to_json": (st, [vp, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
            "ref_region_of": (C.c_int, [vp, u64, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(u64)]),
            "refdg_open": (vp, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, u32, u32, u32, u32,
                                C.POINTER(u64), u32, C.POINTER(u32), u32]),
            "refdg_token": (C.c_int, [vp, C.POINTER(u32), u32, C.POINTER(u32), u32, C.POINTER(i32), C.POINTER(u64)]),
            "refdg_token_run": (C.c_int, [vp, C.POINTER(u32), u32, C.POINTER(u32), u32, C.POINTER(C.c_uint8),
                                          C.POINTER(i32), C.POINTER(u64)]),
            "refdg_counter_names": (C.c_char_p, []),
            "refdg_residency": (u32, [vp, C.POINTER(u32), u32]),
            "refdg_open_disk": (vp, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64), u32,
                                     C.POINTER(u32), u32, u32, u32, u32, u32, C.POINTER(C.c_uint8)]),
            "refdg_open_disk_keep": (vp, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64), u32,
                                          C.POINTER(u32), u32, u32, u32, u32, u32, C.POINTER(C.c_uint8), u32]),
            "refdg_open_disk_land": (vp, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64), u32,
                                          C.POINTER(u32), u32, u32, u32, u32, u32, C.POINTER(C.c_uint8), u32, u32,
                                          u32]),
            "refdg_land_owner": (u32, [vp, C.POINTER(u32), u32]),
            "refdg_open_scored": (vp, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64), u32,
                                       C.POINTER(u32), u32, u32, u32, u32, u32, u32, C.POINTER(u32), u32, u32, u32,
                                       C.POINTER(C.c_uint8)]),
            "refdg_set_policy": (C.c_int, [vp, u32]),
            "refdg_set_keep": (C.c_int, [vp, C.POINTER(u32), u32]),
            "refdg_set_wb_defer": (C.c_int, [vp, u32]),
            "refdg_table": (u32, [vp, C.POINTER(i32), u32]),
            "refdg_set_budgets": (C.c_int, [vp, u32, u32, u32]),
            "refdg_set_clean_evict": (C.c_int, [vp, u32]),
            "refdg_profile_check": (C.c_int, [C.c_char_p, u64, C.POINTER(u32), u32, C.c_char_p]),
            "refdg_score_identity": (C.c_int, [u32, C.POINTER(u32), C.POINTER(u32), C.POINTER(u64), C.POINTER(u64),
                                               C.c_char_p]),
            "refdg_host_order": (u32, [vp, C.POINTER(u32), u32]),
            "refdg_close": (None, [vp]),
            "refdg_cpu_baseline": (C.c_int, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64), u32,
                                              u64, C.POINTER(u32), u32, C.c_char_p, C.POINTER(u64), C.POINTER(u64),
                                              C.POINTER(u32), u32, u32, C.c_int, C.POINTER(C.c_double),
                                              C.POINTER(u64), u32, u32]),
            "refdg_cpu_baseline_disk": (C.c_int, [C.POINTER(u32), u32, u32, u32, u32, u32, u32, u32, C.POINTER(u64),
                                                   u32, u64, C.POINTER(u32), u32, C.POINTER(C.c_char_p), u32,
                                                   C.POINTER(u32), C.POINTER(u64), C.POINTER(u64), C.POINTER(u32), u32,
                                                   u32, C.c_int, C.POINTER(C.c_uint8), u32, u32, u32,
                                                   C.POINTER(C.c_double), C.POINTER(u64), u32, u32]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _ck(st):
    if st != 0:
        raise RuntimeError(f"reference status {st}: {lib().ss_last_error().decode()}")


def desc_roundtrip(desc_json: str) -> dict:
    """The reference's canonical JSON of a descriptor (ss_desc_from_json, then ss_desc_to_json)."""
    import json
    L = lib()
    d = vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    try:
        s, n = C.c_char_p(), C.c_size_t()
        _ck(L.ss_desc_to_json(d, C.byref(s), C.byref(n)))
        out = json.loads(C.string_at(s, n.value).decode())
        L.ss_free(s)
        return out
    finally:
        L.ss_desc_free(d)


def plan_status(desc_json: str, budget, benefit=None) -> int:
    """The reference's status for planning (0 = a plan was made)."""
    L = lib()
    d, p = vp(), vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    try:
        ben = (C.c_double * len(benefit))(*benefit) if benefit is not None else None
        st = L.ss_plan_make(d, C.byref(budget), ben, len(benefit) if benefit is not None else 0, C.byref(p))
        if st == 0:
            L.ss_plan_free(p)
        return st
    finally:
        L.ss_desc_free(d)


def plan_json(desc_json: str, budget, benefit=None) -> dict:
    import json
    L = lib()
    d, p = vp(), vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    try:
        ben = (C.c_double * len(benefit))(*benefit) if benefit is not None else None
        _ck(L.ss_plan_make(d, C.byref(budget), ben, len(benefit) if benefit is not None else 0, C.byref(p)))
        s, n = C.c_char_p(), C.c_size_t()
        _ck(L.ss_plan_to_json(p, C.byref(s), C.byref(n)))
        out = json.loads(C.string_at(s, n.value).decode())
        L.ss_free(s)
        L.ss_plan_free(p)
        return out
    finally:
        L.ss_desc_free(d)


def host_run(desc_json: str, budget, options, routes: np.ndarray, mode: int = 0, prefetch: np.ndarray | None = None,
             checksums: bool = True, host_lookahead: int = 0, tiers=None):
    """The reference CPU backend over `routes` ([steps][layers][max_ids], -1 padded), the engine loop of the product's
    tse_host_run. Per step: {"stats": ..., "tables": [[(kind, index, offset) per unit] per layer], "groups": [...],
    "checksums": [[...]]}; checksums are of the bytes the reference's table entries point at (host memory).
    prefetch (same shape): after layer l's acquire, ss_prefetch of layer l + 1 with its row, CERTAIN on even steps and
    SPECULATIVE on odd ones. host_lookahead H: after each layer's routes, ss_host_prefetch_layer of the next H layers
    with units (as the product's loop). tiers: the plan's tiers, one per unit in descriptor order (None: the planner's
    plan)."""
    from tierstream_amd.ss import SsLayerStats, SsLayerView
    from .fixtures import engine_checksum
    L = lib()
    d, ctx = vp(), vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    options.backend = 0  # SS_BACKEND_CPU
    out = []
    plan = vp()
    try:
        if tiers is not None:
            t = (C.c_uint8 * len(tiers))(*tiers)
            _ck(L.ss_plan_from_tiers(d, C.byref(budget), t, len(tiers), C.byref(plan)))
        _ck(L.ss_open(d, C.byref(budget), plan if tiers is not None else None, C.byref(options), C.byref(ctx)))
        nl = L.ss_desc_n_layers(d)
        steps, _, max_ids = routes.shape
        for s in range(steps):
            before = SsLayerStats()
            _ck(L.ss_stats_total(ctx, C.byref(before)))
            _ck(L.ss_begin(ctx, None, 0))
            step = {"tables": [], "groups": [], "checksums": []}
            for l in range(nl):
                nu = L.ss_desc_layer_units(d, l)
                if nu <= 0:
                    step["tables"].append([])
                    step["groups"].append([])
                    step["checksums"].append([])
                    continue
                r = np.ascontiguousarray(routes[s, l], dtype=np.int32)
                n = int(np.sum(r >= 0)) if mode != 1 else 0
                if mode == 1:
                    _ck(L.ss_layer_all(ctx, l))
                else:
                    _ck(L.ss_layer_routes(ctx, l, r.ctypes.data_as(C.POINTER(i32)), n))
                left = host_lookahead
                for h in range(l + 1, nl):
                    if left <= 0:
                        break
                    if L.ss_desc_layer_units(d, h) > 0:
                        _ck(L.ss_host_prefetch_layer(ctx, h))
                        left -= 1
                v = SsLayerView()
                _ck((L.ss_acquire_groups if mode == 2 else L.ss_acquire)(ctx, l, None, C.byref(v)))
                if mode == 2:
                    for gi in range(1, v.n_groups):
                        _ck(L.ss_group_wait(ctx, l, gi, None))
                if prefetch is not None and l + 1 < nl and L.ss_desc_layer_units(d, l + 1) > 0:
                    q = np.ascontiguousarray(prefetch[s, l + 1], dtype=np.int32)
                    m = int(np.sum(q >= 0))
                    if m:
                        _ck(L.ss_prefetch(ctx, l + 1, q.ctypes.data_as(C.POINTER(i32)), m, s % 2))
                tab = []
                for u in range(nu):
                    a = int(v.table_host[u])
                    k, i, off = C.c_int(), C.c_int(), u64()
                    L.ref_region_of(ctx, a, C.byref(k), C.byref(i), C.byref(off))
                    tab.append((k.value, i.value, int(off.value)) if a else (0, -1, 0))
                step["tables"].append(tab)
                step["groups"].append([[v.groups[gi].units[j] for j in range(v.groups[gi].n_units)]
                                       for gi in range(v.n_groups)])
                ub = int(L.ss_desc_unit_bytes(d, l))
                ids = list(range(nu)) if mode == 1 else [int(x) for x in r[:n]]
                cks = []
                for u in (ids if checksums else []):
                    a = int(v.table_host[u])
                    cks.append(engine_checksum(np.frombuffer(C.string_at(a, ub), dtype=np.uint8)) if a else 0)
                step["checksums"].append(cks)
                _ck(L.ss_release(ctx, l, None))
            _ck(L.ss_end(ctx))
            after = SsLayerStats()
            _ck(L.ss_stats_total(ctx, C.byref(after)))
            step["stats"] = {k: after.as_dict()[k] - before.as_dict()[k] for k in after.as_dict()}
            if s == steps - 1:  # the stats-v1 document after the last step
                txt, n = C.c_void_p(), C.c_size_t()
                _ck(L.ss_stats_to_json(ctx, C.byref(txt), C.byref(n)))
                step["stats_json"] = C.string_at(txt, n.value).decode()
                L.ss_free(txt)
            out.append(step)
    finally:
        if ctx:
            L.ss_close(ctx)
        if tiers is not None and plan:
            L.ss_plan_free(plan)
        L.ss_desc_free(d)
    return out


class RefDg:
    """The reference DgCore on an immediate transport (its canonical schedule)."""

    def __init__(self, n_units, persistent, bank, blocks, spare_target, part_bytes, order, prefetch_reserve=0xFFFFFFFF,
                 pf_layer=4, pf_token=48, wb_defer=1, wb_on_d2h=1, inclusive=0, disk=None, score=None):
        """disk (three-tier): dict(flags=[keys] 0/1 file-tier, home_blocks=P, disk_staging=S, clean_evict=0,
        disk_prefetch=0, bank_keep=0, landing_blocks=0, landing_ttl=0); the prefetch budgets then take their defaults. score (scored eviction): dict(policy=1 SCORED
        or 2 SCORED_AUTO, w=(w_trans, w_freq, w_rec), rows=verify rows per boundary, cells=None or the starting
        transition counts, per gated layer units^2 row-major, concatenated); the prefetch budgets take their defaults
        and disk prefetch stays off."""
        L = lib()
        nu = (u32 * len(n_units))(*n_units)
        pb = (u64 * len(part_bytes))(*part_bytes)
        od = (u32 * len(order))(*order)
        if score is not None:
            w = score.get("w", (700, 200, 100))
            cells = score.get("cells")
            cp = (u32 * len(cells))(*cells) if cells is not None else None
            fl = (C.c_uint8 * sum(n_units))(*disk["flags"]) if disk else None
            dk = disk or {}
            self.h = L.refdg_open_scored(nu, len(n_units), persistent, bank, blocks, spare_target, wb_defer, inclusive,
                                         pb, len(part_bytes), od, len(order), score["policy"], w[0], w[1], w[2],
                                         score.get("rows", 1), cp, dk.get("home_blocks", 0), dk.get("disk_staging", 0),
                                         dk.get("clean_evict", 0), fl)
        elif disk is None:
            self.h = L.refdg_open(nu, len(n_units), persistent, bank, blocks, spare_target, prefetch_reserve, pf_layer,
                                  pf_token, wb_defer, wb_on_d2h, inclusive, pb, len(part_bytes), od, len(order))
        else:
            fl = (C.c_uint8 * sum(n_units))(*disk["flags"])
            self.h = L.refdg_open_disk_land(nu, len(n_units), persistent, bank, blocks, spare_target, wb_defer,
                                            inclusive, pb, len(part_bytes), od, len(order), disk["home_blocks"],
                                            disk["disk_staging"], disk.get("clean_evict", 0),
                                            disk.get("disk_prefetch", 0), fl, disk.get("bank_keep", 0),
                                            disk.get("landing_blocks", 0), disk.get("landing_ttl", 0))
        if not self.h:
            raise RuntimeError("refdg_open failed")
        self.keys = sum(n_units)
        self.G = len(n_units)
        self.names = L.refdg_counter_names().decode().split()

    def token(self, ids: np.ndarray, pred: np.ndarray | None = None, run=None):
        """ids uint32 [G][n]; run: the gated layers the token exports (None: all); returns (table int32 [keys],
        counters dict)."""
        L = lib()
        x = np.ascontiguousarray(ids, dtype=np.uint32)
        n = x.shape[1]
        p = np.ascontiguousarray(pred, dtype=np.uint32) if pred is not None else np.zeros((1, 1), np.uint32)
        n_pred = p.shape[1] if pred is not None else 0
        table = np.zeros(self.keys, dtype=np.int32)
        counts = np.zeros(len(self.names), dtype=np.uint64)
        rv = (C.c_uint8 * self.G)(*run) if run is not None else None
        st = L.refdg_token_run(self.h, x.ctypes.data_as(C.POINTER(u32)), n, p.ctypes.data_as(C.POINTER(u32)), n_pred,
                               rv, table.ctypes.data_as(C.POINTER(i32)), counts.ctypes.data_as(C.POINTER(u64)))
        if st != 0:
            raise RuntimeError("refdg_token failed")
        return table, {k: int(v) for k, v in zip(self.names, counts)}

    def set_policy(self, policy):
        if lib().refdg_set_policy(self.h, policy) != 0:
            raise RuntimeError("refdg_set_policy failed")

    def set_keep(self, keys):
        """The keys every later boundary must not evict (ss_dg_keep of every gated layer, concatenated)."""
        k = np.ascontiguousarray(np.asarray(keys, dtype=np.uint32))
        lib().refdg_set_keep(self.h, k.ctypes.data_as(C.POINTER(u32)), len(k))

    def set_wb_defer(self, on):
        if lib().refdg_set_wb_defer(self.h, int(on)) != 0:
            raise RuntimeError("refdg_set_wb_defer failed")

    def table(self) -> np.ndarray:
        """The slot table now (after open: the seeded placement)."""
        out = np.zeros(self.keys, dtype=np.int32)
        lib().refdg_table(self.h, out.ctypes.data_as(C.POINTER(i32)), self.keys)
        return out

    def set_budgets(self, spare_target, per_layer, per_token):
        if lib().refdg_set_budgets(self.h, spare_target, per_layer, per_token) != 0:
            raise RuntimeError("refdg_set_budgets failed")

    def set_clean_evict(self, on):
        if lib().refdg_set_clean_evict(self.h, int(on)) != 0:
            raise RuntimeError("refdg_set_clean_evict failed")

    def residency(self):
        L = lib()
        out = np.zeros(self.keys, dtype=np.uint32)
        n = L.refdg_residency(self.h, out.ctypes.data_as(C.POINTER(u32)), self.keys)
        return [int(x) for x in out[:n]]

    def host_order(self):
        """Three-tier: the pinned homes, most recently homed first."""
        out = np.zeros(self.keys, dtype=np.uint32)
        n = lib().refdg_host_order(self.h, out.ctypes.data_as(C.POINTER(u32)), self.keys)
        return [int(x) for x in out[:n]]

    def land_owner(self):
        """Landings: per landing block the key it holds (0xFFFFFFFF: none)."""
        out = np.zeros(4096, dtype=np.uint32)
        n = lib().refdg_land_owner(self.h, out.ctypes.data_as(C.POINTER(u32)), 4096)
        return [int(x) for x in out[:n]]

    def close(self):
        if self.h:
            lib().refdg_close(self.h)
            self.h = None


def cpu_baseline(n_units, persistent, bank, blocks, spare_target, part_bytes, host_stride, order, path, unit_offsets,
                 hashes, ids: np.ndarray, wb_defer=1, inclusive=0, setup_threads=16, warm=0, policy=0):
    """The reference DgCore on a synchronous memcpy transport over host memory (refdg_cpu_baseline), timed per token
    on the calling thread. ids uint32 [warm + tokens][G][n]: the first `warm` tokens run untimed. policy: 0 LRU,
    1 SCORED, 2 SCORED_AUTO. Returns (token_ms [tokens], counters dict over the timed tokens)."""
    L = lib()
    x = np.ascontiguousarray(ids, dtype=np.uint32)
    tokens, G, n = x.shape
    nu = (u32 * G)(*n_units)
    pb = (u64 * len(part_bytes))(*part_bytes)
    od = (u32 * len(order))(*order)
    offs = np.ascontiguousarray(unit_offsets, dtype=np.uint64)
    hs = np.ascontiguousarray(hashes, dtype=np.uint64)
    assert 0 <= warm < tokens, "refdg_cpu_baseline: needs at least one timed token after the warmup"
    ms = np.zeros(tokens - warm, dtype=np.float64)
    out = np.zeros(len(BASELINE_COUNTERS), dtype=np.uint64)
    st = L.refdg_cpu_baseline(nu, G, persistent, bank, blocks, spare_target, wb_defer, inclusive, pb, len(part_bytes),
                              host_stride, od, len(order), str(path).encode(), offs.ctypes.data_as(C.POINTER(u64)),
                              hs.ctypes.data_as(C.POINTER(u64)), x.ctypes.data_as(C.POINTER(u32)), n, tokens - warm,
                              setup_threads, ms.ctypes.data_as(C.POINTER(C.c_double)),
                              out.ctypes.data_as(C.POINTER(u64)), warm, policy)
    if st != 0:
        raise RuntimeError("refdg_cpu_baseline failed")
    return ms, {k: int(v) for k, v in zip(BASELINE_COUNTERS, out)}


# The counters refdg_cpu_baseline* report over their timed tokens, in order.
BASELINE_COUNTERS = ["misses", "fetched", "evicted", "writebacks_done", "hash_mismatches", "copied_bytes", "disk_reads",
                     "disk_drops", "score_layers", "score_candidates"]


def cpu_baseline_disk(n_units, persistent, bank, blocks, spare_target, part_bytes, host_stride, order, paths, path_of,
                      unit_offsets, hashes, ids: np.ndarray, disk_flags, home_blocks, disk_staging, clean_evict=0,
                      wb_defer=1, setup_threads=16, warm=0, policy=0):
    """Three tiers (refdg_cpu_baseline_disk): key k's bytes in paths[path_of[k]] at unit_offsets[k]; the file-tier keys
    (disk_flags) are read synchronously into a staging buffer on a miss (direct I/O where the file system allows it).
    Returns (token_ms [tokens], counters dict)."""
    L = lib()
    x = np.ascontiguousarray(ids, dtype=np.uint32)
    tokens, G, n = x.shape
    nu = (u32 * G)(*n_units)
    pb = (u64 * len(part_bytes))(*part_bytes)
    od = (u32 * len(order))(*order)
    pa = (C.c_char_p * len(paths))(*[str(p).encode() for p in paths])
    po = np.ascontiguousarray(path_of, dtype=np.uint32)
    offs = np.ascontiguousarray(unit_offsets, dtype=np.uint64)
    hs = np.ascontiguousarray(hashes, dtype=np.uint64)
    fl = np.ascontiguousarray(disk_flags, dtype=np.uint8)
    assert 0 <= warm < tokens, "refdg_cpu_baseline_disk: needs at least one timed token after the warmup"
    ms = np.zeros(tokens - warm, dtype=np.float64)
    out = np.zeros(len(BASELINE_COUNTERS), dtype=np.uint64)
    st = L.refdg_cpu_baseline_disk(nu, G, persistent, bank, blocks, spare_target, wb_defer, 0, pb, len(part_bytes),
                                   host_stride, od, len(order), pa, len(paths), po.ctypes.data_as(C.POINTER(u32)),
                                   offs.ctypes.data_as(C.POINTER(u64)), hs.ctypes.data_as(C.POINTER(u64)),
                                   x.ctypes.data_as(C.POINTER(u32)), n, tokens - warm, setup_threads,
                                   fl.ctypes.data_as(C.POINTER(C.c_uint8)), home_blocks, disk_staging, clean_evict,
                                   ms.ctypes.data_as(C.POINTER(C.c_double)), out.ctypes.data_as(C.POINTER(u64)), warm,
                                   policy)
    if st != 0:
        raise RuntimeError("refdg_cpu_baseline_disk failed")
    return ms, {k: int(v) for k, v in zip(BASELINE_COUNTERS, out)}


def host_exclusive(desc_json: str, budget, options, routes: np.ndarray, prefetch: np.ndarray | None = None,
                   mode: int = 0) -> dict:
    """The reference CPU backend in exclusive tier mode over `routes` (ss_layer_routes + ss_acquire per layer; mode 2:
    ss_acquire_groups and every group's wait; prefetch as in host_run): its ss_stats_exclusive after the last forward,
    as a dict."""
    from tierstream_amd.ss import SsExclusiveStats, SsLayerView
    L = lib()
    L.ss_stats_exclusive_sized.restype = C.c_int
    L.ss_stats_exclusive_sized.argtypes = [vp, C.POINTER(SsExclusiveStats), u32]
    d, ctx = vp(), vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    options.backend = 0  # SS_BACKEND_CPU
    try:
        _ck(L.ss_open(d, C.byref(budget), None, C.byref(options), C.byref(ctx)))
        nl = L.ss_desc_n_layers(d)
        for s in range(routes.shape[0]):
            _ck(L.ss_begin(ctx, None, 0))
            for l in range(nl):
                if L.ss_desc_layer_units(d, l) <= 0:
                    continue
                r = np.ascontiguousarray(routes[s, l], dtype=np.int32)
                _ck(L.ss_layer_routes(ctx, l, r.ctypes.data_as(C.POINTER(i32)), int(np.sum(r >= 0))))
                v = SsLayerView()
                _ck((L.ss_acquire_groups if mode == 2 else L.ss_acquire)(ctx, l, None, C.byref(v)))
                if mode == 2:
                    for gi in range(1, v.n_groups):
                        _ck(L.ss_group_wait(ctx, l, gi, None))
                if prefetch is not None and l + 1 < nl and L.ss_desc_layer_units(d, l + 1) > 0:
                    q = np.ascontiguousarray(prefetch[s, l + 1], dtype=np.int32)
                    m = int(np.sum(q >= 0))
                    if m:
                        _ck(L.ss_prefetch(ctx, l + 1, q.ctypes.data_as(C.POINTER(i32)), m, s % 2))
                _ck(L.ss_release(ctx, l, None))
            _ck(L.ss_end(ctx))
        x = SsExclusiveStats()
        _ck(L.ss_stats_exclusive_sized(ctx, C.byref(x), C.sizeof(x)))
        return {k: getattr(x, k) for k, _ in SsExclusiveStats._fields_ if k != "struct_size"}
    finally:
        if ctx:
            L.ss_close(ctx)
        L.ss_desc_free(d)


def host_time(desc_json: str, budget, options, routes: np.ndarray, mode: int = 0):
    """The reference CPU backend's step time over `routes` (the contract calls of tse_host_run's loop: begin, per
    layer routes or layer_all, acquire or acquire_groups with every group waited for, release; end), no tables or
    checksums. Returns (step_ms [steps], open_s)."""
    import time
    from tierstream_amd.ss import SsLayerView
    L = lib()
    d, ctx = vp(), vp()
    b = desc_json.encode()
    _ck(L.ss_desc_from_json(b, len(b), C.byref(d)))
    options.backend = 0  # SS_BACKEND_CPU
    steps, nl, max_ids = routes.shape
    ms = np.zeros(steps)
    try:
        t0 = time.perf_counter()
        _ck(L.ss_open(d, C.byref(budget), None, C.byref(options), C.byref(ctx)))
        open_s = time.perf_counter() - t0
        units = [L.ss_desc_layer_units(d, l) for l in range(nl)]
        rr = [[np.ascontiguousarray(routes[s, l], dtype=np.int32) for l in range(nl)] for s in range(steps)]
        v = SsLayerView()
        for s in range(steps):
            t = time.perf_counter()
            _ck(L.ss_begin(ctx, None, 0))
            for l in range(nl):
                if units[l] <= 0:
                    continue
                r = rr[s][l]
                if mode == 1:
                    _ck(L.ss_layer_all(ctx, l))
                else:
                    _ck(L.ss_layer_routes(ctx, l, r.ctypes.data_as(C.POINTER(i32)), int(np.sum(r >= 0))))
                _ck((L.ss_acquire_groups if mode == 2 else L.ss_acquire)(ctx, l, None, C.byref(v)))
                if mode == 2:
                    for gi in range(1, v.n_groups):
                        _ck(L.ss_group_wait(ctx, l, gi, None))
                _ck(L.ss_release(ctx, l, None))
            _ck(L.ss_end(ctx))
            ms[s] = (time.perf_counter() - t) * 1e3
    finally:
        if ctx:
            L.ss_close(ctx)
        L.ss_desc_free(d)
    return ms, open_s
