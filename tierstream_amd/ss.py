"""ctypes mirror of the strix-stream C ABI the library serves (include/strix_stream/ss.h), plus the synthetic engine
(libtsa_engine.so) the tests and the benchmark drive it with. Struct layouts are declared field for field; a CPU test
checks them against the C compiler's sizeof / offsetof."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import ENGINE_PATH, SsError, check, lib

u32, u64, i32, vp = C.c_uint32, C.c_uint64, C.c_int32, C.c_void_p


class SsBudget(C.Structure):
    _fields_ = [("struct_size", u32), ("device_bytes", u64), ("host_pinned_bytes", u64), ("workspace_bytes", u64),
                ("margin_gib", C.c_double), ("margin_fraction", C.c_double), ("dynamic_slots_per_layer", u32),
                ("ring_slots", u32), ("pinned_backing", C.c_int), ("reserved0", u32), ("tier_mode", C.c_int),
                ("host_spare_units", u32)]


_OPT = [("struct_size", u32), ("backend", C.c_int), ("device", C.c_int), ("policy", C.c_int),
        ("lookahead_budget", u32), ("reader_threads", u32), ("staging_buffers", u32), ("staging_bytes", u64),
        ("copy_piece_bytes", u64), ("verify_hash", C.c_int), ("fill_residents", C.c_int), ("score_window", u32),
        ("pin_planned", C.c_int), ("direct_io", C.c_int), ("group_units", u32), ("spec_persistent", C.c_int),
        ("reserved0", u32), ("readahead_units", u32), ("reserved1", u32), ("forward_mode", C.c_int),
        ("dg_max_ids", u32), ("dg_prefetch_reserve", u32), ("dg_prefetch_per_layer", u32),
        ("dg_prefetch_per_token", u32), ("dg_wait_timeout_ms", u32), ("dg_service_boost", u32), ("dg_diag", u32),
        ("dg_test_hooks", u32), ("dg_spare_target", u32), ("dg_seed_n", u32), ("dg_seed", vp),
        ("dg_spare_slots", u32), ("dg_flush_ready", u32), ("dg_wb_defer", u32), ("dg_wb_stream", u32),
        ("dg_wb_layer_bytes", u32), ("dg_wb_max_outstanding", u32), ("dg_prior_len", u64), ("dg_prior", vp),
        ("exclusive_discard", u32), ("reserved2", u32), ("dg_score_w_trans", u32), ("dg_score_w_freq", u32),
        ("dg_score_w_recency", u32), ("reserved3", u32), ("dg_score_profile_len", u64), ("dg_score_profile", vp),
        ("weight_dirs", vp), ("drive_readers", u32), ("weight_verify", C.c_int), ("dg_disk_tier", u32),
        ("dg_disk_prefetch", u32), ("dg_disk_staging", u32), ("dg_inclusive_blocks", u32), ("dg_disk_queue", u32),
        ("reserved4", u32), ("source_identity_n", u32), ("reserved5", u32), ("source_identities", vp),
        ("budget", vp), ("dg_no_admit", u32), ("reserved6", u32), ("dg_clean_evict", u32), ("reserved7", u32),
        ("dg_pf_revert_unused", u32), ("reserved8", u32), ("dg_pf_strict_admit", u32), ("reserved9", u32),
        ("dg_landing_blocks", u32), ("dg_landing_max_queued", u32), ("dg_landing_ttl", u32), ("reserved10", u32),
        ("dg_landing_chunk", u32), ("reserved11", u32), ("dg_bank_keep", u32), ("reserved12", u32),
        ("dg_disk_queue_adapt", u32), ("reserved13", u32)]


class SsOptions(C.Structure):
    _fields_ = _OPT


class SsGroup(C.Structure):
    _fields_ = [("units", C.POINTER(i32)), ("n_units", C.c_int)]


class SsLayerView(C.Structure):
    _fields_ = [("table_dev", vp), ("table_host", C.POINTER(u64)), ("n_units", C.c_int),
                ("groups", C.POINTER(SsGroup)), ("n_groups", C.c_int)]


STAT_FIELDS = ["routed", "hits", "admitted", "transient", "evicted", "prefetched", "spec_issued", "spec_used",
               "spec_dropped", "bytes_pinned", "bytes_disk", "wait_ns"]


class SsLayerStats(C.Structure):
    _fields_ = [(n, u64) for n in STAT_FIELDS]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n in STAT_FIELDS}


class SsSnapshotInfo(C.Structure):
    _fields_ = [("struct_size", u32), ("flags", u32), ("sequence", u64), ("forwards", u64)] + [
        (n, u64) for n in ("readahead_buffers readahead_buffer_bytes readahead_requested readahead_read "
                           "readahead_landed readahead_unused readahead_failed readahead_fallback readahead_bytes "
                           "exclusive_writebacks exclusive_writeback_bytes exclusive_deferred exclusive_promoted "
                           "exclusive_free_blocks exclusive_min_free_blocks exclusive_rereads exclusive_blocks "
                           "exclusive_discards").split()]


class SsExclusiveStats(C.Structure):
    _fields_ = [("struct_size", u32), ("writebacks", u64), ("writeback_bytes", u64), ("deferred", u64),
                ("promoted", u64), ("free_blocks", u64), ("min_free_blocks", u64), ("rereads", u64),
                ("discards", u64)]


class SsPlanTotals(C.Structure):
    _fields_ = [(n, u64) for n in ["fixed_bytes", "margin_bytes", "resident_bytes", "dynamic_bytes", "ring_bytes",
                                   "peak_device_bytes", "pinned_bytes", "disk_bytes", "n_resident", "n_pinned",
                                   "n_disk"]]


class SsDgUnit(C.Structure):
    _fields_ = [("gated", C.c_int32), ("unit", C.c_int32)]


def dg_seed(units) -> tuple:
    """(array, count) for ss_options.dg_seed / dg_seed_n from (gated layer, unit) pairs; keep the array alive while the
    context opens."""
    arr = (SsDgUnit * max(len(units), 1))(*[SsDgUnit(int(g), int(u)) for g, u in units])
    return arr, len(units)


class SsDgPart(C.Structure):
    _fields_ = [("base", vp), ("stride", u64), ("bytes", u64)]


class SsDgDeviceView(C.Structure):
    _fields_ = [("struct_size", u32), ("protocol", u32), ("n_gated", u32), ("n_parts", u32), ("guard_slot", u32),
                ("slots", u32), ("slot_of", vp), ("unit_base", vp), ("abort", vp), ("parts", SsDgPart * 4),
                ("absent_err", vp)]


DG_STAT_U64 = ("tokens lookups misses covered fetched prefetched prefetch_used pred_invalid resurrected bank_serves "
               "collected_mid evicted evict_short writebacks_done stalled free_slots blocks slots predicted "
               "predicted_true miss_layers device_timeouts covered_waits wb_deferred wb_cancelled wb_forced "
               "wb_boundary_flushed wb_issued_bytes wb_completed_bytes wb_cancelled_bytes wb_boundary_flushed_bytes "
               "wb_outstanding_bytes wb_forced_wait_ns winpf_hints winpf_hint_rows prior_issued prior_used prior_late "
               "prior_reverted l1_candidates l1_issued l1_used l1_late l1_reverted l1_priced_out l1_skipped_ahead "
               "prior_budget_stops score_fallbacks scored_victims score_layers score_candidates score_saturated "
               "score_ns score_deferred score_last_ns disk_reads disk_read_bytes disk_read_ns disk_stage_waits "
               "disk_drops disk_discards inclusive_kept inclusive_drops disk_units backed_units disk_wait_ns "
               "disk_overlapped disk_max_in_flight disk_carried disk_carried_bytes resident_units resident_evicted "
               "resident_bytes resident_ns round_count round_units round_bytes round_ns round_cancelled").split()
DG_STAT_TAIL = [("cuda_module_loading", u32), ("reserved1", u32)] + [(n, u64) for n in (
    "clean_drops clean_drop_bytes mkres_file_reads mkres_file_bytes mkres_read_ns mkres_h2d_bytes mkres_wb_bytes "
    "lm_tokens lm_parts lm_mid_evictions lm_early_admits pf_reverted pf_revert_bytes pred_skipped_ahead "
    "pf_strict_refused pred_shadow_file_predicted pred_shadow_file_demanded pred_shadow_file_hit "
    "pred_shadow_file_predicted_bytes pred_shadow_file_demanded_bytes pred_shadow_file_hit_bytes").split()] + \
    [("disk_queue_resolved", u32), ("disk_locations", u32)] + [(n, u64) for n in (
        "landing_issued landing_promoted landing_late landing_wait_ns landing_expired landing_dropped_full "
        "landing_read_bytes landing_cancelled landing_expired_layer landing_skipped_passed landing_yields "
        "landing_aborted_bytes bank_kept").split()] + \
    [("disk_depth_active", u32), ("disk_depth_adapt", u32), ("disk_depth_changes", u64),
     ("disk_depth_calibrations", u64)]


class TsaTestProfile(C.Structure):
    _fields_ = [(n, u64) for n in ("copies copy_bytes copy_ns writebacks writeback_bytes writeback_ns verifies "
                                   "verify_units verify_bytes verify_ns pending").split()]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


class SsDgStats(C.Structure):
    _fields_ = [("struct_size", u32), ("reserved0", u32)] + [(n, u64) for n in DG_STAT_U64] + DG_STAT_TAIL

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_ if not n.startswith("reserved")}


class SsDgLayerTimeline(C.Structure):
    _fields_ = [("struct_size", u32), ("layer", u32)] + [(n, C.c_double) for n in (
        "seen_us", "demand_us", "pred_wait_us", "prefetch_us", "serve_us")] + [(n, u32) for n in (
            "ids", "misses", "covered", "fetched", "prefetched", "reserved0")] + [("dma_ms", C.c_double)] + \
        [("predicted_true", u32), ("covered_waits", u32)] + [(n, C.c_double) for n in (
            "gpu_wait_us", "gpu_export_ready_us", "wb_left_ms", "dma_first_ms")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_ if not n.startswith("reserved") and n != "struct_size"}


class SsDgBoundaryTimeline(C.Structure):
    _fields_ = [("struct_size", u32), ("writebacks", u32)] + [(n, C.c_double) for n in (
        "sync_us", "select_us", "upload_us", "issue_us")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_ if n != "struct_size"}


_declared = False


def _declare() -> C.CDLL:
    global _declared
    L = lib()
    if _declared:
        return L
    st = C.c_int
    sigs = {
        "ss_desc_from_json": (st, [C.c_char_p, C.c_size_t, C.POINTER(vp)]),
        "ss_desc_from_file": (st, [C.c_char_p, C.POINTER(vp)]),
        "ss_desc_free": (None, [vp]),
        "ss_desc_n_layers": (C.c_int, [vp]),
        "ss_desc_layer_units": (C.c_int, [vp, C.c_int]),
        "ss_desc_unit_bytes": (u64, [vp, C.c_int]),
        "ss_desc_total_units": (C.c_int64, [vp]),
        "ss_desc_to_json": (st, [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]),
        "ss_free": (None, [vp]),
        "ss_budget_defaults_sized": (None, [C.POINTER(SsBudget), u32]),
        "ss_options_defaults_sized": (None, [C.POINTER(SsOptions), u32]),
        "ss_plan_make": (st, [vp, C.POINTER(SsBudget), C.POINTER(C.c_double), C.c_size_t, C.POINTER(vp)]),
        "ss_plan_from_tiers": (st, [vp, C.POINTER(SsBudget), C.POINTER(C.c_uint8), C.c_size_t, C.POINTER(vp)]),
        "ss_plan_free": (None, [vp]),
        "ss_plan_unit_tier": (C.c_int, [vp, C.c_int, C.c_int]),
        "ss_plan_get_totals": (None, [vp, C.POINTER(SsPlanTotals)]),
        "ss_plan_to_json": (st, [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]),
        "ss_open": (st, [vp, C.POINTER(SsBudget), vp, C.POINTER(SsOptions), C.POINTER(vp)]),
        "ss_close": (None, [vp]),
        "ss_begin": (st, [vp, vp, C.c_int]),
        "ss_layer_routes": (st, [vp, C.c_int, C.POINTER(i32), C.c_int]),
        "ss_layer_all": (st, [vp, C.c_int]),
        "ss_acquire": (st, [vp, C.c_int, vp, C.POINTER(SsLayerView)]),
        "ss_acquire_groups": (st, [vp, C.c_int, vp, C.POINTER(SsLayerView)]),
        "ss_group_wait": (st, [vp, C.c_int, C.c_int, vp]),
        "ss_release": (st, [vp, C.c_int, vp]),
        "ss_end": (st, [vp]),
        "ss_check_unit": (st, [vp, C.c_int, C.c_int]),
        "ss_stats_layer": (st, [vp, C.c_int, C.POINTER(SsLayerStats)]),
        "ss_stats_total": (st, [vp, C.POINTER(SsLayerStats)]),
        "ss_stats_exclusive_sized": (st, [vp, C.POINTER(SsExclusiveStats), u32]),
        "ss_stats_to_json": (st, [vp, C.POINTER(vp), C.POINTER(C.c_size_t)]),
        "ss_stats_snapshot_sized": (st, [vp, C.POINTER(SsLayerStats), C.POINTER(SsSnapshotInfo), u32]),
        "ss_stats_snapshot_json": (st, [vp, C.POINTER(vp), C.POINTER(C.c_size_t)]),
        "ss_stats_reset": (None, [vp]),
        "ss_stats_dg_sized": (st, [vp, C.POINTER(SsDgStats), u32]),
        "ss_dg_timeline_sized": (st, [vp, C.c_int, C.POINTER(SsDgLayerTimeline), u32]),
        "ss_dg_boundary_timeline_sized": (st, [vp, C.POINTER(SsDgBoundaryTimeline), u32]),
        "ss_dg_set_policy": (st, [vp, C.c_int]),
        "ss_dg_end_rows": (st, [vp, u32]),
        "ss_dg_keep": (st, [vp, C.c_int, C.POINTER(i32), C.c_int]),
        "ss_dg_set_sched": (st, [vp, u32, u32]),
        "ss_dg_set_budgets": (st, [vp, u32, u32, u32]),
        "ss_host_prefetch": (st, [vp, C.c_int, C.POINTER(i32), C.c_int]),
        "ss_host_prefetch_layer": (st, [vp, C.c_int]),
        "tsa_test_sha256": (st, [C.c_char_p, u64, C.c_char_p]),
        "tsa_test_score_profile_check": (st, [C.c_char_p, u64, C.POINTER(u32), u32, C.c_char_p, C.c_char_p, u32]),
        "ss_dg_get_device_view_sized": (st, [vp, C.POINTER(SsDgDeviceView), u32]),
        "ss_dg_gated_index": (C.c_int, [vp, C.c_int]),
        "ss_dg_residency": (st, [vp, vp, u32, C.POINTER(u32)]),
        "ss_dg_set_clean_evict": (st, [vp, u32]),
        "ss_source_direct": (C.c_int, [vp, C.c_int]),
        "ss_test_dg_check": (st, [vp]),
        "ss_test_dg_stop_service": (st, [vp]),
        "tsa_test_region_of": (st, [vp, u64, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(u64)]),
        "tsa_test_dg_table": (st, [vp, C.POINTER(i32), u32, C.POINTER(u32)]),
        "tsa_test_verify_failures": (u64, [vp]),
        "tsa_test_dg_hsa_copies": (C.c_int, [vp]),
        "tsa_test_host_copies": (st, [vp, C.POINTER(u64), C.POINTER(u64)]),
        "tsa_test_host_waits": (st, [vp, C.POINTER(u64), C.POINTER(u64)]),
        "tsa_test_stream_order": (st, [u32, u32, u32, C.c_int, C.POINTER(u64)]),
        "tsa_test_profile_enable": (st, [vp, C.c_int]),
        "tsa_test_profile_read": (st, [vp, C.c_int, C.POINTER(TsaTestProfile)]),
        "tsa_test_dg_stamps": (st, [vp, C.POINTER(u64), u32, C.POINTER(u32)]),
        "tsa_test_dg_corrupt_block": (st, [vp, C.c_int, C.c_int, u64]),
        "tsa_xxh64_host": (u64, [vp, u64]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _declared = True
    return L


_engine = None


def engine() -> C.CDLL:
    global _engine
    if _engine is None:
        if not ENGINE_PATH.exists():
            raise RuntimeError(f"{ENGINE_PATH} is not built: run python -m tierstream_amd.build")
        _declare()
        _engine = C.CDLL(str(ENGINE_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        E = _engine
        E.tse_host_run.restype = C.c_int
        E.tse_host_run.argtypes = [vp, vp, C.c_int, C.POINTER(i32), C.c_int, C.c_int, C.c_int, C.POINTER(u64),
                                   C.POINTER(u64), C.POINTER(SsLayerStats), C.POINTER(C.c_double)]
        E.tse_host_run_ex.restype = C.c_int
        E.tse_host_run_ex.argtypes = [vp, vp, C.c_int, C.POINTER(i32), C.POINTER(i32), C.c_int, C.c_int, C.c_int,
                                      C.c_int, C.POINTER(u64), C.POINTER(u64), C.POINTER(SsLayerStats),
                                      C.POINTER(C.c_double)]
        E.tse_dg_create.restype = C.c_int
        E.tse_dg_create.argtypes = [vp, u32, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]
        E.tse_dg_token.restype = C.c_int
        E.tse_dg_token.argtypes = [vp, C.POINTER(i32), C.POINTER(u64), C.POINTER(C.c_double)]
        E.tse_dg_create_pred.restype = C.c_int
        E.tse_dg_create_pred.argtypes = [vp, u32, u32, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]
        E.tse_dg_token_pred.restype = C.c_int
        E.tse_dg_token_pred.argtypes = [vp, C.POINTER(i32), C.POINTER(i32), C.POINTER(u64), C.POINTER(C.c_double)]
        E.tse_dg_create_ex.restype = C.c_int
        E.tse_dg_create_ex.argtypes = [vp, u32, u32, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]
        E.tse_dg_token_open.restype = C.c_int
        E.tse_dg_token_open.argtypes = [vp, C.POINTER(i32)]
        E.tse_dg_early.restype = C.c_int
        E.tse_dg_early.argtypes = [vp, C.POINTER(u64), C.POINTER(u32)]
        E.tse_dg_stamps.restype = C.c_int
        E.tse_dg_stamps.argtypes = [vp, C.POINTER(u64)]
        E.tse_dg_set_rows.restype = C.c_int
        E.tse_dg_set_rows.argtypes = [vp, u32]
        E.tse_dg_destroy.restype = None
        E.tse_dg_destroy.argtypes = [vp]
    return _engine


def budget(device_bytes: int, host_pinned_bytes: int, **kw) -> SsBudget:
    L = _declare()
    b = SsBudget()
    L.ss_budget_defaults_sized(C.byref(b), C.sizeof(b))
    b.device_bytes = device_bytes
    b.host_pinned_bytes = host_pinned_bytes
    b.margin_gib = 0.0
    b.margin_fraction = 0.0
    for k, v in kw.items():
        setattr(b, k, v)
    return b


def options(**kw) -> SsOptions:
    L = _declare()
    o = SsOptions()
    L.ss_options_defaults_sized(C.byref(o), C.sizeof(o))
    for k, v in kw.items():
        setattr(o, k, v)
    return o


class Desc:
    def __init__(self, json_text: str):
        L = _declare()
        self.h = vp()
        b = json_text.encode()
        check(L.ss_desc_from_json(b, len(b), C.byref(self.h)))
        self.n_layers = L.ss_desc_n_layers(self.h)

    def json(self) -> dict:
        """The canonical descriptor JSON (ss_desc_to_json)."""
        import json as _json
        L = _declare()
        s, n = C.c_char_p(), C.c_size_t()
        check(L.ss_desc_to_json(self.h, C.byref(s), C.byref(n)))
        out = _json.loads(C.string_at(s, n.value).decode())
        L.ss_free(s)
        return out

    def units(self, layer):
        return _declare().ss_desc_layer_units(self.h, layer)

    def unit_bytes(self, layer):
        return int(_declare().ss_desc_unit_bytes(self.h, layer))

    def close(self):
        if self.h:
            _declare().ss_desc_free(self.h)
            self.h = None


class Plan:
    def __init__(self, desc: Desc, b: SsBudget, benefit=None, tiers=None):
        """ss_plan_make, or with `tiers` (one SS_TIER_* per unit in descriptor order) ss_plan_from_tiers."""
        L = _declare()
        self.h = vp()
        if tiers is not None:
            t = (C.c_uint8 * len(tiers))(*tiers)
            check(L.ss_plan_from_tiers(desc.h, C.byref(b), t, len(tiers), C.byref(self.h)))
        else:
            ben = (C.c_double * len(benefit))(*benefit) if benefit is not None else None
            check(L.ss_plan_make(desc.h, C.byref(b), ben, len(benefit) if benefit is not None else 0,
                                 C.byref(self.h)))
        self.desc = desc

    def tiers(self):
        L = _declare()
        return [[L.ss_plan_unit_tier(self.h, l, u) for u in range(self.desc.units(l))]
                for l in range(self.desc.n_layers)]

    def totals(self) -> SsPlanTotals:
        t = SsPlanTotals()
        _declare().ss_plan_get_totals(self.h, C.byref(t))
        return t

    def json(self) -> dict:
        import json as _json
        L = _declare()
        s, n = C.c_char_p(), C.c_size_t()
        check(L.ss_plan_to_json(self.h, C.byref(s), C.byref(n)))
        out = _json.loads(C.string_at(s, n.value).decode())
        L.ss_free(s)
        return out

    def close(self):
        if self.h:
            _declare().ss_plan_free(self.h)
            self.h = None


class Ctx:
    def __init__(self, desc: Desc, b: SsBudget, plan: Plan | None, o: SsOptions):
        L = _declare()
        self.h = vp()
        self.desc = desc
        check(L.ss_open(desc.h, C.byref(b), plan.h if plan else None, C.byref(o), C.byref(self.h)))

    def close(self):
        if self.h:
            _declare().ss_close(self.h)
            self.h = None

    def stats_total(self) -> dict:
        s = SsLayerStats()
        check(_declare().ss_stats_total(self.h, C.byref(s)))
        return s.as_dict()

    def stats_layer(self, layer) -> dict:
        s = SsLayerStats()
        check(_declare().ss_stats_layer(self.h, layer, C.byref(s)))
        return s.as_dict()

    def _text(self, fn) -> str:
        L = _declare()
        p, n = vp(), C.c_size_t()
        check(fn(self.h, C.byref(p), C.byref(n)))
        try:
            return C.string_at(p, n.value).decode()
        finally:
            L.ss_free(p)

    def stats_json(self) -> str:
        """ss_stats_to_json: the stats-v1 document of the counters now."""
        return self._text(_declare().ss_stats_to_json)

    def snapshot(self):
        """ss_stats_snapshot: (total dict, info dict); raises SsError (SS_E_INVALID) until something is published."""
        t, i = SsLayerStats(), SsSnapshotInfo()
        check(_declare().ss_stats_snapshot_sized(self.h, C.byref(t), C.byref(i), C.sizeof(i)))
        return t.as_dict(), {n: int(getattr(i, n)) for n, _ in i._fields_}

    def snapshot_json(self) -> str:
        return self._text(_declare().ss_stats_snapshot_json)

    def stats_reset(self):
        _declare().ss_stats_reset(self.h)

    def exclusive_stats(self) -> dict:
        x = SsExclusiveStats()
        check(_declare().ss_stats_exclusive_sized(self.h, C.byref(x), C.sizeof(x)))
        return {n: int(getattr(x, n)) for n, _ in x._fields_ if n != "struct_size"}

    def dg_stats(self) -> dict:
        s = SsDgStats()
        check(_declare().ss_stats_dg_sized(self.h, C.byref(s), C.sizeof(s)))
        return s.as_dict()

    def dg_timeline(self, g: int) -> dict:
        """dg_diag = 1, between tokens: gated layer g's row of the last completed token (ss_dg_timeline_sized)."""
        t = SsDgLayerTimeline()
        check(_declare().ss_dg_timeline_sized(self.h, g, C.byref(t), C.sizeof(t)))
        return t.as_dict()

    def dg_boundary_timeline(self) -> dict:
        """dg_diag = 1, between tokens: the last boundary's phases (ss_dg_boundary_timeline_sized)."""
        t = SsDgBoundaryTimeline()
        check(_declare().ss_dg_boundary_timeline_sized(self.h, C.byref(t), C.sizeof(t)))
        return t.as_dict()

    def dg_set_policy(self, policy: int):
        """Between tokens: 0 LRU, 1 SCORED, 2 SCORED_AUTO (ss_dg_set_policy)."""
        check(_declare().ss_dg_set_policy(self.h, policy))

    def dg_keep(self, g: int, ids):
        """Between tokens: the units of gated layer g no later boundary may evict (ss_dg_keep; empty releases)."""
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        check(_declare().ss_dg_keep(self.h, g, a.ctypes.data_as(C.POINTER(i32)) if len(a) else None, len(a)))

    def dg_set_sched(self, wb_defer: int, flush_ready: int = 0):
        """Between tokens: write-back deferral and dg_flush_ready (ss_dg_set_sched)."""
        check(_declare().ss_dg_set_sched(self.h, wb_defer, flush_ready))

    def dg_set_clean_evict(self, on: int):
        """Between tokens: dg_clean_evict on / off (ss_dg_set_clean_evict)."""
        check(_declare().ss_dg_set_clean_evict(self.h, on))

    def dg_set_budgets(self, spare_target: int, per_layer: int, per_token: int):
        """Between tokens: the spare target and the prefetch budgets (ss_dg_set_budgets)."""
        check(_declare().ss_dg_set_budgets(self.h, spare_target, per_layer, per_token))

    def dg_gated_index(self, layer: int) -> int:
        """The gated ordinal of a descriptor layer, -1 for a layer without units or out of range."""
        return int(_declare().ss_dg_gated_index(self.h, layer))

    def dg_residency(self) -> list[tuple[int, int]]:
        """Between tokens: the units on the device, most recently used first, as (gated layer, unit)."""
        L = _declare()
        n = u32(0)
        check(L.ss_dg_residency(self.h, None, 0, C.byref(n)))
        arr = (SsDgUnit * max(n.value, 1))()
        check(L.ss_dg_residency(self.h, C.cast(arr, vp), n.value, C.byref(n)))
        return [(int(arr[i].gated), int(arr[i].unit)) for i in range(n.value)]

    def source_direct(self, source: int = 0) -> int:
        """1: the source is read with O_DIRECT; 0: buffered (its file system refused O_DIRECT); < 0: an error."""
        return int(_declare().ss_source_direct(self.h, source))

    def test_dg_check(self) -> int:
        """ss_test_dg_check: the status (no raise)."""
        return int(_declare().ss_test_dg_check(self.h))

    def test_dg_stop_service(self) -> int:
        return int(_declare().ss_test_dg_stop_service(self.h))

    def host_prefetch(self, layer: int, ids) -> int:
        """ss_host_prefetch; returns the status (no raise)."""
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        return int(_declare().ss_host_prefetch(self.h, layer, a.ctypes.data_as(C.POINTER(i32)) if len(a) else None,
                                               len(a)))

    def dg_table(self) -> np.ndarray:
        L = _declare()
        n = u32(0)
        check(L.tsa_test_dg_table(self.h, None, 0, C.byref(n)))
        out = np.zeros(max(n.value, 1), dtype=np.int32)
        check(L.tsa_test_dg_table(self.h, out.ctypes.data_as(C.POINTER(i32)), n.value, C.byref(n)))
        return out[:n.value]

    def dg_view(self) -> SsDgDeviceView:
        v = SsDgDeviceView()
        check(_declare().ss_dg_get_device_view_sized(self.h, C.byref(v), C.sizeof(v)))
        return v

    def verify_failures(self) -> int:
        return int(_declare().tsa_test_verify_failures(self.h))

    def hsa_copies(self) -> bool:
        """Device-gated: whether unit copies go through the HSA runtime's copy engines (else HIP streams)."""
        return bool(_declare().tsa_test_dg_hsa_copies(self.h))

    def host_copies(self) -> tuple[int, int]:
        """Host contract: (unit copies from pinned blocks since open, the copies they were issued as)."""
        units, copies = u64(), u64()
        check(_declare().tsa_test_host_copies(self.h, C.byref(units), C.byref(copies)))
        return int(units.value), int(copies.value)

    def host_waits(self) -> tuple[int, int]:
        """Host contract: (cross-stream waits given to the runtime since open, waits skipped as implied)."""
        issued, skipped = u64(), u64()
        check(_declare().tsa_test_host_waits(self.h, C.byref(issued), C.byref(skipped)))
        return int(issued.value), int(skipped.value)

    PROF_COPY, PROF_WRITEBACK, PROF_VERIFY = 0x2, 0x4, 0x8

    def profile_enable(self, on=True):
        """on: True / False (every kind / none), or a mask of PROF_COPY | PROF_WRITEBACK | PROF_VERIFY."""
        check(_declare().tsa_test_profile_enable(self.h, int(on)))

    def profile_read(self, wait: bool = True) -> dict:
        p = TsaTestProfile()
        check(_declare().tsa_test_profile_read(self.h, int(wait), C.byref(p)))
        return p.as_dict()

    def dg_stamps(self) -> np.ndarray:
        """uint64 [G][4] wall-clock ticks of the last token: export end, wait entry, ready seen (0: the layer had no
        miss), wait exit."""
        L = _declare()
        n = u32(0)
        check(L.tsa_test_dg_stamps(self.h, None, 0, C.byref(n)))
        out = np.zeros(n.value, dtype=np.uint64)
        check(L.tsa_test_dg_stamps(self.h, out.ctypes.data_as(C.POINTER(u64)), n.value, C.byref(n)))
        return out.reshape(-1, 4)

    def dg_corrupt_block(self, gated: int, unit: int, offset: int = 0):
        """Flip one byte of a unit's pinned copy (the unit must be off the device): its next landing fails the device
        check."""
        check(_declare().tsa_test_dg_corrupt_block(self.h, gated, unit, offset))

    def region_of(self, addr: int):
        k, i, off = C.c_int(), C.c_int(), u64()
        check(_declare().tsa_test_region_of(self.h, addr, C.byref(k), C.byref(i), C.byref(off)))
        return k.value, i.value, int(off.value)

    # ---- engine drivers ----
    def host_run(self, routes: np.ndarray, mode: int = 0, want_tables=True, host_lookahead: int = 0,
                 prefetch: np.ndarray | None = None):
        """routes int32 [steps][layers][max_ids]; host_lookahead H: ss_host_prefetch_layer of the next H layers after
        each layer's routes; prefetch (routes' shape): after layer l's acquire, ss_prefetch of layer l + 1 with its
        row, CERTAIN on even steps and SPECULATIVE on odd ones; returns checksums, tables, per-step stats, step ms."""
        E = engine()
        steps, L, max_ids = routes.shape
        max_units = max(self.desc.units(l) for l in range(L))
        r = np.ascontiguousarray(routes, dtype=np.int32)
        q = None
        if prefetch is not None:
            q = np.ascontiguousarray(prefetch, dtype=np.int32)
            assert q.shape == r.shape
        cks = np.zeros((steps, L, max_ids), dtype=np.uint64)
        tabs = np.zeros((steps, L, max_units), dtype=np.uint64) if want_tables else None
        stats = (SsLayerStats * steps)()
        ms = np.zeros(steps, dtype=np.float64)
        st = E.tse_host_run_ex(self.h, self.desc.h, steps, r.ctypes.data_as(C.POINTER(i32)),
                               q.ctypes.data_as(C.POINTER(i32)) if q is not None else None, max_ids, max_units,
                               mode, host_lookahead, cks.ctypes.data_as(C.POINTER(u64)),
                               tabs.ctypes.data_as(C.POINTER(u64)) if want_tables else None, stats,
                               ms.ctypes.data_as(C.POINTER(C.c_double)))
        check(st)
        return cks, tabs, [s.as_dict() for s in stats], ms


class DgEngine:
    """A graph-captured device-gated engine over a context (tse_dg_*)."""

    def __init__(self, ctx: Ctx, n_ids: int, use_graph=True, checksum=True, gated=True, n_pred=0, early=False):
        """n_pred: ids predicted at every gated layer but the last for the next one (ss_dg_enqueue_predict).
        early: resident-first reads through ss_dg_slot_if_ready before every layer's wait (early())."""
        E = engine()
        self.h = vp()
        self.G = ctx.dg_view().n_gated
        self.n_ids = n_ids
        self.n_pred = n_pred
        check(E.tse_dg_create_ex(ctx.h, n_ids, n_pred, int(use_graph), int(checksum), int(gated), int(early),
                                 C.byref(self.h)))

    def token(self, routes: np.ndarray, want_checksums=True, preds=None):
        """routes int32 [G][n_ids]; preds int32 [G][n_pred] (row g for layer g + 1); returns (checksums [G][n_ids]
        or None, ms)."""
        st, cks, ms = self.token_status(routes, want_checksums, preds)
        check(st)
        return cks, ms

    def token_status(self, routes: np.ndarray, want_checksums=True, preds=None):
        """As token(), without raising: (status, checksums, ms); a failed token's checksums are still read back."""
        E = engine()
        r = np.ascontiguousarray(routes, dtype=np.int32)
        assert r.shape == (self.G, self.n_ids)
        p = None
        if preds is not None:
            p = np.ascontiguousarray(preds, dtype=np.int32)
            assert p.shape == (self.G, self.n_pred)
        cks = np.zeros((self.G, self.n_ids), dtype=np.uint64) if want_checksums else None
        ms = C.c_double(0)
        st = E.tse_dg_token_pred(self.h, r.ctypes.data_as(C.POINTER(i32)),
                                 p.ctypes.data_as(C.POINTER(i32)) if p is not None else None,
                                 cks.ctypes.data_as(C.POINTER(u64)) if want_checksums else None, C.byref(ms))
        return int(st), cks, ms.value

    def token_open(self, routes: np.ndarray):
        """ss_begin and the token's kernels enqueued, without ss_end: the token stays open (a failing engine)."""
        r = np.ascontiguousarray(routes, dtype=np.int32)
        assert r.shape == (self.G, self.n_ids)
        check(engine().tse_dg_token_open(self.h, r.ctypes.data_as(C.POINTER(i32))))

    def set_rows(self, rows: int):
        """The verify rows each later token closes (ss_dg_end_rows above one)."""
        check(engine().tse_dg_set_rows(self.h, rows))

    def early(self):
        """The last token's resident-first reads: (checksums uint64 [G][n_ids], ready uint32 [G][n_ids])."""
        sums = np.zeros((self.G, self.n_ids), dtype=np.uint64)
        ready = np.zeros((self.G, self.n_ids), dtype=np.uint32)
        check(engine().tse_dg_early(self.h, sums.ctypes.data_as(C.POINTER(u64)), ready.ctypes.data_as(C.POINTER(u32))))
        return sums, ready

    def stamps(self) -> np.ndarray:
        """uint64 [G]: the last token's per-layer compute-start wall-clock ticks."""
        out = np.zeros(self.G, dtype=np.uint64)
        check(engine().tse_dg_stamps(self.h, out.ctypes.data_as(C.POINTER(u64))))
        return out

    def close(self):
        if self.h:
            engine().tse_dg_destroy(self.h)
            self.h = None


__all__ = ["SsBudget", "SsOptions", "SsLayerStats", "SsDgStats", "Desc", "Plan", "Ctx", "DgEngine", "budget",
           "options", "SsError", "TsaTestProfile"]
