/*
 * strix-stream C ABI (v1), served by the MI355X build of tierstream (libtierstream_amd).
 *
 * This header declares the serve-path subset of the strix-stream ABI with the same names, argument meanings, enum
 * values and struct layouts as reference include/strix_stream/ss.h, so an engine built against that header links this
 * library unchanged for these calls. Functions of the reference ABI that are not on the serve path (recipes, device
 * profiles, budgets, packs, multi-location files, placement rounds, window prefetch) are not declared here.
 *
 * Threading: one engine thread drives a context (every call on it from one thread, or serialized by the caller). The
 * library owns its file reader threads (host contract) and one service thread (device-gated contract).
 *
 * Streams: a stream argument is a hipStream_t passed as void*. One engine stream per forward. A ss_layer_view is valid
 * from ss_acquire* of a layer until ss_release of that layer.
 *
 * Versioned structs (ss_budget, ss_options, ss_exclusive_stats, ss_dg_device_view, ss_dg_stats) start with
 * struct_size: a reader takes min(struct_size, its own sizeof) bytes and defaults the rest; an output struct gets
 * min(struct_size, sizeof) bytes written.
 *
 * Failures: SS_E_INVALID / SS_E_IO / SS_E_HASH / SS_E_CAPACITY leave the context usable. SS_E_BACKEND / SS_E_NOMEM
 * inside a context call poison it: every later call except ss_close and the stats calls fails.
 *
 * Exactness: bytes are never changed. A unit's device bytes are identical whether resident, landed from the pinned
 * tier or read from a file; placement is visible to the engine only through the tables.
 *
 * Backend: SS_BACKEND_HIP is a discrete AMD Instinct GPU (gfx950): slots in HBM, a hipHostMalloc pinned tier, copies on
 * dedicated SDMA streams. SS_BACKEND_CPU and SS_BACKEND_CUDA are refused with SS_E_UNSUPPORTED by this library.
 */
#ifndef STRIX_STREAM_SS_H
#define STRIX_STREAM_SS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define SS_API __attribute__((visibility("default")))
#else
#define SS_API
#endif

#define SS_ABI_VERSION 1

typedef enum ss_status {
  SS_OK = 0,
  SS_E_INVALID = 1,     /* bad argument or call order */
  SS_E_DESC = 2,        /* descriptor parse / validation error */
  SS_E_IO = 3,          /* file open / read error */
  SS_E_NOMEM = 4,       /* device or host allocation failed */
  SS_E_BACKEND = 5,     /* HIP runtime error */
  SS_E_CAPACITY = 6,    /* plan or ring cannot hold what a layer needs */
  SS_E_HASH = 7,        /* landed bytes differ from the descriptor hash */
  SS_E_UNSUPPORTED = 8, /* backend or feature not in this library */
  SS_E_RECIPE = 9       /* (reference recipes; never returned here) */
} ss_status;

/* The calling thread's last error message (valid until its next failing call). */
SS_API const char* ss_last_error(void);
SS_API int ss_abi_version(void);

/* ---- descriptor: strix-stream/desc-v1 JSON ---------------------------------------------------------------------- */
typedef struct ss_desc ss_desc;

SS_API ss_status ss_desc_from_json(const char* json_text, size_t len, ss_desc** out);
SS_API ss_status ss_desc_from_file(const char* path, ss_desc** out);
SS_API ss_status ss_desc_from_model(const char* manifest_path, ss_desc** out);
SS_API void ss_desc_free(ss_desc* d);
SS_API int ss_desc_n_layers(const ss_desc* d);
SS_API int ss_desc_layer_units(const ss_desc* d, int layer);
SS_API uint64_t ss_desc_unit_bytes(const ss_desc* d, int layer);
/* Canonical JSON (sorted keys, no whitespace). Freed with ss_free. */
SS_API ss_status ss_desc_to_json(const ss_desc* d, char** out_json, size_t* out_len);
SS_API void ss_free(void* p);

/* ---- planner ---------------------------------------------------------------------------------------------------- */
typedef enum ss_tier {
  SS_TIER_RESIDENT = 0,
  SS_TIER_PINNED = 1,
  SS_TIER_DISK = 2,
  SS_TIER_PAIR = 3,
  SS_TIER_RESIDENT_BACKED = 4
} ss_tier;

typedef enum ss_tier_mode {
  SS_TIER_MODE_INCLUSIVE = 0,
  SS_TIER_MODE_EXCLUSIVE = 1
} ss_tier_mode;

typedef struct ss_budget {
  uint32_t struct_size;
  uint64_t device_bytes;       /* the device cap */
  uint64_t host_pinned_bytes;  /* pinned host the library may lock */
  uint64_t workspace_bytes;
  double margin_gib;           /* default 2.0 */
  double margin_fraction;      /* default 0.03 */
  uint32_t dynamic_slots_per_layer;
  uint32_t ring_slots;
  int pinned_backing;
  uint32_t reserved0;          /* never read */
  int tier_mode;               /* ss_tier_mode */
  uint32_t host_spare_units;   /* EXCLUSIVE: spare blocks per unit size, 0 = min(64, units of that size) */
} ss_budget;

typedef struct ss_plan ss_plan;

SS_API void ss_budget_defaults_sized(ss_budget* b, uint32_t size);
static inline void ss_budget_defaults(ss_budget* b) { ss_budget_defaults_sized(b, (uint32_t)sizeof *b); }
SS_API ss_status ss_plan_make(const ss_desc* d, const ss_budget* b, const double* benefit, size_t n_benefit,
                              ss_plan** out);
SS_API ss_status ss_plan_from_tiers(const ss_desc* d, const ss_budget* b, const uint8_t* tiers, size_t n,
                                    ss_plan** out);
SS_API ss_status ss_plan_from_json(const ss_desc* d, const ss_budget* b, const char* plan_json, size_t len,
                                   ss_plan** out);
SS_API void ss_plan_free(ss_plan* p);
SS_API ss_tier ss_plan_unit_tier(const ss_plan* p, int layer, int unit);
typedef struct ss_plan_totals {
  uint64_t fixed_bytes, margin_bytes, resident_bytes, dynamic_bytes, ring_bytes, peak_device_bytes;
  uint64_t pinned_bytes, disk_bytes;
  uint64_t n_resident, n_pinned, n_disk;
} ss_plan_totals;
SS_API void ss_plan_get_totals(const ss_plan* p, ss_plan_totals* out);
SS_API ss_status ss_plan_to_json(const ss_plan* p, char** out_json, size_t* out_len);
SS_API int64_t ss_desc_unit_index(const ss_desc* d, int layer, int unit);
SS_API int64_t ss_desc_total_units(const ss_desc* d);

/* ---- context ---------------------------------------------------------------------------------------------------- */
typedef enum ss_backend_kind {
  SS_BACKEND_CPU = 0,
  SS_BACKEND_CUDA = 1,
  SS_BACKEND_HIP = 2   /* this library: a discrete AMD Instinct GPU */
} ss_backend_kind;

typedef enum ss_policy {
  SS_POLICY_LRU = 0,
  SS_POLICY_SCORED = 1,
  SS_POLICY_SCORED_AUTO = 2
} ss_policy;

struct ss_dg_unit;
typedef struct ss_file_identity {
  uint64_t volume;
  uint64_t index;
  uint64_t size;
} ss_file_identity;
struct ss_budget_ledger;

/* Field for field the reference layout (padding words included); fields this library does not act on are read and
 * validated where the serve path needs them, otherwise ignored. */
typedef struct ss_options {
  uint32_t struct_size;
  ss_backend_kind backend;
  int device;
  ss_policy policy;
  uint32_t lookahead_budget;
  uint32_t reader_threads;
  uint32_t staging_buffers;
  uint64_t staging_bytes;
  uint64_t copy_piece_bytes;
  int verify_hash;
  int fill_residents;
  uint32_t score_window;
  int pin_planned;
  int direct_io;
  uint32_t group_units;
  int spec_persistent;
  uint32_t reserved0;
  uint32_t readahead_units;
  uint32_t reserved1;
  int forward_mode;               /* ss_forward_mode */
  uint32_t dg_max_ids;
  uint32_t dg_prefetch_reserve;
  uint32_t dg_prefetch_per_layer;
  uint32_t dg_prefetch_per_token;
  uint32_t dg_wait_timeout_ms;
  uint32_t dg_service_boost;
  uint32_t dg_diag;
  uint32_t dg_test_hooks;
  uint32_t dg_spare_target;
  uint32_t dg_seed_n;
  const struct ss_dg_unit* dg_seed;
  uint32_t dg_spare_slots;
  uint32_t dg_flush_ready;
  uint32_t dg_wb_defer;
  uint32_t dg_wb_stream;
  uint32_t dg_wb_layer_bytes;
  uint32_t dg_wb_max_outstanding;
  uint64_t dg_prior_len;
  const void* dg_prior;
  uint32_t exclusive_discard;
  uint32_t reserved2;
  uint32_t dg_score_w_trans, dg_score_w_freq, dg_score_w_recency;
  uint32_t reserved3;
  uint64_t dg_score_profile_len;
  const void* dg_score_profile;
  const char* weight_dirs;
  uint32_t drive_readers;
  int weight_verify;
  uint32_t dg_disk_tier;
  uint32_t dg_disk_prefetch;
  uint32_t dg_disk_staging;
  uint32_t dg_inclusive_blocks;
  uint32_t dg_disk_queue;
  uint32_t reserved4;
  uint32_t source_identity_n;
  uint32_t reserved5;
  const ss_file_identity* source_identities;
  struct ss_budget_ledger* budget;
  uint32_t dg_no_admit;
  uint32_t reserved6;
  uint32_t dg_clean_evict;
  uint32_t reserved7;
  uint32_t dg_pf_revert_unused;
  uint32_t reserved8;
  uint32_t dg_pf_strict_admit;
  uint32_t reserved9;
  uint32_t dg_landing_blocks;
  uint32_t dg_landing_max_queued;
  uint32_t dg_landing_ttl;
  uint32_t reserved10;
  uint32_t dg_landing_chunk;
  uint32_t reserved11;
  uint32_t dg_bank_keep;
  uint32_t reserved12;
  uint32_t dg_disk_queue_adapt;
  uint32_t reserved13;
} ss_options;

typedef enum ss_forward_mode { SS_FORWARD_HOST = 0, SS_FORWARD_DEVICE_GATED = 1 } ss_forward_mode;

typedef struct ss_ctx ss_ctx;

SS_API void ss_options_defaults_sized(ss_options* o, uint32_t size);
static inline void ss_options_defaults(ss_options* o) { ss_options_defaults_sized(o, (uint32_t)sizeof *o); }
/* plan may be NULL (made from the budget); a given plan must have been made with this budget. */
SS_API ss_status ss_open(const ss_desc* d, const ss_budget* budget, const ss_plan* plan, const ss_options* opt,
                         ss_ctx** out);
SS_API void ss_close(ss_ctx* c);
SS_API int ss_source_direct(const ss_ctx* c, int source);
SS_API ss_status ss_seed(ss_ctx* c, int layer, const int32_t* units, int n);

/* ---- one forward (host contract) -------------------------------------------------------------------------------- */
SS_API ss_status ss_begin(ss_ctx* c, const uint32_t* rows_per_layer, int n_layers);
SS_API ss_status ss_layer_routes(ss_ctx* c, int layer, const int32_t* ids, int n);
SS_API ss_status ss_layer_routes_dev(ss_ctx* c, int layer, const int32_t* ids_dev, int n, void* engine_stream);
SS_API ss_status ss_layer_all(ss_ctx* c, int layer);

typedef enum ss_prefetch_kind {
  SS_PREFETCH_CERTAIN = 0,
  SS_PREFETCH_SPECULATIVE = 1
} ss_prefetch_kind;
SS_API ss_status ss_prefetch(ss_ctx* c, int layer, const int32_t* ids, int n, ss_prefetch_kind kind);
SS_API ss_status ss_prefetch_layer(ss_ctx* c, int layer);
/* Host-only read-ahead of file-backed units into host buffers, no device slot (reference ss.h:489-494,
 * src/stream_ctx.cpp:1441-1449, src/capi.cpp:698-710). A no-op while readahead_units is 0; arguments are checked. */
SS_API ss_status ss_host_prefetch(ss_ctx* c, int layer, const int32_t* ids, int n);
SS_API ss_status ss_host_prefetch_layer(ss_ctx* c, int layer);
/* Lookahead helper (reference ss.h:496-499, src/capi.cpp:577-612): rows x n_experts router scores of the next layer;
 * per row its top_k (score descending, lower id first), the union ordered by (best rank, best score at that rank,
 * id); up to max_out ids into out, the count into *n_out. */
SS_API ss_status ss_lookahead_select(const float* scores, int rows, int n_experts, int top_k, int32_t* out,
                                     int max_out, int* n_out);

typedef struct ss_group {
  const int32_t* units;
  int n_units;
} ss_group;
typedef struct ss_layer_view {
  const uint64_t* table_dev;   /* device array of n_units addresses (0 = absent this forward) */
  const uint64_t* table_host;  /* host copy */
  int n_units;
  const ss_group* groups;
  int n_groups;
} ss_layer_view;

SS_API ss_status ss_acquire(ss_ctx* c, int layer, void* engine_stream, ss_layer_view* out);
SS_API ss_status ss_acquire_groups(ss_ctx* c, int layer, void* engine_stream, ss_layer_view* out);
SS_API ss_status ss_group_wait(ss_ctx* c, int layer, int group, void* engine_stream);
SS_API ss_status ss_release(ss_ctx* c, int layer, void* engine_stream);
SS_API ss_status ss_end(ss_ctx* c);
SS_API ss_status ss_check_unit(ss_ctx* c, int layer, int unit);

/* ---- stats ------------------------------------------------------------------------------------------------------- */
typedef struct ss_layer_stats {
  uint64_t routed;
  uint64_t hits;
  uint64_t admitted;
  uint64_t transient;
  uint64_t evicted;
  uint64_t prefetched;
  uint64_t spec_issued, spec_used, spec_dropped;
  uint64_t bytes_pinned;
  uint64_t bytes_disk;
  uint64_t wait_ns;
} ss_layer_stats;

SS_API ss_status ss_stats_layer(const ss_ctx* c, int layer, ss_layer_stats* out);
SS_API ss_status ss_stats_total(const ss_ctx* c, ss_layer_stats* out);
SS_API void ss_stats_reset(ss_ctx* c);
typedef void (*ss_stats_hook)(void* user, const ss_layer_stats* forward_total, const ss_layer_stats* per_layer,
                              int n_layers);
SS_API void ss_set_stats_hook(ss_ctx* c, ss_stats_hook hook, void* user);
/* The strix-stream/stats-v1 document of the counters now (reference include/strix_stream/ss.h:552): the backend,
 * forwards, sources_direct, total, layers, and the exclusive (EXCLUSIVE tier mode) and device_gated objects. Freed
 * with ss_free. */
SS_API ss_status ss_stats_to_json(const ss_ctx* c, char** out_json, size_t* out_len);

typedef struct ss_exclusive_stats {
  uint32_t struct_size;
  uint64_t writebacks;
  uint64_t writeback_bytes;
  uint64_t deferred;
  uint64_t promoted;
  uint64_t free_blocks;
  uint64_t min_free_blocks;
  uint64_t rereads;
  uint64_t discards;
} ss_exclusive_stats;
SS_API ss_status ss_stats_exclusive_sized(const ss_ctx* c, ss_exclusive_stats* out, uint32_t size);
static inline ss_status ss_stats_exclusive(const ss_ctx* c, ss_exclusive_stats* out) {
  return ss_stats_exclusive_sized(c, out, (uint32_t)sizeof *out);
}

/* Stats snapshot (reference include/strix_stream/ss.h:573-615): callable from any thread (not concurrently with or
 * after ss_close), also on a poisoned context. The first call arms the context and returns SS_E_INVALID; from then on
 * each ss_end that folds a forward (or token) and each ss_stats_reset between forwards publishes an immutable copy of
 * the counters, which the calls return. The read-ahead fields stay 0 (read-ahead is not served by this library). */
#define SS_HAVE_STATS_SNAPSHOT 1
#define SS_SNAPSHOT_READAHEAD 1u
#define SS_SNAPSHOT_EXCLUSIVE 2u
typedef struct ss_snapshot_info {
  uint32_t struct_size;
  uint32_t flags;
  uint64_t sequence;
  uint64_t forwards;
  uint64_t readahead_buffers, readahead_buffer_bytes, readahead_requested, readahead_read, readahead_landed;
  uint64_t readahead_unused, readahead_failed, readahead_fallback, readahead_bytes;
  uint64_t exclusive_writebacks, exclusive_writeback_bytes, exclusive_deferred, exclusive_promoted;
  uint64_t exclusive_free_blocks, exclusive_min_free_blocks, exclusive_rereads, exclusive_blocks;
  uint64_t exclusive_discards;
} ss_snapshot_info;
SS_API ss_status ss_stats_snapshot_sized(const ss_ctx* c, ss_layer_stats* total_out, ss_snapshot_info* info_out,
                                         uint32_t info_size);
static inline ss_status ss_stats_snapshot(const ss_ctx* c, ss_layer_stats* total_out, ss_snapshot_info* info_out) {
  return ss_stats_snapshot_sized(c, total_out, info_out, (uint32_t)sizeof *info_out);
}
/* The stats-v1 document of the last publication, byte for byte what ss_stats_to_json gave then. Freed with ss_free. */
SS_API ss_status ss_stats_snapshot_json(const ss_ctx* c, char** out_json, size_t* out_len);

/* ---- device-gated decode ---------------------------------------------------------------------------------------- */
#define SS_DG_MAX_PARTS 4
#define SS_DG_MAX_IDS 64
#define SS_DG_PROTOCOL 1
typedef struct ss_dg_part {
  void* base;       /* device arena of this part, `slots` entries */
  uint64_t stride;  /* bytes between slots (== bytes) */
  uint64_t bytes;
} ss_dg_part;
typedef struct ss_dg_device_view {
  uint32_t struct_size, protocol;
  uint32_t n_gated, n_parts, guard_slot, slots;
  const int32_t* slot_of;           /* device, unit_base[n_gated] entries */
  const uint32_t* unit_base;        /* device, n_gated + 1 entries */
  const uint32_t* abort;            /* device word, sticky */
  ss_dg_part parts[SS_DG_MAX_PARTS];
  uint32_t* absent_err;             /* device word: a lookup met an absent entry without abort */
} ss_dg_device_view;
typedef struct ss_dg_unit {
  int32_t gated, unit;
} ss_dg_unit;
SS_API ss_status ss_dg_get_device_view_sized(const ss_ctx* c, ss_dg_device_view* out, uint32_t size);
static inline ss_status ss_dg_get_device_view(const ss_ctx* c, ss_dg_device_view* out) {
  return ss_dg_get_device_view_sized(c, out, (uint32_t)sizeof *out);
}
SS_API int ss_dg_gated_index(const ss_ctx* c, int layer);
/* Launchers on `stream` (legal during hipStreamBeginCapture; ids_dev, n and n_pred are baked into a captured graph). */
SS_API ss_status ss_dg_enqueue_begin(ss_ctx* c, void* stream);
SS_API ss_status ss_dg_enqueue_export(ss_ctx* c, int g, const int32_t* ids_dev, int n, int n_pred, void* stream);
SS_API ss_status ss_dg_enqueue_predict(ss_ctx* c, int g, const int32_t* ids_dev, int n, void* stream);
SS_API ss_status ss_dg_enqueue_wait(ss_ctx* c, int g, void* stream);
SS_API ss_status ss_dg_enqueue_end(ss_ctx* c, void* stream);
#define SS_DG_RESIDENCY 1
SS_API ss_status ss_dg_residency(ss_ctx* c, ss_dg_unit* out, uint32_t cap, uint32_t* total);
SS_API ss_status ss_dg_set_budgets(ss_ctx* c, uint32_t spare_target, uint32_t prefetch_per_layer,
                                   uint32_t prefetch_per_token);
/* Between tokens: the units of gated layer g no later boundary may evict; replaces g's previous set, n = 0 releases
 * it (reference ss.h:683-688, src/capi.cpp:957-959, src/dg_ctx.cpp:678-689). */
SS_API ss_status ss_dg_keep(ss_ctx* c, int g, const int32_t* ids, int n);
/* Between tokens: dg_wb_defer and dg_flush_ready at runtime, 0 / 1 each; turning deferral off submits the deferred
 * write-backs first. Placement and submission only: the same bytes (reference ss.h:693-699, src/capi.cpp:1021-1023,
 * src/dg_ctx.cpp:580-592). dg_flush_ready has no effect on HIP, which submits work as it is enqueued. */
#define SS_DG_SET_SCHED 1
SS_API ss_status ss_dg_set_sched(ss_ctx* c, uint32_t wb_defer, uint32_t flush_ready);
/* Three-tier clean eviction (ss_options.dg_clean_evict) between tokens: on = 0 or 1, from the next boundary's victims
 * on; refused inside a token (SS_E_INVALID). Placement only: the same bytes (reference ss.h:1756-1760,
 * src/capi.cpp:1024-1025). */
#define SS_DG_CLEAN_EVICT 1
SS_API ss_status ss_dg_set_clean_evict(ss_ctx* c, uint32_t on);
/* dg_diag = 1: gated layer g's row of the last completed token, between tokens (reference ss.h:702-729). Host
 * microseconds: seen_us = from the previous layer's service end (layer 0: the previous token's) to its export flag
 * seen; demand_us = flag seen -> its misses' copies and ready enqueued; pred_wait_us = -> its prediction's flag seen;
 * prefetch_us = -> the prediction served; serve_us = flag seen -> the layer's service done (write-back slice included).
 * Counts as the stats count them, for this layer: ids (unique), misses, covered, fetched, prefetched (for the next
 * layer), predicted_true, covered_waits. Device: dma_ms = the demand stream's time from before the layer's first copy
 * to its ready word (-1: no miss); dma_first_ms = to the first fetched unit's copies (-1: no fetch); wb_left_ms = how
 * long the previous boundary's write-backs still ran after the layer's copies began (0: done before; -2: still running
 * at this boundary; -1: none or no miss); gpu_wait_us / gpu_export_ready_us = the wait kernel's entry / the export
 * flag -> ready seen, on the device clock (-1: no miss). A failed token's rows keep their host fields, device ones -1. */
typedef struct ss_dg_layer_timeline {
  uint32_t struct_size, layer;
  double seen_us, demand_us, pred_wait_us, prefetch_us, serve_us;
  uint32_t ids, misses, covered, fetched, prefetched, reserved0;
  double dma_ms;
  uint32_t predicted_true, covered_waits;
  double gpu_wait_us, gpu_export_ready_us, wb_left_ms, dma_first_ms;
} ss_dg_layer_timeline;
SS_API ss_status ss_dg_timeline_sized(const ss_ctx* c, int g, ss_dg_layer_timeline* out, uint32_t size);
/* dg_diag = 1: the last successful boundary's host microseconds: sync = the copy streams' synchronize, select =
 * admissions, retired write-backs and the victims, upload = the table upload, issue = enqueueing the write-backs;
 * writebacks = the victims written back. */
typedef struct ss_dg_boundary_timeline {
  uint32_t struct_size, writebacks;
  double sync_us, select_us, upload_us, issue_us;
} ss_dg_boundary_timeline;
SS_API ss_status ss_dg_boundary_timeline_sized(const ss_ctx* c, ss_dg_boundary_timeline* out, uint32_t size);
/* Scored eviction (policy SS_POLICY_SCORED or SS_POLICY_SCORED_AUTO; reference include/strix_stream/ss.h:730-746).
 * Only the boundary's choice of victims changes: the eligible units (on the device, no write-back in flight) are taken
 * lowest score first, score = w_t P + w_f F + w_r Rec in integers (P: the transition estimate from this token's union
 * of the layer's routed ids; F: how many of the layer's last 16 unions hold the unit; Rec: 1 / (1 + tokens since its
 * last routed use)); ties go to the older use, then to the less recent unit. The history lives as long as the context
 * (ss_stats_reset keeps it). dg_score_w_* (thousandths, summing to 1000; all 0 = 700 / 200 / 100) and an optional
 * TSSCPRF1 dg_score_profile of starting counts, bound to the descriptor's per-unit hashes, are read at ss_open. Host
 * memory: 4 x units^2 bytes per gated layer (twice that with a profile), pageable. */
#define SS_DG_SCORED 1
/* ss_end for a token that closed `rows` verify rows (rows >= 1; ss_end is one row): SCORED_AUTO ranks by score only
 * when rows > 1, else it takes the recency tail (its history still learns). */
SS_API ss_status ss_dg_end_rows(ss_ctx* c, uint32_t rows);
/* Between tokens: drains the write-backs, switches LRU / SCORED / SCORED_AUTO and resets the learning to the open
 * profile's counts (or zero) and every demand epoch, keeping placement and recency. Switching to scoring needs a
 * context opened with SCORED or SCORED_AUTO (SS_E_INVALID otherwise). */
#define SS_DG_SET_POLICY 1
SS_API ss_status ss_dg_set_policy(ss_ctx* c, ss_policy policy);

/* The reference layout in full (fields this library does not count stay 0). */
typedef struct ss_dg_stats {
  uint32_t struct_size, reserved0;
  uint64_t tokens, lookups, misses, covered, fetched, prefetched, prefetch_used, pred_invalid;
  uint64_t resurrected, bank_serves, collected_mid, evicted, evict_short, writebacks_done, stalled;
  uint64_t free_slots, blocks, slots;
  uint64_t predicted, predicted_true, miss_layers, device_timeouts, covered_waits;
  uint64_t wb_deferred, wb_cancelled, wb_forced, wb_boundary_flushed;
  uint64_t wb_issued_bytes, wb_completed_bytes, wb_cancelled_bytes, wb_boundary_flushed_bytes, wb_outstanding_bytes;
  uint64_t wb_forced_wait_ns;
  uint64_t winpf_hints, winpf_hint_rows, prior_issued, prior_used, prior_late, prior_reverted;
  uint64_t l1_candidates, l1_issued, l1_used, l1_late, l1_reverted, l1_priced_out, l1_skipped_ahead;
  uint64_t prior_budget_stops;
  uint64_t score_fallbacks, scored_victims, score_layers, score_candidates, score_saturated, score_ns;
  uint64_t score_deferred, score_last_ns;
  uint64_t disk_reads, disk_read_bytes, disk_read_ns, disk_stage_waits, disk_drops, disk_discards;
  uint64_t inclusive_kept, inclusive_drops, disk_units, backed_units;
  uint64_t disk_wait_ns;
  uint64_t disk_overlapped, disk_max_in_flight, disk_carried, disk_carried_bytes;
  uint64_t resident_units, resident_evicted, resident_bytes, resident_ns;
  uint64_t round_count, round_units, round_bytes, round_ns, round_cancelled;
  uint32_t cuda_module_loading;
  uint32_t reserved1;
  uint64_t clean_drops, clean_drop_bytes;
  uint64_t mkres_file_reads, mkres_file_bytes, mkres_read_ns, mkres_h2d_bytes, mkres_wb_bytes;
  uint64_t lm_tokens, lm_parts, lm_mid_evictions, lm_early_admits;
  uint64_t pf_reverted, pf_revert_bytes;
  uint64_t pred_skipped_ahead, pf_strict_refused;
  uint64_t pred_shadow_file_predicted, pred_shadow_file_demanded, pred_shadow_file_hit;
  uint64_t pred_shadow_file_predicted_bytes, pred_shadow_file_demanded_bytes, pred_shadow_file_hit_bytes;
  uint32_t disk_queue_resolved, disk_locations;
  uint64_t landing_issued, landing_promoted, landing_late, landing_wait_ns, landing_expired, landing_dropped_full;
  uint64_t landing_read_bytes;
  uint64_t landing_cancelled;
  uint64_t landing_expired_layer, landing_skipped_passed;
  uint64_t landing_yields, landing_aborted_bytes;
  uint64_t bank_kept;
  uint32_t disk_depth_active, disk_depth_adapt;
  uint64_t disk_depth_changes, disk_depth_calibrations;
} ss_dg_stats;
SS_API ss_status ss_stats_dg_sized(const ss_ctx* c, ss_dg_stats* out, uint32_t size);
static inline ss_status ss_stats_dg(const ss_ctx* c, ss_dg_stats* out) {
  return ss_stats_dg_sized(c, out, (uint32_t)sizeof *out);
}

/* Engine-side slot lookup (inline device code). The reference header offers it to CUDA only (__CUDACC__); hipcc for
 * gfx950 defines __HIPCC__, so this branch gives HIP engines the same two rules: abort set or id out of range -> the
 * guard slot; an absent entry (< 0) -> absent_err |= 1 (when the view's struct_size covers it) and the guard slot. */
#if defined(__HIPCC__)
static __device__ __forceinline__ int32_t ss_dg_slot(const ss_dg_device_view* v, uint32_t g, int32_t id) {
  if (__hip_atomic_load(v->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return (int32_t)v->guard_slot;
  const uint32_t b = v->unit_base[g];
  if ((uint32_t)id >= v->unit_base[g + 1] - b) return (int32_t)v->guard_slot;
  const int32_t s = __hip_atomic_load(v->slot_of + b + (uint32_t)id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (s >= 0) return s;
  if ((uint32_t)((const char*)&v->absent_err - (const char*)v) + (uint32_t)sizeof(void*) <= v->struct_size &&
      v->absent_err)
    atomicOr(v->absent_err, 1u);
  return (int32_t)v->guard_slot;
}
/* Before the layer's wait (resident-first execution): the slot if published, else -1 (acquire at system scope). */
static __device__ __forceinline__ int32_t ss_dg_slot_if_ready(const ss_dg_device_view* v, uint32_t g, int32_t id) {
  if (__hip_atomic_load(v->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return (int32_t)v->guard_slot;
  const uint32_t b = v->unit_base[g];
  if ((uint32_t)id >= v->unit_base[g + 1] - b) return (int32_t)v->guard_slot;
  const int32_t s = __hip_atomic_load(v->slot_of + b + (uint32_t)id, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
  return s >= 0 ? s : -1;
}
#endif

#ifdef __cplusplus
}
#endif

#endif /* STRIX_STREAM_SS_H */
