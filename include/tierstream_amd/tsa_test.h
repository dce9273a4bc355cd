/*
 * Test hooks of libtierstream_amd (the counterpart of reference include/strix_stream/ss_test.h: calls tests link by
 * name that an engine never needs). None changes the cache state.
 */
#ifndef TIERSTREAM_AMD_TSA_TEST_H
#define TIERSTREAM_AMD_TSA_TEST_H

#include <stdint.h>

#include "../strix_stream/ss.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Host contract: where a table address points. kind 1 = layer `index`'s resident pool, 2 = stream ring class `index`
 * (ascending slot size), 0 = neither; offset = bytes from that region's base (slot = offset / unit stride). */
SS_API ss_status tsa_test_region_of(const ss_ctx* c, uint64_t addr, int* kind, int* index, uint64_t* offset);
/* Device-gated: the host mirror of slot_of (one int32 per gated key, -1 = not on the device); *n = keys. */
SS_API ss_status tsa_test_dg_table(const ss_ctx* c, int32_t* out, uint32_t cap, uint32_t* n);
/* verify_hash = 2: landed units whose device check failed, since open. */
SS_API uint64_t tsa_test_verify_failures(const ss_ctx* c);
/* Device-gated: 1 when the context's unit copies go through the HSA runtime's copy engines (each with a completion
 * signal), 0 when they go through HIP streams (the file tier, parts small enough to be staged and scattered, or
 * TSA_DG_COPIES=hip at open). */
SS_API int tsa_test_dg_hsa_copies(const ss_ctx* c);
/* Host contract test hooks under the reference's names (its src/capi.cpp:721-734; its tests declare them by hand):
 * reader threads take no job while held (closing the context still ends them); wait until every read-ahead read of
 * the open forward has ended (readers not held). */
SS_API ss_status ss_test_hold_readers(ss_ctx* c, int hold);
SS_API ss_status ss_test_ra_quiesce(ss_ctx* c);
/* One-shot fault injection in the host read-ahead path (reference src/capi.cpp:717-719, src/stream_ctx.cpp:508-1015):
 * 1 queueing a read fails, 2 queueing a landing fails, 3 a landing's copy fails before it starts, 4 after its first
 * piece (the buffer is quarantined), 5 a read fails, 8 a read fails after a part, 9 a read's bytes fail the hash.
 * The reference's copy mutations 6, 7 and 10 (a copy that skips a wait) are refused with SS_E_UNSUPPORTED. */
SS_API ss_status ss_test_inject(ss_ctx* c, int what);
/* Exclusive tier mode, between forwards: every pinned block held exactly once (a unit off the device, or a free list),
 * no write-back pending (reference src/capi.cpp:691-696, src/stream_ctx.cpp:1914-1938). SS_E_INVALID names the first
 * broken rule; the context is not poisoned. */
SS_API ss_status ss_test_check_exclusive(ss_ctx* c);
/* Device-gated, for a context opened with dg_test_hooks = 1 (reference include/strix_stream/ss_test.h:19, :30,
 * src/capi.cpp:898-921): the cache core's ownership invariants between tokens (SS_E_BACKEND names the first broken
 * one, nothing is poisoned); stop the service thread (the next token fails closed and poisons the context). */
SS_API ss_status ss_test_dg_check(ss_ctx* c);
SS_API ss_status ss_test_dg_stop_service(ss_ctx* c);
/* Host contract: unit copies from pinned blocks since open, and the host-to-device copies they were issued as (a run
 * of neighbouring units is one copy). SS_E_INVALID on a device-gated context. */
SS_API ss_status tsa_test_host_copies(const ss_ctx* c, uint64_t* units, uint64_t* copies);

/* Device-gated timing (measurement only; the cache state is untouched). While enabled the library brackets every unit
 * copy host -> HBM, every write-back HBM -> host and every device verify launch with timed events on the stream that
 * runs it; durations are summed once the events completed. Enabling (or disabling) resets the totals. */
typedef struct tsa_test_profile {
  uint64_t copies;          /* unit copies into HBM (demand and prefetch) */
  uint64_t copy_bytes;
  uint64_t copy_ns;         /* summed durations: the copy engines' busy time */
  uint64_t writebacks;      /* unit (or part) copies out of HBM */
  uint64_t writeback_bytes;
  uint64_t writeback_ns;
  uint64_t verifies;        /* verify kernel launches (verify_hash = 2) */
  uint64_t verify_units;
  uint64_t verify_bytes;    /* bytes hashed: the units' bytes */
  uint64_t verify_ns;
  uint64_t pending;         /* bracketed operations whose events had not completed at the read */
} tsa_test_profile;
/* on: a mask of what is bracketed, TSA_TEST_PROF_COPY | _WRITEBACK | _VERIFY (0: nothing); 1 keeps its older meaning
 * of everything. The verify launches take the dispatch's own begin and end stamps (no extra stream work); a copy
 * bracket records two events on the copy's stream. A host-contract context brackets its check launches only
 * (TSA_TEST_PROF_VERIFY; between forwards); a device-gated one every kind (between tokens). */
#define TSA_TEST_PROF_COPY 0x2
#define TSA_TEST_PROF_WRITEBACK 0x4
#define TSA_TEST_PROF_VERIFY 0x8
SS_API ss_status tsa_test_profile_enable(ss_ctx* c, int on);
/* Between tokens; wait = 1 first waits for every bracketed operation (write-backs may still run after ss_end). */
SS_API ss_status tsa_test_profile_read(ss_ctx* c, int wait, tsa_test_profile* out);
/* Between tokens: the device-gated kernels' wall-clock stamps of the last token (100 MHz ticks), 4 per gated layer:
 * export end, wait entry, ready seen (0: the layer had no miss and the wait returned at once), wait exit. *n = 4 G. */
SS_API ss_status tsa_test_dg_stamps(const ss_ctx* c, uint64_t* out, uint32_t cap, uint32_t* n);
/* Between tokens: flips byte `offset` of unit (gated, unit)'s copy in its pinned block (the unit must live in its block,
 * off the device), so that its next landing fails the device check (verify_hash = 2). SS_E_INVALID otherwise. */
SS_API ss_status tsa_test_dg_corrupt_block(ss_ctx* c, int gated, int unit, uint64_t offset);

/* The device-gated cache state machine alone (no device, no context): this library's DgCore driven on an eager
 * transport whose copies, entries, events and file reads complete at once - the reference's canonical schedule
 * (reference tests/test_dg.cpp:201) - so its placement can be compared with the reference core's on the CPU. Each
 * token: per gated layer the export mask from the table as the device would read it, serve_demand, serve_use, the
 * deferred write-back slice, then the boundary and the ownership check. */
typedef struct tsa_test_dgcore_config {
  const uint32_t* n_units; /* per gated layer */
  uint32_t n_gated;
  uint32_t persistent_slots, bank_slots, blocks, spare_target;
  uint32_t prefetch_reserve; /* 0xFFFFFFFF: automatic (min(24, spare_target / 4)) */
  uint32_t prefetch_per_layer, prefetch_per_token;
  uint32_t wb_defer, wb_on_d2h, inclusive;
  const uint64_t* part_bytes;
  uint32_t n_parts;
  uint32_t disk_tier, home_blocks, disk_staging, clean_evict, disk_prefetch;
  const uint8_t* disk; /* three-tier: 1 per key for the plan's file tier (key order) */
  /* appended, scored eviction: policy 0 LRU / 1 SCORED / 2 SCORED_AUTO, the score weights (thousandths, sum 1000), the
   * verify rows each token's boundary closes (0 = 1), starting transition counts (per gated layer units^2 uint32
   * row-major [previous unit][unit], layers concatenated; null = an empty table). The union width is bank_slots. */
  uint32_t policy, w_trans, w_freq, w_rec, rows;
  const uint32_t* score_cells;
  /* appended: dg_bank_keep (0, 1, 2; three-tier only) */
  uint32_t bank_keep;
  /* appended: dg_landing_blocks and dg_landing_ttl (three-tier only; 0 blocks: no landing) */
  uint32_t landing_blocks, landing_ttl;
} tsa_test_dgcore_config;
SS_API ss_status tsa_test_dgcore_open(const tsa_test_dgcore_config* cfg, const uint32_t* order, uint32_t n_order,
                                      void** out);
/* ids [n_gated][n]; table_out [keys]; counts [n_counts] in the order of tsa_test_dgcore_counter_names. */
SS_API ss_status tsa_test_dgcore_token(void* h, const uint32_t* ids, uint32_t n, int32_t* table_out, uint64_t* counts,
                                       uint32_t n_counts);
SS_API const char* tsa_test_dgcore_counter_names(void);
/* dg_disk_queue_adapt's read-depth controller alone (no pool, no clock): n busy periods (reads[i], bytes[i], ns[i])
 * fed in order; depth[i] = the depth after period i; counters[13] = changes, calibrations, windows, verdicts,
 * reads_1, bytes_1, ns_1, reads_u, bytes_u, ns_u, depth, bound, calibrating; recent[16 * 7] = the last verdicts (seq,
 * reads, from, to, GB/s at U, GB/s at 1, why: 0 start, 1 keep U, 2 keep 1, 3 split, 4 recheck, 5 drift); *n_recent
 * their count. */
SS_API ss_status tsa_test_depth_ctl(uint32_t bound, uint32_t n, const uint64_t* reads, const uint64_t* bytes,
                                    const uint64_t* ns, uint32_t* depth, uint64_t* counters, double* recent,
                                    uint32_t* n_recent);
/* The three-tier read pool alone (no device, no file): scenario 0..9 on a pool whose reader blocks each unit's pieces
 * behind a gate the scenario opens - demand reads before landing reads, the landing cap, the reader kept free of
 * landing reads, a drop (cancelled, cut short), a claim, failures, a yield, whole landing reads, stop, one read per
 * word. SS_OK when the scenario's checks hold, else SS_E_BACKEND with the failed check in msg. */
SS_API ss_status tsa_test_read_pool(uint32_t scenario, char* msg, uint32_t cap);
/* The host contract's cross-stream wait bookkeeping alone (no device): n_ops random event records, waits and stream
 * replacements over n_streams (1..16) streams, checked against vector clocks that apply every wait. counts[0] = 0 when
 * every stream's clock stays equal to the reference's, else the first step (1-based) at which one differs; counts[1] =
 * the waits skipped as implied. mode 0: the library's bookkeeping; 1 and 2: planted mistakes the check must catch (an
 * earlier wait counted whatever its mark; a replaced stream keeping its predecessor's waits). */
SS_API ss_status tsa_test_stream_order(uint32_t seed, uint32_t n_ops, uint32_t n_streams, int mode, uint64_t* counts);
/* Host contract: cross-stream waits given to the runtime since open, and those skipped as implied by an earlier wait of
 * the same stream. SS_E_INVALID on a device-gated context. */
SS_API ss_status tsa_test_host_waits(const ss_ctx* c, uint64_t* issued, uint64_t* skipped);
/* As tsa_test_dgcore_token with run [n_gated] (null: all): the gated layers the token exports (ss_begin's rows). */
SS_API ss_status tsa_test_dgcore_token_run(void* h, const uint32_t* ids, uint32_t n, const uint8_t* run,
                                           int32_t* table_out, uint64_t* counts, uint32_t n_counts);
/* As tsa_test_dgcore_token_run with predictions pred [n_gated][n_pred] (row g: the ids predicted at layer g for layer
 * g + 1, served right after layer g's use when layer g + 1 exports; n_pred 0: none). */
SS_API ss_status tsa_test_dgcore_token_pred(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred,
                                            uint32_t n_pred, const uint8_t* run, int32_t* table_out, uint64_t* counts,
                                            uint32_t n_counts);
/* Between tokens: the policy switch of ss_dg_set_policy on the core alone. */
SS_API ss_status tsa_test_dgcore_set_policy(void* h, uint32_t policy);
/* The keys every later boundary must not evict (ss_dg_keep of every gated layer; n = 0: none), and the runtime switch
 * of write-back deferral (ss_dg_set_sched's wb_defer), on the core alone. */
SS_API ss_status tsa_test_dgcore_set_keep(void* h, const uint32_t* keys, uint32_t n);
/* Copy-order checking on the core's CPU transport: the copies kept as a device would run them (each stream in order,
 * streams ordered only by the waits the core asks for); a later token call fails at the first file read, copy in or
 * copy out whose memory a copy not ordered before it may still use. */
SS_API ss_status tsa_test_dgcore_check_order(void* h, int on);
/* The host contract's placement alone on the CPU (no device): a context over desc_json and the budget (plan_make,
 * no benefit), `steps` forwards of the engine loop - ss_begin; per layer with units ss_layer_routes (mode 0, 2) or
 * ss_layer_all (mode 1), ss_acquire (modes 0, 1) or ss_acquire_groups (mode 2); prefetch (may be NULL): the next
 * layer's predicted ids ([steps][layers][max_ids], -1 padded), ss_prefetch of layer l + 1 after layer l's acquire,
 * CERTAIN on even steps and SPECULATIVE on odd ones; ss_release; ss_end - every copy complete when issued. Outputs
 * per [step][layer][unit < max_units]: the table entry's kind (0 none, 1 the layer's pool, 2 the ring) and index (pool
 * slot or global ring slot), the unit's group (-1: none); per step the forward's total counters. */
SS_API ss_status tsa_test_hostplace_run(const char* desc_json, size_t len, const ss_budget* budget,
                                        const ss_options* opt, int steps, const int32_t* routes,
                                        const int32_t* prefetch, int max_ids, int mode, int max_units,
                                        int32_t* spot_kind, int32_t* spot_index, int32_t* group_of,
                                        ss_layer_stats* stats);
/* The device-gated open's geometry alone (no device): the descriptor, the budget and the plan (tiers, one per unit in
 * descriptor order; NULL: plan_make) under the options. out[0..22]: keys, gated layers, R, D, B, P, F, Q, I, staging
 * buffers, disk queue, persistent slots, slots, guard slot, blocks, scored, w_trans, w_freq, w_rec, landing blocks,
 * landing pieces running at most, landing TTL, landing piece bytes (0: one per part); residents: the planned
 * residents' keys (up to res_cap). A refused configuration returns its status. */
SS_API ss_status tsa_test_dg_geometry(const char* desc_json, size_t len, const ss_budget* budget, const uint8_t* tiers,
                                      size_t n_tiers, const ss_options* opt, uint32_t* out, uint32_t* residents,
                                      uint32_t res_cap);
/* The host contract's copy runs alone (no device): orders k = 0 .. n-1 with their layer, source and destination
 * allocations (-1 source: not a pinned block) and addresses; run_of[k] = the index of the copy that carries order k
 * (neighbouring units in both allocations, one slot apart, at most cap bytes per copy). */
SS_API ss_status tsa_test_copy_runs(const int32_t* layer, const int32_t* src_alloc, const int32_t* dst_alloc,
                                    const uint64_t* src, const uint64_t* dst, size_t n, uint64_t unit_bytes,
                                    uint64_t cap, uint32_t* run_of);
/* The host contract's read scheduler alone, single-threaded: ops[3k .. 3k+2] = (op, class, id) with op 0 push,
 * 1 raise (from class to the head of demand), 2 remove, 3 take (a reader asks for a read: taken[2j] = its id or -1,
 * taken[2j+1] = its class or -1), 4 end (a read of class ended), 5 hold (id != 0) or release, 6 stop; classes
 * 0 demand, 1 read-ahead, 2 speculative. *n_taken = the takes. No reference counterpart: it pins the executor's rule. */
SS_API ss_status tsa_test_read_sched(const int32_t* ops, size_t n_ops, int readers, int32_t* taken, size_t* n_taken);
/* The aligned windows covering [off, off + n) with reads aligned to al, at most cap bytes of the range each:
 * windows[5k .. 5k+4] = (at, len, a0, span, lead). No reference counterpart. */
SS_API ss_status tsa_test_cover_windows(uint64_t off, uint64_t n, uint64_t al, uint64_t cap, uint64_t* windows,
                                        size_t max_w, size_t* n_w);
/* The same loop (prefetch may be NULL); the exclusive-mode counters after the last forward. */
SS_API ss_status tsa_test_hostplace_exclusive(const char* desc_json, size_t len, const ss_budget* budget,
                                              const ss_options* opt, int steps, const int32_t* routes,
                                              const int32_t* prefetch, int max_ids, int mode,
                                              ss_exclusive_stats* out);
SS_API ss_status tsa_test_dgcore_set_wb_defer(void* h, uint32_t on);
/* Scored eviction's profile rules without a context: the SHA-256 of data[0..n) (32 raw bytes into out), and the
 * TSSCPRF1 checks of a profile against the gated layers' units and a 32-byte identity (SS_E_INVALID naming the first
 * broken rule; the provenance into prov, NUL-terminated, when it passes). */
SS_API ss_status tsa_test_sha256(const void* data, uint64_t n, unsigned char* out);
SS_API ss_status tsa_test_score_profile_check(const void* data, uint64_t len, const uint32_t* units, uint32_t n_gated,
                                              const unsigned char* identity, char* prov, uint32_t prov_cap);
/* Three-tier: the pinned homes, most recently homed first; the return is the count. */
SS_API uint32_t tsa_test_dgcore_host_order(void* h, uint32_t* out, uint32_t cap);
/* Landings: per landing block the key it holds (0xFFFFFFFF: none); the return is the landing blocks. */
SS_API uint32_t tsa_test_dgcore_land_owner(void* h, uint32_t* out, uint32_t cap);
SS_API void tsa_test_dgcore_close(void* h);

#ifdef __cplusplus
}
#endif

#endif
