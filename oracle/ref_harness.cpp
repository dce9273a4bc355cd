// ORACLE (test infrastructure only): a harness over the reference's own code, compiled with its sources in place by
// oracle/Makefile (target `ref`) into _ref/libtsref_harness.so. It never ships in the product.
//
//  * ref_region_of: where a host-contract table address of a reference CPU context points (layer pool + offset, or
//    stream ring class + offset), read from the reference Ctx's own fields, so tables compare "up to base offset".
//  * refdg_*: the reference DgCore (src/dg_core.cpp) driven exactly as its CPU tests drive it in eager mode
//    (tests/test_dg.cpp:201): a transport whose copies, entries and events complete at once (done() is always true)
//    and a service loop that never sees the device "ahead". Each token: begin_token, per gated layer the export mask
//    from the table as the device would read it, serve_demand, serve_use, issue_writebacks, then end_token.
//  * refdg_cpu_baseline: the same core on a synchronous memcpy transport over host memory, timed per token: the CPU
//    baseline the benchmark reports beside the device numbers (device-gated decode has no CPU backend in the reference).
// every standard header the reference headers pull in, first (the access override below must not reach them)
#include <algorithm>
#include <atomic>
#include <cctype>
#include <chrono>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <filesystem>
#include <fstream>
#include <functional>
#include <iostream>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#define private public
#define protected public
#include "dg_core.hpp"
#include "dg_score.hpp"
#include "dg_load.hpp"
#include "stream_ctx.hpp"
#include "dg_layout.hpp"
#include "xxh64.hpp"
#undef private
#undef protected

extern "C" {

int ref_region_of(void* ctx, uint64_t addr, int* kind, int* index, uint64_t* offset) {
  // ss_ctx's first member is the host-contract Ctx (reference src/capi.cpp:31-34)
  auto* up = reinterpret_cast<std::unique_ptr<ts::Ctx>*>(ctx);
  ts::Ctx* c = up->get();
  *kind = 0;
  *index = -1;
  *offset = 0;
  if (!c || !addr) return 0;
  for (size_t L = 0; L < c->L_.size(); ++L) {
    const auto& s = c->L_[L];
    if (!s.pool || !s.rs) continue;
    const uint64_t b = uint64_t(uintptr_t(s.pool));
    const uint64_t n = uint64_t(s.rs->capacity()) * c->d_.unit_stride(int(L));
    if (addr >= b && addr < b + n) {
      *kind = 1;
      *index = int(L);
      *offset = addr - b;
      return 1;
    }
  }
  for (size_t k = 0; k < c->ring_classes_.size(); ++k) {
    const auto& r = c->ring_classes_[k];
    const uint64_t b = uint64_t(uintptr_t(r.base));
    if (addr >= b && addr < b + r.stride * r.count) {
      *kind = 2;
      *index = int(k);
      *offset = addr - b;
      return 1;
    }
  }
  return 0;
}

}  // extern "C"

namespace {

// Everything completes at once; events are counters.
class Eager final : public ts::DgTransport {
 public:
  explicit Eager(std::vector<uint64_t> parts) : parts_(std::move(parts)) {}
  void h2d(Stream, int32_t, int32_t) override {}
  void d2h(int32_t, int32_t) override {}
  void d2h_part(Stream, int32_t, int32_t, uint32_t) override {}
  void d2d(int32_t, int32_t) override {}
  void h2h(int32_t, int32_t) override {}
  uint32_t parts() const override { return uint32_t(parts_.size()); }
  uint64_t part_bytes(uint32_t p) const override { return parts_[p]; }
  void write_entry(Stream, uint32_t, int32_t) override {}
  void signal_ready(uint32_t, uint32_t) override {}
  void* event_create() override { return new int(0); }
  void event_destroy(void* ev) override { delete static_cast<int*>(ev); }
  void record(void*, Stream) override {}
  void wait(Stream, void*) override {}
  bool done(void*) override { return true; }
  void event_sync(void*) override {}
  void sync(Stream) override {}
  void upload_table(const int32_t*, uint32_t) override {}
  void upload_table_ranges(const int32_t*, const uint32_t*, uint32_t) override {}
  void read_unit(uint32_t, int32_t) override {}  // three-tier: the file read completes at once too

 private:
  std::vector<uint64_t> parts_;
};

struct RefDg {
  std::unique_ptr<Eager> t;
  std::unique_ptr<ts::DgCore> core;
  uint32_t seq = 0;
  uint32_t rows = 1;  // the verify rows each token's boundary closes (scored auto ranks only above one)
  std::vector<uint32_t> keep;  // the boundary's keep list, as the reference context builds it (DgSteps::all_kept)
};

}  // namespace

extern "C" {

// Three-tier options of refdg_open (disk_tier 0: none of the others is read): home_blocks = the plan's pinned units,
// disk_staging buffers, the file-tier flags of the keys (keys entries, key order), clean_evict, disk_prefetch.
struct RefDiskOpts {
  uint32_t disk_tier = 0, home_blocks = 0, disk_staging = 0, clean_evict = 0, disk_prefetch = 0, bank_keep = 0;
  uint32_t landing_blocks = 0, landing_ttl = 0;
  const uint8_t* disk = nullptr;
};
// Scored eviction options of refdg_open (policy 0 = LRU: none of the others is read): policy 1 SCORED / 2 SCORED_AUTO,
// the weights, the verify rows each boundary closes, and optional starting counts (per gated layer units^2 uint32
// row-major, layers concatenated; null: an empty table), loaded as the reference loads a TSSCPRF1 profile (written by
// its own dg_profile_write under a fixed identity).
struct RefScoreOpts {
  uint32_t policy = 0, w_trans = 700, w_freq = 200, w_rec = 100, rows = 1;
  const uint32_t* cells = nullptr;
};
void* refdg_open_impl(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                      uint32_t spare_target, uint32_t prefetch_reserve, uint32_t pf_layer, uint32_t pf_token,
                      uint32_t wb_defer, uint32_t wb_on_d2h, uint32_t inclusive, const uint64_t* part_bytes,
                      uint32_t n_parts, const uint32_t* order, uint32_t n_order, const RefDiskOpts& dk,
                      const RefScoreOpts& so = RefScoreOpts{});

void* refdg_open(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                 uint32_t spare_target, uint32_t prefetch_reserve, uint32_t pf_layer, uint32_t pf_token,
                 uint32_t wb_defer, uint32_t wb_on_d2h, uint32_t inclusive, const uint64_t* part_bytes,
                 uint32_t n_parts, const uint32_t* order, uint32_t n_order) {
  return refdg_open_impl(n_units, G, persistent, bank, blocks, spare_target, prefetch_reserve, pf_layer, pf_token,
                         wb_defer, wb_on_d2h, inclusive, part_bytes, n_parts, order, n_order, RefDiskOpts{});
}

void* refdg_open_disk(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                      uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                      uint32_t n_parts, const uint32_t* order, uint32_t n_order, uint32_t home_blocks,
                      uint32_t disk_staging, uint32_t clean_evict, uint32_t disk_prefetch, const uint8_t* disk) {
  RefDiskOpts dk;
  dk.disk_tier = 1;
  dk.home_blocks = home_blocks;
  dk.disk_staging = disk_staging;
  dk.clean_evict = clean_evict;
  dk.disk_prefetch = disk_prefetch;
  dk.disk = disk;
  return refdg_open_impl(n_units, G, persistent, bank, blocks, spare_target, 0xFFFFFFFFu, 4, 48, wb_defer, 1, inclusive,
                         part_bytes, n_parts, order, n_order, dk);
}

// refdg_open_disk with dg_bank_keep (0, 1, 2) and landings (landing_blocks 0: none; landing_ttl).
void* refdg_open_disk_land(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                           uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                           uint32_t n_parts, const uint32_t* order, uint32_t n_order, uint32_t home_blocks,
                           uint32_t disk_staging, uint32_t clean_evict, uint32_t disk_prefetch, const uint8_t* disk,
                           uint32_t bank_keep, uint32_t landing_blocks, uint32_t landing_ttl) {
  RefDiskOpts dk;
  dk.disk_tier = 1;
  dk.home_blocks = home_blocks;
  dk.disk_staging = disk_staging;
  dk.clean_evict = clean_evict;
  dk.disk_prefetch = disk_prefetch;
  dk.disk = disk;
  dk.bank_keep = bank_keep;
  dk.landing_blocks = landing_blocks;
  dk.landing_ttl = landing_ttl;
  return refdg_open_impl(n_units, G, persistent, bank, blocks, spare_target, 0xFFFFFFFFu, 4, 48, wb_defer, 1, inclusive,
                         part_bytes, n_parts, order, n_order, dk);
}

// refdg_open_disk with dg_bank_keep (0, 1, 2).
void* refdg_open_disk_keep(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                           uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                           uint32_t n_parts, const uint32_t* order, uint32_t n_order, uint32_t home_blocks,
                           uint32_t disk_staging, uint32_t clean_evict, uint32_t disk_prefetch, const uint8_t* disk,
                           uint32_t bank_keep) {
  RefDiskOpts dk;
  dk.disk_tier = 1;
  dk.home_blocks = home_blocks;
  dk.disk_staging = disk_staging;
  dk.clean_evict = clean_evict;
  dk.disk_prefetch = disk_prefetch;
  dk.disk = disk;
  dk.bank_keep = bank_keep;
  return refdg_open_impl(n_units, G, persistent, bank, blocks, spare_target, 0xFFFFFFFFu, 4, 48, wb_defer, 1, inclusive,
                         part_bytes, n_parts, order, n_order, dk);
}

// refdg_open with scored eviction (RefScoreOpts) on the two-tier cache, or with disk flags (disk non-null) three-tier.
void* refdg_open_scored(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                        uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                        uint32_t n_parts, const uint32_t* order, uint32_t n_order, uint32_t policy, uint32_t w_trans,
                        uint32_t w_freq, uint32_t w_rec, uint32_t rows, const uint32_t* cells, uint32_t home_blocks,
                        uint32_t disk_staging, uint32_t clean_evict, const uint8_t* disk) {
  RefDiskOpts dk;
  if (disk) {
    dk.disk_tier = 1;
    dk.home_blocks = home_blocks;
    dk.disk_staging = disk_staging;
    dk.clean_evict = clean_evict;
    dk.disk = disk;
  }
  RefScoreOpts so;
  so.policy = policy;
  so.w_trans = w_trans;
  so.w_freq = w_freq;
  so.w_rec = w_rec;
  so.rows = rows ? rows : 1;
  so.cells = cells;
  return refdg_open_impl(n_units, G, persistent, bank, blocks, spare_target, 0xFFFFFFFFu, 4, 48, wb_defer, 1, inclusive,
                         part_bytes, n_parts, order, n_order, dk, so);
}

// The reference's model identity of a profile (dg_score_identity): per gated layer its model layer index, units, unit
// bytes and per-unit xxh64 (hashes concatenated); the 32 raw bytes into out.
int refdg_score_identity(uint32_t n_gated, const uint32_t* index, const uint32_t* units, const uint64_t* unit_bytes,
                         const uint64_t* hashes, unsigned char* out) {
  try {
    std::vector<std::vector<uint64_t>> h(n_gated);
    std::vector<ts::DgScoreIdLayer> v(n_gated);
    for (uint32_t g = 0; g < n_gated; ++g) {
      h[g].assign(hashes, hashes + units[g]);
      hashes += units[g];
      v[g].index = index[g];
      v[g].units = units[g];
      v[g].unit_bytes = unit_bytes[g];
      v[g].hash = &h[g];
    }
    const std::string id = ts::dg_score_identity(v);
    std::memcpy(out, id.data(), 32);
    return 0;
  } catch (const std::exception& e) {
    return 1;
  }
}

// The reference's TSSCPRF1 checks (dg_profile_check): 0 when the profile passes, 1 when it refuses it.
int refdg_profile_check(const void* data, uint64_t len, const uint32_t* units, uint32_t n_gated,
                        const unsigned char* identity) {
  try {
    (void)ts::dg_profile_check(data, len, std::vector<uint32_t>(units, units + n_gated),
                               std::string(reinterpret_cast<const char*>(identity), 32));
    return 0;
  } catch (const std::exception& e) {
    return 1;
  }
}

// Between tokens: the reference's set_policy (drains, switches, resets the learning, renumbers the stamps).
int refdg_set_policy(void* h, uint32_t policy) {
  try {
    static_cast<RefDg*>(h)->core->set_policy(policy);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_set_policy: %s\n", e.what());
    return 1;
  }
}

void* refdg_open_impl(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                      uint32_t spare_target, uint32_t prefetch_reserve, uint32_t pf_layer, uint32_t pf_token,
                      uint32_t wb_defer, uint32_t wb_on_d2h, uint32_t inclusive, const uint64_t* part_bytes,
                      uint32_t n_parts, const uint32_t* order, uint32_t n_order, const RefDiskOpts& dk,
                      const RefScoreOpts& so) {
  try {
    auto* r = new RefDg;
    r->t = std::make_unique<Eager>(std::vector<uint64_t>(part_bytes, part_bytes + n_parts));
    ts::DgConfig c;
    c.n_units.assign(n_units, n_units + G);
    c.persistent_slots = persistent;
    c.bank_slots = bank;
    c.blocks = blocks;
    c.spare_target = spare_target;
    c.prefetch_reserve_auto = prefetch_reserve == 0xFFFFFFFFu;
    c.prefetch_reserve = c.prefetch_reserve_auto ? std::min<uint32_t>(24, spare_target / 4) : prefetch_reserve;
    c.prefetch_per_layer = pf_layer;
    c.prefetch_per_token = pf_token;
    c.wb_defer = wb_defer != 0;
    c.wb_on_d2h = wb_on_d2h != 0;
    c.inclusive = inclusive;
    c.max_ids = bank;
    c.pf_legacy = true;
    std::vector<uint8_t> disk;
    if (dk.disk_tier) {
      c.disk_tier = true;
      c.disk_prefetch = dk.disk_prefetch != 0;
      c.home_blocks = dk.home_blocks;
      c.disk_staging = dk.disk_staging;
      c.disk_queue = 1;
      c.clean_evict = dk.clean_evict != 0;
      c.bank_keep = dk.bank_keep;
      c.landing_blocks = dk.landing_blocks;
      c.landing_ttl = dk.landing_ttl;
      uint32_t keys = 0;
      for (uint32_t g = 0; g < G; ++g) keys += n_units[g];
      disk.assign(dk.disk, dk.disk + keys);
    }
    if (so.policy) {  // as the reference context sets it up for SCORED / SCORED_AUTO
      c.scored = true;
      c.scored_auto = so.policy == 2;
      c.boundary_score = true;
      c.w_trans = so.w_trans;
      c.w_freq = so.w_freq;
      c.w_rec = so.w_rec;
    }
    r->rows = so.rows;
    r->core = std::make_unique<ts::DgCore>(c, r->t.get());
    r->core->place(std::vector<uint32_t>(order, order + n_order), dk.disk_tier ? &disk : nullptr);
    if (so.policy && so.cells) {
      const std::string identity(32, '\x5a');
      std::vector<std::vector<uint32_t>> cells(G);
      const uint32_t* p = so.cells;
      for (uint32_t g = 0; g < G; ++g) {
        cells[g].assign(p, p + size_t(n_units[g]) * n_units[g]);
        p += size_t(n_units[g]) * n_units[g];
      }
      const std::string prof = ts::dg_profile_write(c.n_units, identity, "oracle", cells);
      r->core->load_profile(prof.data(), prof.size(), identity);
    }
    return r;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_open: %s\n", e.what());
    return nullptr;
  }
}

// One token: ids [G][n] (every gated layer exported), pred [G][n_pred] (the prediction for layer g + 1 made at g;
// n_pred = 0: none). Writes the table after the boundary (keys int32) and the counters (see refdg_counter_names).
int refdg_token_run(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred, uint32_t n_pred,
                    const uint8_t* run, int32_t* table_out, uint64_t* counts);
int refdg_token(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred, uint32_t n_pred, int32_t* table_out,
                uint64_t* counts) {
  return refdg_token_run(h, ids, n, pred, n_pred, nullptr, table_out, counts);
}

// As refdg_token with run [G] (null: all): the gated layers the token exports, the others skipped as the reference
// service skips them (src/dg_service.cpp:269-365).
int refdg_token_run(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred, uint32_t n_pred,
                    const uint8_t* run, int32_t* table_out, uint64_t* counts) {
  auto* r = static_cast<RefDg*>(h);
  try {
    ts::DgCore& c = *r->core;
    const uint32_t G = c.gated();
    ++r->seq;
    std::vector<uint8_t> rv(G, 1);
    if (run) rv.assign(run, run + G);
    c.begin_token(r->seq, &rv);
    for (uint32_t g = 0; g < G; ++g) {
      if (!rv[g]) continue;
      uint32_t nx = g + 1;
      while (nx < G && !rv[nx]) ++nx;
      const uint32_t* x = ids + size_t(g) * n;
      uint64_t mask = 0;
      for (uint32_t i = 0; i < n; ++i)  // the export kernel: slot_of[unit_base[g] + id] < 0 at export time
        if (x[i] < c.units(g) && c.table()[c.key(g, x[i])] < 0) mask |= uint64_t(1) << i;
      c.serve_demand(g, x, n, mask);
      c.serve_use(g, x, n, mask);
      if (n_pred && g + 1 < G && rv[g + 1]) c.serve_prediction(g + 1, pred + size_t(g) * n_pred, n_pred, n, false);
      if (c.deferred() && nx < G) c.issue_writebacks(g, nullptr);
      c.score_layer(g);  // the service closes each layer after its write-back slice (nothing when not scored)
    }
    c.end_token(r->keep, r->rows);
    c.check();
    std::memcpy(table_out, c.table().data(), 4ull * c.keys());
    const ts::DgStats& s = c.stats();
    const uint64_t v[] = {s.tokens,        s.lookups,       s.misses,         s.covered,      s.fetched,
                          s.prefetched,    s.prefetch_used, s.pred_invalid,   s.resurrected,  s.bank_serves,
                          s.evicted,       s.evict_short,   s.writebacks_done, s.predicted,   s.predicted_true,
                          s.miss_layers,   s.covered_waits, s.wb_deferred,    s.wb_cancelled, s.wb_forced,
                          s.wb_boundary_flushed, s.wb_issued_bytes, s.wb_cancelled_bytes, s.inclusive_kept,
                          s.inclusive_drops, uint64_t(c.free_slots()), uint64_t(c.free_blocks()),
                          uint64_t(c.on_device()), uint64_t(c.backed_units()), s.disk_reads, s.disk_drops,
                          s.disk_discards, s.clean_drops, uint64_t(c.file_units()), s.score_fallbacks,
                          s.scored_victims, s.score_layers, s.score_candidates, s.score_saturated, s.bank_kept,
                          s.bank_keep_drops, s.bank_keep_rereads, s.landing_issued, s.landing_promoted,
                          s.landing_expired, s.landing_expired_layer, s.landing_dropped_full,
                          s.landing_skipped_passed, s.landing_read_bytes, uint64_t(c.landing_units()),
                          uint64_t(c.landing_free()), s.landing_late, s.landing_cancelled, s.landing_failed};
    std::memcpy(counts, v, sizeof v);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_token: %s\n", e.what());
    return 1;
  }
}

const char* refdg_counter_names() {
  return "tokens lookups misses covered fetched prefetched prefetch_used pred_invalid resurrected bank_serves evicted "
         "evict_short writebacks_done predicted predicted_true miss_layers covered_waits wb_deferred wb_cancelled "
         "wb_forced wb_boundary_flushed wb_issued_bytes wb_cancelled_bytes inclusive_kept inclusive_drops free_slots "
         "free_blocks on_device backed_units disk_reads disk_drops disk_discards clean_drops file_units "
         "score_fallbacks scored_victims score_layers score_candidates score_saturated bank_kept bank_keep_drops "
         "bank_keep_rereads landing_issued landing_promoted landing_expired landing_expired_layer "
         "landing_dropped_full landing_skipped_passed landing_read_bytes landing_units landing_free landing_late "
         "landing_cancelled landing_failed";
}

// The device keys in recency order, most recent first.
uint32_t refdg_residency(void* h, uint32_t* out, uint32_t cap) {
  auto* r = static_cast<RefDg*>(h);
  const std::vector<uint32_t> v = r->core->residency();
  for (uint32_t i = 0; i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

// Landings: per landing block the key it holds (0xFFFFFFFF: none).
uint32_t refdg_land_owner(void* h, uint32_t* out, uint32_t cap) {
  const auto& v = static_cast<RefDg*>(h)->core->land_owner_;
  for (uint32_t i = 0; i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

// Three-tier: the pinned homes in recency order, most recently homed first.
uint32_t refdg_host_order(void* h, uint32_t* out, uint32_t cap) {
  auto* r = static_cast<RefDg*>(h);
  const std::vector<uint32_t> v = r->core->host_order();
  for (uint32_t i = 0; i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

// ss_dg_keep of every gated layer, concatenated (the reference context passes DgSteps::all_kept() to end_token).
int refdg_set_keep(void* h, const uint32_t* keys, uint32_t n) {
  static_cast<RefDg*>(h)->keep.assign(keys, keys + n);
  return 0;
}

// ss_dg_set_sched's write-back deferral (the reference context calls DgCore::set_wb_defer between tokens).
int refdg_set_wb_defer(void* h, uint32_t on) {
  try {
    static_cast<RefDg*>(h)->core->set_wb_defer(on != 0);
    static_cast<RefDg*>(h)->core->check();
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_set_wb_defer: %s\n", e.what());
    return 1;
  }
}

// The slot table now (after open: the seeded placement, before any token).
uint32_t refdg_table(void* h, int32_t* out, uint32_t cap) {
  const auto& t = static_cast<RefDg*>(h)->core->table();
  for (uint32_t i = 0; i < cap && i < t.size(); ++i) out[i] = t[i];
  return uint32_t(t.size());
}

// ss_dg_set_budgets between tokens (the reference context: src/dg_ctx.cpp:892-899).
int refdg_set_budgets(void* h, uint32_t spare_target, uint32_t per_layer, uint32_t per_token) {
  try {
    ts::DgCore& c = *static_cast<RefDg*>(h)->core;
    c.set_spare_target(spare_target);
    c.set_prefetch_budget(per_layer, per_token);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_set_budgets: %s\n", e.what());
    return 1;
  }
}

// ss_dg_set_clean_evict between tokens (the reference context: src/dg_ctx.cpp:595-605).
int refdg_set_clean_evict(void* h, uint32_t on) {
  try {
    static_cast<RefDg*>(h)->core->set_clean_evict(on != 0);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_set_clean_evict: %s\n", e.what());
    return 1;
  }
}

void refdg_close(void* h) { delete static_cast<RefDg*>(h); }

}  // extern "C"

// ---- the device-gated layout -------------------------------------------------------------------------------------------

extern "C" {

// The reference's dg_layout over a descriptor, a budget, the plan (tiers, one per unit; null: plan_make) and the
// options. Returns the refusal's status (0 = laid out); out[0..22]: keys, G, R, D, B, P, F, Q, I, S, disk_queue,
// persistent_slots, slots, guard_slot, blocks, scored, w_trans, w_freq, w_rec, L, landing_queued, landing_ttl,
// landing_chunk; residents: the tier-R keys.
int ref_dg_layout(const char* desc_json, size_t len, const ss_budget* b, const uint8_t* tiers, size_t n_tiers,
                  const ss_options* o, uint32_t* out, uint32_t* residents, uint32_t res_cap, char* err, size_t err_cap) {
  try {
    const ts::Desc d = ts::desc_from_json(ts::json_parse(std::string(desc_json, len)));
    const ts::Plan p = tiers ? ts::plan_from_tiers(d, *b, std::vector<uint8_t>(tiers, tiers + n_tiers))
                             : ts::plan_make(d, *b, {});
    const ts::DgLayout x = ts::dg_layout(d, p, *o);
    const uint32_t v[] = {x.keys, uint32_t(x.gated.size()), x.R, x.D, x.B, x.P, x.F, x.Q, x.I, x.S, x.disk_queue,
                          x.persistent_slots, x.slots, x.guard_slot, x.blocks, uint32_t(x.scored), x.w_trans,
                          x.w_freq, x.w_rec, x.L, x.landing_queued, x.landing_ttl, x.landing_chunk};
    std::memcpy(out, v, sizeof v);
    for (uint32_t i = 0; i < res_cap && i < x.residents.size(); ++i) residents[i] = x.residents[i];
    return 0;
  } catch (const ts::Error& e) {
    std::snprintf(err, err_cap, "%s", e.what());
    return int(e.status());
  }
}

}  // extern "C"

// ---- the CPU baseline -----------------------------------------------------------------------------------------------
// The reference DgCore on a transport shaped like the reference CPU backend (src/backend_cpu.cpp:20-59: host memory
// stands in for the device, copies are synchronous memcpy), plus a host XXH64 of every landed unit (src/xxh64.cpp), the
// CPU counterpart of the device verify. The "device" is one anonymous array per part (slots x part bytes); every host
// block is anonymous memory of one unit stride, filled from the source file before timing.
namespace {

void* map_anon(uint64_t bytes) {
  void* p = ::mmap(nullptr, size_t(bytes), PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
  if (p == MAP_FAILED) throw std::runtime_error("mmap of " + std::to_string(bytes) + " bytes failed");
  return p;
}

class Memcpy final : public ts::DgTransport {
 public:
  // blocks: the pinned homes and spares, then (three tiers) the staging buffers; block -1 is a one-unit buffer
  Memcpy(std::vector<uint64_t> parts, uint64_t host_stride, uint32_t slots, uint32_t blocks)
      : parts_(std::move(parts)), stride_(host_stride), slots_(slots), blk_(size_t(blocks) + 1, nullptr) {
    uint64_t off = 0;
    for (uint64_t pb : parts_) {
      off_.push_back(off);
      off += pb;
      arena_.push_back(static_cast<char*>(map_anon(pb * slots)));
    }
    unit_ = off;
    for (auto& b : blk_) b = static_cast<char*>(map_anon(stride_));
  }
  ~Memcpy() override {
    for (size_t p = 0; p < parts_.size(); ++p) ::munmap(arena_[p], size_t(parts_[p] * slots_));
    for (char* b : blk_) ::munmap(b, size_t(stride_));
  }
  char* slot(uint32_t p, int32_t s) const { return arena_[p] + uint64_t(s) * parts_[p]; }
  char* block(int32_t b) const { return blk_[size_t(b + 1)]; }  // block -1: the one-unit staging buffer
  uint64_t part_offset(uint32_t p) const { return off_[p]; }

  void h2d(Stream, int32_t s, int32_t b) override {
    for (uint32_t p = 0; p < parts_.size(); ++p) std::memcpy(slot(p, s), block(b) + off_[p], parts_[p]);
  }
  void d2h(int32_t s, int32_t b) override {
    for (uint32_t p = 0; p < parts_.size(); ++p) std::memcpy(block(b) + off_[p], slot(p, s), parts_[p]);
  }
  void d2d(int32_t a, int32_t b) override {
    for (uint32_t p = 0; p < parts_.size(); ++p) std::memcpy(slot(p, b), slot(p, a), parts_[p]);
  }
  void h2h(int32_t a, int32_t b) override { std::memcpy(block(b), block(a), unit_); }
  void d2h_part(Stream, int32_t s, int32_t b, uint32_t p) override {
    std::memcpy(block(b) + off_[p], slot(p, s), parts_[p]);
  }
  uint32_t parts() const override { return uint32_t(parts_.size()); }
  uint64_t part_bytes(uint32_t p) const override { return parts_[p]; }
  void write_entry(Stream, uint32_t, int32_t) override {}
  void signal_ready(uint32_t, uint32_t) override {}
  void* event_create() override { return new int(0); }
  void event_destroy(void* ev) override { delete static_cast<int*>(ev); }
  void record(void*, Stream) override {}
  void wait(Stream, void*) override {}
  bool done(void*) override { return true; }
  void event_sync(void*) override {}
  void sync(Stream) override {}
  void upload_table(const int32_t*, uint32_t) override {}
  void upload_table_ranges(const int32_t*, const uint32_t*, uint32_t) override {}
  // three tiers: a file-tier unit's bytes from its file into a staging buffer (as the reference reads them: one
  // positional read of the unit, direct I/O where the file system allows it)
  std::function<void(uint32_t, char*)> reader;
  void read_unit(uint32_t key, int32_t b) override { reader(key, block(b)); }

 private:
  std::vector<uint64_t> parts_, off_;
  uint64_t stride_, unit_ = 0;
  uint32_t slots_;
  std::vector<char*> arena_, blk_;
};

// Runs `work(i)` for i in [0, n) on `threads` threads.
template <class F>
void parallel_for(uint32_t n, int threads, F work) {
  std::atomic<uint32_t> next{0};
  std::vector<std::thread> th;
  for (int t = 0; t < std::max(1, threads); ++t)
    th.emplace_back([&] {
      for (uint32_t i; (i = next.fetch_add(1)) < n;) work(i);
    });
  for (auto& t : th) t.join();
}

}  // namespace

extern "C" {

// The CPU baseline over n_warm + n_tokens tokens of ids [n_warm + n_tokens][G][n]: the same placement as refdg_open,
// then per token begin_token, per gated layer the export mask, serve_demand (synchronous memcpy of every miss), a host
// XXH64 of every landed unit against hashes[key], serve_use, issue_writebacks and score_layer (the reference service's
// close of each exported layer, the last one included), and end_token, on the calling thread. The first n_warm tokens
// run untimed (the placement the timed tokens start from is the one after warmup, as on the device); token_ms[t] = the
// wall time of timed token t. policy: 0 LRU, 1 SCORED, 2 SCORED_AUTO (weights 700 / 200 / 100, no profile). The
// source file holds unit `key` at unit_offset[key] (unit bytes contiguous). out[10], sums over the timed tokens:
// misses, fetched, evicted, writebacks_done, hash mismatches, bytes copied into slots, file reads, drops of pinned
// units to their file, score_layers, score_candidates.
// Three-tier variant: n_paths source files, key k in paths[path_of[k]] at unit_offset[k]; disk[k] = 1 for the
// file-tier keys, home_blocks = the pinned homes, disk_staging buffers; reads are synchronous (one at a time inside
// their fetch: dg_disk_queue 1).
int refdg_cpu_baseline_disk(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                            uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                            uint32_t n_parts, uint64_t host_stride, const uint32_t* order, uint32_t n_order,
                            const char* const* paths, uint32_t n_paths, const uint32_t* path_of,
                            const uint64_t* unit_offset, const uint64_t* hashes, const uint32_t* ids, uint32_t n,
                            uint32_t n_tokens, int setup_threads, const uint8_t* disk, uint32_t home_blocks,
                            uint32_t disk_staging, uint32_t clean_evict, double* token_ms, uint64_t* out,
                            uint32_t n_warm, uint32_t policy);

int refdg_cpu_baseline(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                       uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                       uint32_t n_parts, uint64_t host_stride, const uint32_t* order, uint32_t n_order,
                       const char* path, const uint64_t* unit_offset, const uint64_t* hashes, const uint32_t* ids,
                       uint32_t n, uint32_t n_tokens, int setup_threads, double* token_ms, uint64_t* out,
                       uint32_t n_warm, uint32_t policy) {
  uint32_t keys = 0;
  for (uint32_t g = 0; g < G; ++g) keys += n_units[g];
  const std::vector<uint32_t> path_of(keys, 0);
  return refdg_cpu_baseline_disk(n_units, G, persistent, bank, blocks, spare_target, wb_defer, inclusive, part_bytes,
                                 n_parts, host_stride, order, n_order, &path, 1, path_of.data(), unit_offset, hashes,
                                 ids, n, n_tokens, setup_threads, nullptr, 0, 0, 0, token_ms, out, n_warm, policy);
}

int refdg_cpu_baseline_disk(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                            uint32_t spare_target, uint32_t wb_defer, uint32_t inclusive, const uint64_t* part_bytes,
                            uint32_t n_parts, uint64_t host_stride, const uint32_t* order, uint32_t n_order,
                            const char* const* paths, uint32_t n_paths, const uint32_t* path_of,
                            const uint64_t* unit_offset, const uint64_t* hashes, const uint32_t* ids, uint32_t n,
                            uint32_t n_tokens, int setup_threads, const uint8_t* disk, uint32_t home_blocks,
                            uint32_t disk_staging, uint32_t clean_evict, double* token_ms, uint64_t* out,
                            uint32_t n_warm, uint32_t policy) {
  std::vector<int> fds, dfds;
  auto close_all = [&] {
    for (int f : fds) ::close(f);
    for (int f : dfds)
      if (f >= 0) ::close(f);
  };
  try {
    const std::vector<uint64_t> parts(part_bytes, part_bytes + n_parts);
    uint64_t unit = 0;
    for (uint64_t pb : parts) unit += pb;
    const uint32_t slots = persistent + 2 * bank + 1;
    Memcpy t(parts, host_stride, slots, blocks + (disk ? disk_staging : 0));
    for (uint32_t i = 0; i < n_paths; ++i) {
      const int fd = ::open(paths[i], O_RDONLY | O_CLOEXEC);
      if (fd < 0) throw std::runtime_error(std::string("open ") + paths[i]);
      fds.push_back(fd);
      dfds.push_back(::open(paths[i], O_RDONLY | O_CLOEXEC | O_DIRECT));  // -1: buffered reads
    }
    auto pread_all = [](int fd, char* dst, uint64_t bytes, uint64_t off) {
      uint64_t got = 0;
      while (got < bytes) {
        const ssize_t r = ::pread(fd, dst + got, size_t(bytes - got), off_t(off + got));
        if (r <= 0) return false;
        got += uint64_t(r);
      }
      return true;
    };
    const bool aligned = unit % 4096 == 0;
    t.reader = [&](uint32_t k, char* dst) {
      const int dfd = dfds[path_of[k]];
      const bool direct = dfd >= 0 && aligned && unit_offset[k] % 4096 == 0;
      if (!pread_all(direct ? dfd : fds[path_of[k]], dst, unit, unit_offset[k]))
        throw std::runtime_error("short read of a file-tier unit");
    };
    ts::DgConfig c;
    c.n_units.assign(n_units, n_units + G);
    c.persistent_slots = persistent;
    c.bank_slots = bank;
    c.blocks = blocks;
    c.spare_target = spare_target;
    c.prefetch_reserve = std::min<uint32_t>(24, spare_target / 4);
    c.prefetch_per_layer = 4;
    c.prefetch_per_token = 48;
    c.wb_defer = wb_defer != 0;
    c.inclusive = inclusive;
    c.max_ids = bank;
    c.pf_legacy = true;
    if (policy) {
      c.scored = true;
      c.scored_auto = policy == 2;
      c.boundary_score = true;
    }
    uint32_t n_keys = 0;
    for (uint32_t g = 0; g < G; ++g) n_keys += n_units[g];
    std::vector<uint8_t> dflags;
    if (disk) {
      c.disk_tier = true;
      c.home_blocks = home_blocks;
      c.disk_staging = disk_staging;
      c.disk_queue = 1;
      c.clean_evict = clean_evict != 0;
      dflags.assign(disk, disk + n_keys);
    }
    ts::DgCore core(c, &t);
    core.place(std::vector<uint32_t>(order, order + n_order), disk ? &dflags : nullptr);
    // fill: every key's bytes into its home (a slot or a block), from the file; spare blocks and free slots touched
    const uint32_t keys = core.keys();
    std::atomic<int> io_err{0};
    parallel_for(keys, setup_threads, [&](uint32_t k) {
      std::vector<char> buf;
      const int32_t s = core.table()[k];
      const int32_t b = core.block_of(k);
      char* dst = b >= 0 ? t.block(b) : nullptr;
      if (s >= 0) {
        buf.resize(size_t(unit));
        dst = buf.data();
      }
      if (!dst) return;
      if (!pread_all(fds[path_of[k]], dst, unit, unit_offset[k])) {
        io_err = 1;
        return;
      }
      if (s >= 0)
        for (uint32_t p = 0; p < n_parts; ++p) std::memcpy(t.slot(p, s), dst + t.part_offset(p), parts[p]);
    });
    if (io_err) throw std::runtime_error("short read of a source file at the fill");
    std::vector<uint8_t> used_slot(slots, 0);
    for (uint32_t k = 0; k < keys; ++k)
      if (core.table()[k] >= 0) used_slot[size_t(core.table()[k])] = 1;
    const uint32_t all_blocks = blocks + (disk ? disk_staging : 0);
    std::vector<int32_t> used_block(size_t(all_blocks) + 1, 0);
    for (uint32_t k = 0; k < keys; ++k)
      if (core.block_of(k) >= 0) used_block[size_t(core.block_of(k)) + 1] = 1;
    parallel_for(slots, setup_threads, [&](uint32_t s) {
      if (!used_slot[s])
        for (uint32_t p = 0; p < n_parts; ++p) std::memset(t.slot(p, int32_t(s)), 0, parts[p]);
    });
    parallel_for(all_blocks + 1, setup_threads, [&](uint32_t b) {
      if (!used_block[b]) std::memset(t.block(int32_t(b) - 1), 0, host_stride);
    });
    // the warmup tokens (untimed), then the timed ones
    ts::DgStats s0 = core.stats();
    uint64_t bad = 0, copied = 0;
    for (uint32_t tok = 0; tok < n_warm + n_tokens; ++tok) {
      if (tok == n_warm) {
        s0 = core.stats();
        bad = copied = 0;
      }
      const auto t0 = std::chrono::steady_clock::now();
      core.begin_token(tok + 1);
      for (uint32_t g = 0; g < G; ++g) {
        const uint32_t* x = ids + (size_t(tok) * G + g) * n;
        uint64_t mask = 0;
        for (uint32_t i = 0; i < n; ++i)
          if (x[i] < core.units(g) && core.table()[core.key(g, x[i])] < 0) mask |= uint64_t(1) << i;
        core.serve_demand(g, x, n, mask);
        for (uint32_t i = 0; i < n; ++i) {
          if (!(mask >> i & 1u)) continue;
          const uint32_t k = core.key(g, x[i]);
          const int32_t s = core.table()[k];
          ts::Xxh64 h;
          for (uint32_t p = 0; p < n_parts; ++p) h.update(t.slot(p, s), size_t(parts[p]));
          bad += h.digest() != hashes[k];
          copied += unit;
        }
        core.serve_use(g, x, n, mask);
        if (core.deferred() && g + 1 < G) core.issue_writebacks(g, nullptr);
        core.score_layer(g);  // (nothing under LRU)
      }
      core.end_token({}, 1);
      if (tok >= n_warm)
        token_ms[tok - n_warm] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    }
    const ts::DgStats& s1 = core.stats();
    out[0] = s1.misses - s0.misses;
    out[1] = s1.fetched - s0.fetched;
    out[2] = s1.evicted - s0.evicted;
    out[3] = s1.writebacks_done - s0.writebacks_done;
    out[4] = bad;
    out[5] = copied;
    out[6] = s1.disk_reads - s0.disk_reads;
    out[7] = s1.disk_drops - s0.disk_drops;
    out[8] = s1.score_layers - s0.score_layers;
    out[9] = s1.score_candidates - s0.score_candidates;
    close_all();
    return 0;
  } catch (const std::exception& e) {
    close_all();
    std::fprintf(stderr, "refdg_cpu_baseline: %s\n", e.what());
    return 1;
  }
}

}  // extern "C"

// The reference's read-depth controller (DgDepthCtl) fed n busy periods; outputs as tsa_test_depth_ctl.
extern "C" int refdg_depth_ctl(uint32_t bound, uint32_t n, const uint64_t* reads, const uint64_t* bytes,
                               const uint64_t* ns, uint32_t* depth, uint64_t* counters, double* recent,
                               uint32_t* n_recent) {
  try {
    ts::DgDepthCtl c(bound);
    for (uint32_t i = 0; i < n; ++i) depth[i] = c.on_busy(reads[i], bytes[i], ns[i]);
    const uint64_t v[] = {c.changes, c.calibrations, c.windows, c.decisions(), c.reads1, c.bytes1, c.ns1,
                          c.readsu, c.bytesu, c.nsu, c.depth(), c.bound(), uint64_t(c.calibrating())};
    std::memcpy(counters, v, sizeof v);
    uint32_t k = 0;
    for (const ts::DgDepthCtl::Decision& d : c.ring()) {
      const double r[] = {double(d.seq), double(d.reads), double(d.from), double(d.to), d.rate_u, d.rate_1,
                          double(int(d.reason))};
      std::memcpy(recent + 7 * k++, r, sizeof r);
    }
    *n_recent = k;
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_depth_ctl: %s\n", e.what());
    return 1;
  }
}
