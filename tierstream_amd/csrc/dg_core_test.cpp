// Test hooks over the device-gated cache state machine alone (include/tierstream_amd/tsa_test.h, tsa_test_dgcore_*):
// this library's DgCore on an eager transport, the schedule the reference's CPU tests run its core on
// (reference tests/test_dg.cpp:201), so placement compares with the reference core's token by token without a GPU.
#include <algorithm>
#include <cstring>
#include <memory>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"
#include "dg_core.hpp"
#include "depth_ctl.hpp"
#include "score_profile.hpp"
#include "sha256.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {
namespace {

// Every copy, entry write, event and file read completes when issued. With check_order on, the transport also keeps
// the copies as a device would run them - each stream in order, streams ordered only by the waits the core asks for and
// by the protocol (a layer's export is served only after the engine passed the previous ready word, which followed that
// layer's copies on the demand stream) - and fails the token at the first call whose memory could still be in use by a
// copy not ordered before it: a file read
// into a block (the host writes it at once) while any copy reads or writes that block and the host has not waited for
// it; a copy in (block -> slot) while a copy still writes the block or reads or writes the slot; a copy out (slot ->
// block, at once or prestaged) while a copy still writes the slot or reads or writes the block.
class EagerTransport final : public DgTransport {
 public:
  explicit EagerTransport(std::vector<uint64_t> parts) : parts_(std::move(parts)) {}
  ~EagerTransport() override = default;
  void h2d(Stream s, int32_t slot, int32_t block, uint32_t) override { copy(s, block, -1 - slot, "copy in"); }
  void d2h(int32_t slot, int32_t block) override { copy(kD2h, -1 - slot, block, "write-back"); }
  void d2h_part(Stream s, int32_t slot, int32_t block, uint32_t) override {
    if (staged_.count({slot, block})) return;  // (copied at the boundary already)
    copy(s, -1 - slot, block, "write-back part");
  }
  void prestage(int32_t slot, int32_t block) override {
    copy(kD2h, -1 - slot, block, "prestaged write-back");
    staged_.insert({slot, block});
  }
  void unqueue(int32_t slot, int32_t block) override { staged_.erase({slot, block}); }
  uint32_t parts() const override { return uint32_t(parts_.size()); }
  uint64_t part_bytes(uint32_t p) const override { return parts_[p]; }
  void write_entry(Stream, uint32_t, int32_t) override {}
  void signal_ready(uint32_t, uint32_t) override {
    for (int t = 0; t < 3; ++t) ready_cover_[t] = t == kDem ? last_[kDem] : seen_[kDem][t];
  }
  // A layer's export is served: the engine passed every earlier ready word, so their copies have ended.
  void layer_begins() {
    for (int t = 0; t < 3; ++t) host_[t] = std::max(host_[t], ready_cover_[t]);
  }
  void* event_create() override { return new Ev(); }
  void event_destroy(void* ev) override { delete static_cast<Ev*>(ev); }
  void record(void* ev, Stream s) override {
    Ev& e = *static_cast<Ev*>(ev);
    for (int t = 0; t < 3; ++t) e.cover[t] = t == s ? last_[s] : seen_[s][t];
  }
  void wait(Stream s, void* ev) override { after(s, *static_cast<Ev*>(ev)); }
  bool done(void* ev) override {
    host(*static_cast<Ev*>(ev));
    return true;
  }
  bool query(void* ev) override { return done(ev); }
  void event_sync(void* ev) override { host(*static_cast<Ev*>(ev)); }
  void sync(Stream s) override {
    host_[s] = last_[s];
    for (int t = 0; t < 3; ++t) host_[t] = std::max(host_[t], seen_[s][t]);
  }
  void upload_table(const int32_t*, uint32_t) override {}
  void read_unit(uint32_t key, int32_t block, int32_t) override {
    if (!check_) return;
    for (const Copy& c : copies_)
      if ((c.from == block || c.to == block) && host_[c.s] < c.id)
        fail("a file read of key " + std::to_string(key) + " into block " + std::to_string(block) + " while " +
             c.what + " " + std::to_string(c.id) + " (" + where(c.from) + " -> " + where(c.to) + ", stream " +
             std::to_string(c.s) + ") may still use it");
  }
  // As the MI355X transport: a landing read first waits on the host for the block's last copy out.
  void read_landing(uint32_t key, int32_t block) override {
    for (const Copy& c : copies_)
      if (c.from == block) host_[c.s] = std::max(host_[c.s], c.id);
    read_unit(key, block, -1);
  }
  void wait_copy_in(Stream s, int32_t, int32_t, void* slot_ev, void* block_ev) override {
    if (slot_ev) wait(s, slot_ev);
    if (block_ev) wait(s, block_ev);
  }
  void check_order(bool on) { check_ = on; }
  const std::string& violation() const { return violation_; }

 private:
  // A copy: from / to as block b (>= 0) or slot s (encoded -1 - s), on stream s, id in issue order.
  struct Copy {
    int s;
    int32_t from, to;
    uint64_t id;
    std::string what;
  };
  struct Ev {
    uint64_t cover[3] = {0, 0, 0};  // per stream: the last copy id the event's completion implies
  };
  bool before(const Copy& c, int s) const { return c.s == s || seen_[s][c.s] >= c.id || host_[c.s] >= c.id; }
  void after(int s, const Ev& e) {
    for (int t = 0; t < 3; ++t) seen_[s][t] = std::max(seen_[s][t], e.cover[t]);
  }
  void host(const Ev& e) {
    for (int t = 0; t < 3; ++t) host_[t] = std::max(host_[t], e.cover[t]);
  }
  void copy(int s, int32_t from, int32_t to, const char* what) {
    if (check_)
      for (const Copy& c : copies_) {
        const bool clash = c.to == to || c.to == from || c.from == to;  // (two reads of one place do not clash)
        if (clash && !before(c, s))
          fail(std::string(what) + " (" + where(from) + " -> " + where(to) + ") on stream " + std::to_string(s) +
               " while " + c.what + " " + std::to_string(c.id) + " (" + where(c.from) + " -> " + where(c.to) +
               ", stream " + std::to_string(c.s) + ") may still run");
      }
    copies_.push_back(Copy{s, from, to, ++next_, what});
    last_[s] = next_;
  }
  static std::string where(int32_t x) { return x >= 0 ? "block " + std::to_string(x) : "slot " + std::to_string(-1 - x); }
  void fail(const std::string& why) {
    if (violation_.empty()) violation_ = why;
  }

  std::vector<uint64_t> parts_;
  bool check_ = false;
  std::string violation_;
  std::vector<Copy> copies_;
  std::set<std::pair<int32_t, int32_t>> staged_;
  uint64_t next_ = 0, last_[3] = {0, 0, 0}, host_[3] = {0, 0, 0}, seen_[3][3] = {}, ready_cover_[3] = {0, 0, 0};
};

struct TestCore {
  std::unique_ptr<EagerTransport> t;
  std::unique_ptr<DgCore> core;
  uint32_t seq = 0, rows = 1;
  std::vector<uint32_t> keep;  // the boundary's keep list (ss_dg_keep of every gated layer)
};

constexpr const char* kNames =
    "tokens lookups misses covered fetched prefetched prefetch_used resurrected bank_serves evicted evict_short "
    "writebacks_done miss_layers covered_waits wb_deferred wb_cancelled wb_forced wb_boundary_flushed wb_issued_bytes "
    "wb_cancelled_bytes inclusive_kept inclusive_drops free_slots free_blocks on_device backed_units disk_reads "
    "disk_drops disk_discards clean_drops file_units score_fallbacks scored_victims score_layers score_candidates "
    "score_saturated pred_invalid predicted predicted_true bank_kept bank_keep_drops bank_keep_rereads "
    "landing_issued landing_promoted landing_expired landing_expired_layer landing_dropped_full "
    "landing_skipped_passed landing_read_bytes landing_units landing_free";

}  // namespace
}  // namespace tsa

extern "C" {

ss_status tsa_test_dgcore_open(const tsa_test_dgcore_config* cfg, const uint32_t* order, uint32_t n_order,
                               void** out) {
  return tsa::guard([&] {
    using namespace tsa;
    require(cfg && out && cfg->n_units && cfg->part_bytes && (order || n_order == 0), SS_E_INVALID,
            "tsa_test_dgcore_open: null argument");
    auto r = std::make_unique<TestCore>();
    r->t = std::make_unique<EagerTransport>(std::vector<uint64_t>(cfg->part_bytes, cfg->part_bytes + cfg->n_parts));
    DgConfig c;
    c.n_units.assign(cfg->n_units, cfg->n_units + cfg->n_gated);
    c.persistent_slots = cfg->persistent_slots;
    c.bank_slots = cfg->bank_slots;
    c.blocks = cfg->blocks;
    c.spare_target = cfg->spare_target;
    c.prefetch_reserve_auto = cfg->prefetch_reserve == 0xFFFFFFFFu;
    c.prefetch_reserve = c.prefetch_reserve_auto ? 0 : cfg->prefetch_reserve;
    c.prefetch_per_layer = cfg->prefetch_per_layer;
    c.prefetch_per_token = cfg->prefetch_per_token;
    c.wb_defer = cfg->wb_defer != 0;
    c.wb_on_d2h = cfg->wb_on_d2h != 0;
    c.inclusive = cfg->inclusive;
    c.disk_tier = cfg->disk_tier != 0;
    c.disk_prefetch = cfg->disk_prefetch != 0;
    c.home_blocks = cfg->home_blocks;
    c.disk_staging = cfg->disk_staging;
    c.clean_evict = cfg->clean_evict != 0;
    c.bank_keep = cfg->bank_keep;
    c.landing_blocks = cfg->landing_blocks;
    c.landing_ttl = cfg->landing_ttl;
    require(cfg->policy <= 2, SS_E_INVALID, "tsa_test_dgcore_open: policy must be 0, 1 or 2");
    c.scored = cfg->policy != 0;
    c.scored_auto = cfg->policy == 2;
    c.w_trans = cfg->w_trans;
    c.w_freq = cfg->w_freq;
    c.w_rec = cfg->w_rec;
    c.max_ids = cfg->bank_slots;
    r->rows = cfg->rows ? cfg->rows : 1;
    r->core = std::make_unique<DgCore>(c, r->t.get());
    std::vector<uint8_t> disk;
    if (c.disk_tier) {
      require(cfg->disk != nullptr, SS_E_INVALID, "tsa_test_dgcore_open: the disk tier needs its flags");
      disk.assign(cfg->disk, cfg->disk + r->core->keys());
    }
    r->core->seat(std::vector<uint32_t>(order, order + n_order), c.disk_tier ? &disk : nullptr);
    if (cfg->score_cells) {
      std::vector<unsigned char> le;
      uint64_t cells = 0;
      for (uint32_t g = 0; g < cfg->n_gated; ++g) cells += uint64_t(cfg->n_units[g]) * cfg->n_units[g];
      le.resize(4 * cells);
      for (uint64_t i = 0; i < cells; ++i)
        for (int b = 0; b < 4; ++b) le[4 * i + b] = (unsigned char)(cfg->score_cells[i] >> (8 * b));
      r->core->seed_transitions(le.data());
    }
    r->core->audit();
    *out = r.release();
  });
}

ss_status tsa_test_dgcore_token(void* h, const uint32_t* ids, uint32_t n, int32_t* table_out, uint64_t* counts,
                                uint32_t n_counts) {
  return tsa_test_dgcore_token_pred(h, ids, n, nullptr, 0, nullptr, table_out, counts, n_counts);
}

ss_status tsa_test_dgcore_token_run(void* h, const uint32_t* ids, uint32_t n, const uint8_t* run, int32_t* table_out,
                                    uint64_t* counts, uint32_t n_counts) {
  return tsa_test_dgcore_token_pred(h, ids, n, nullptr, 0, run, table_out, counts, n_counts);
}

ss_status tsa_test_dgcore_token_pred(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred, uint32_t n_pred,
                                     const uint8_t* run, int32_t* table_out, uint64_t* counts, uint32_t n_counts) {
  return tsa::guard([&] {
    using namespace tsa;
    require(h && ids && n >= 1 && n <= 64, SS_E_INVALID, "tsa_test_dgcore_token: bad argument");
    auto* r = static_cast<TestCore*>(h);
    DgCore& c = *r->core;
    const uint32_t G = c.gated();
    std::vector<uint8_t> rv(G, 1);
    if (run) rv.assign(run, run + G);
    c.open_token(++r->seq, &rv);
    for (uint32_t g = 0; g < G; ++g) {
      if (!rv[g]) continue;
      const uint32_t* x = ids + size_t(g) * n;
      uint64_t mask = 0;
      for (uint32_t i = 0; i < n; ++i)  // the export kernel: slot_of[unit_base[g] + id] < 0 at export time
        if (x[i] < c.units(g) && c.table()[c.key(g, x[i])] < 0) mask |= uint64_t(1) << i;
      r->t->layer_begins();
      c.serve_misses(g, x, n, mask);
      c.note_uses(g, x, n, mask);
      // the prediction for the next layer made at this one (the service serves it when that layer exports)
      if (pred && n_pred && g + 1 < G && rv[g + 1]) c.prefetch_next(g + 1, pred + size_t(g) * n_pred, n_pred);
      uint32_t nx = g + 1;  // the next exported layer: no slice after the token's last one
      while (nx < G && !rv[nx]) ++nx;
      if (c.queued_writebacks() && nx < G) c.spend_wb_credit(g);
    }
    c.close_token(r->rows, r->keep);
    c.audit();
    require(r->t->violation().empty(), SS_E_BACKEND, "copy order: " + r->t->violation());
    if (table_out) std::memcpy(table_out, c.table().data(), 4ull * c.keys());
    if (counts) {
      const DgCounts& s = c.counts();
      const uint64_t v[] = {s.tokens, s.lookups, s.misses, s.covered, s.fetched, s.prefetched, s.prefetch_used,
                            s.resurrected, s.bank_serves, s.evicted, s.evict_short, s.writebacks_done, s.miss_layers,
                            s.covered_waits, s.wb_deferred, s.wb_cancelled, s.wb_forced, s.wb_boundary_flushed,
                            s.wb_issued_bytes, s.wb_cancelled_bytes, s.inclusive_kept, s.inclusive_drops,
                            uint64_t(c.free_slots()), uint64_t(c.free_blocks()), uint64_t(c.on_device()),
                            uint64_t(c.clean_copies()), s.disk_reads, s.disk_drops, s.disk_discards, s.clean_drops,
                            uint64_t(c.file_units()), s.score_fallbacks, s.scored_victims, s.score_layers,
                            s.score_candidates, s.score_saturated, s.pred_invalid, s.predicted, s.predicted_true,
                            s.bank_kept, s.bank_keep_drops, s.bank_keep_rereads, s.landing_issued,
                            s.landing_promoted, s.landing_expired, s.landing_expired_layer, s.landing_dropped_full,
                            s.landing_skipped_passed, s.landing_read_bytes, uint64_t(c.landing_units()),
                            uint64_t(c.landing_free())};
      const uint32_t m = uint32_t(sizeof v / sizeof v[0]);
      std::memcpy(counts, v, 8ull * (n_counts < m ? n_counts : m));
    }
  });
}

const char* tsa_test_dgcore_counter_names(void) { return tsa::kNames; }

ss_status tsa_test_dgcore_set_policy(void* h, uint32_t policy) {
  return tsa::guard([&] {
    tsa::require(h != nullptr, SS_E_INVALID, "tsa_test_dgcore_set_policy: null handle");
    auto* r = static_cast<tsa::TestCore*>(h);
    r->core->set_policy(policy);
    r->core->audit();
  });
}

ss_status tsa_test_dgcore_check_order(void* h, int on) {
  return tsa::guard([&] {
    tsa::require(h != nullptr, SS_E_INVALID, "tsa_test_dgcore_check_order: null handle");
    static_cast<tsa::TestCore*>(h)->t->check_order(on != 0);
  });
}

ss_status tsa_test_dgcore_set_keep(void* h, const uint32_t* keys, uint32_t n) {
  return tsa::guard([&] {
    tsa::require(h != nullptr && (keys || n == 0), SS_E_INVALID, "tsa_test_dgcore_set_keep: null argument");
    static_cast<tsa::TestCore*>(h)->keep.assign(keys, keys + n);
  });
}

ss_status tsa_test_dgcore_set_wb_defer(void* h, uint32_t on) {
  return tsa::guard([&] {
    tsa::require(h != nullptr, SS_E_INVALID, "tsa_test_dgcore_set_wb_defer: null handle");
    auto* r = static_cast<tsa::TestCore*>(h);
    r->core->defer_writebacks(on != 0);
    r->core->audit();
  });
}

ss_status tsa_test_sha256(const void* data, uint64_t n, unsigned char* out) {
  return tsa::guard([&] {
    tsa::require((data || n == 0) && out, SS_E_INVALID, "tsa_test_sha256: null argument");
    const std::string d = tsa::sha256(data ? data : "", size_t(n));
    std::memcpy(out, d.data(), 32);
  });
}

ss_status tsa_test_score_profile_check(const void* data, uint64_t len, const uint32_t* units, uint32_t n_gated,
                                       const unsigned char* identity, char* prov, uint32_t prov_cap) {
  return tsa::guard([&] {
    tsa::require((units || n_gated == 0) && identity, SS_E_INVALID, "tsa_test_score_profile_check: null argument");
    const tsa::ScoreProfile v = tsa::check_score_profile(
        data, len, std::vector<uint32_t>(units, units + n_gated),
        std::string(reinterpret_cast<const char*>(identity), 32));
    if (prov && prov_cap) {
      const size_t n = std::min<size_t>(v.provenance.size(), prov_cap - 1);
      std::memcpy(prov, v.provenance.data(), n);
      prov[n] = '\0';
    }
  });
}

uint32_t tsa_test_dgcore_host_order(void* h, uint32_t* out, uint32_t cap) {
  if (!h) return 0;
  const std::vector<uint32_t> v = static_cast<tsa::TestCore*>(h)->core->pinned_order();
  for (uint32_t i = 0; out && i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

uint32_t tsa_test_dgcore_land_owner(void* h, uint32_t* out, uint32_t cap) {
  if (!h) return 0;
  const std::vector<uint32_t>& v = static_cast<tsa::TestCore*>(h)->core->landing_owners();
  for (uint32_t i = 0; out && i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

void tsa_test_dgcore_close(void* h) { delete static_cast<tsa::TestCore*>(h); }

}  // extern "C"

// ---- the read-depth controller alone ----------------------------------------------------------------------------------
// n busy periods (reads[i], bytes[i], ns[i]) fed in order: depth[i] = the depth after period i; counters[13] =
// changes, calibrations, windows, verdicts, reads_1, bytes_1, ns_1, reads_u, bytes_u, ns_u, depth, bound, calibrating;
// recent[16 * 7] = the last verdicts (seq, reads, from, to, gbps_u, gbps_1, why) as doubles; *n_recent their count.
extern "C" ss_status tsa_test_depth_ctl(uint32_t bound, uint32_t n, const uint64_t* reads, const uint64_t* bytes,
                                        const uint64_t* ns, uint32_t* depth, uint64_t* counters, double* recent,
                                        uint32_t* n_recent) {
  return tsa::guard([&] {
    tsa::require((n == 0 || (reads && bytes && ns && depth)) && counters && recent && n_recent, SS_E_INVALID,
                 "tsa_test_depth_ctl: null argument");
    tsa::ReadDepthController c(bound);
    for (uint32_t i = 0; i < n; ++i) depth[i] = c.feed(reads[i], bytes[i], ns[i]);
    const uint64_t v[] = {c.changes, c.calibrations, c.windows, c.verdicts(), c.reads_1, c.bytes_1, c.ns_1,
                          c.reads_u, c.bytes_u, c.ns_u, c.depth(), c.bound(), uint64_t(c.calibrating())};
    std::memcpy(counters, v, sizeof v);
    uint32_t k = 0;
    for (const tsa::ReadDepthController::Verdict& d : c.recent()) {
      const double r[] = {double(d.seq), double(d.reads), double(d.from), double(d.to), d.gbps_u, d.gbps_1,
                          double(int(d.why))};
      std::memcpy(recent + 7 * k++, r, sizeof r);
    }
    *n_recent = k;
  });
}
