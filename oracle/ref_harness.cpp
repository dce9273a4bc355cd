// ORACLE (test infrastructure only): a harness over the reference's own code, compiled with its sources in place by
// oracle/Makefile (target `ref`) into _ref/libtsref_harness.so. It never ships in the product.
//
//  * ref_region_of: where a host-contract table address of a reference CPU context points (layer pool + offset, or
//    stream ring class + offset), read from the reference Ctx's own fields, so tables compare "up to base offset".
//  * refdg_*: the reference DgCore (src/dg_core.cpp) driven exactly as its CPU tests drive it in eager mode
//    (tests/test_dg.cpp:201): a transport whose copies, entries and events complete at once (done() is always true)
//    and a service loop that never sees the device "ahead". Each token: begin_token, per gated layer the export mask
//    from the table as the device would read it, serve_demand, serve_use, issue_writebacks, then end_token.
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

#define private public
#define protected public
#include "dg_core.hpp"
#include "stream_ctx.hpp"
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

 private:
  std::vector<uint64_t> parts_;
};

struct RefDg {
  std::unique_ptr<Eager> t;
  std::unique_ptr<ts::DgCore> core;
  uint32_t seq = 0;
};

}  // namespace

extern "C" {

void* refdg_open(const uint32_t* n_units, uint32_t G, uint32_t persistent, uint32_t bank, uint32_t blocks,
                 uint32_t spare_target, uint32_t prefetch_reserve, uint32_t pf_layer, uint32_t pf_token,
                 uint32_t wb_defer, uint32_t wb_on_d2h, uint32_t inclusive, const uint64_t* part_bytes,
                 uint32_t n_parts, const uint32_t* order, uint32_t n_order) {
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
    r->core = std::make_unique<ts::DgCore>(c, r->t.get());
    r->core->place(std::vector<uint32_t>(order, order + n_order));
    return r;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "refdg_open: %s\n", e.what());
    return nullptr;
  }
}

// One token: ids [G][n] (every gated layer exported), pred [G][n_pred] (the prediction for layer g + 1 made at g;
// n_pred = 0: none). Writes the table after the boundary (keys int32) and the counters (see refdg_counter_names).
int refdg_token(void* h, const uint32_t* ids, uint32_t n, const uint32_t* pred, uint32_t n_pred, int32_t* table_out,
                uint64_t* counts) {
  auto* r = static_cast<RefDg*>(h);
  try {
    ts::DgCore& c = *r->core;
    const uint32_t G = c.gated();
    ++r->seq;
    c.begin_token(r->seq);
    for (uint32_t g = 0; g < G; ++g) {
      const uint32_t* x = ids + size_t(g) * n;
      uint64_t mask = 0;
      for (uint32_t i = 0; i < n; ++i)  // the export kernel: slot_of[unit_base[g] + id] < 0 at export time
        if (x[i] < c.units(g) && c.table()[c.key(g, x[i])] < 0) mask |= uint64_t(1) << i;
      c.serve_demand(g, x, n, mask);
      c.serve_use(g, x, n, mask);
      if (n_pred && g + 1 < G) c.serve_prediction(g + 1, pred + size_t(g) * n_pred, n_pred, n, false);
      if (c.deferred() && g + 1 < G) c.issue_writebacks(g, nullptr);
    }
    c.end_token({}, 1);
    c.check();
    std::memcpy(table_out, c.table().data(), 4ull * c.keys());
    const ts::DgStats& s = c.stats();
    const uint64_t v[] = {s.tokens,        s.lookups,       s.misses,         s.covered,      s.fetched,
                          s.prefetched,    s.prefetch_used, s.pred_invalid,   s.resurrected,  s.bank_serves,
                          s.evicted,       s.evict_short,   s.writebacks_done, s.predicted,   s.predicted_true,
                          s.miss_layers,   s.covered_waits, s.wb_deferred,    s.wb_cancelled, s.wb_forced,
                          s.wb_boundary_flushed, s.wb_issued_bytes, s.wb_cancelled_bytes, s.inclusive_kept,
                          s.inclusive_drops, uint64_t(c.free_slots()), uint64_t(c.free_blocks()),
                          uint64_t(c.on_device()), uint64_t(c.backed_units())};
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
         "free_blocks on_device backed_units";
}

// The device keys in recency order, most recent first.
uint32_t refdg_residency(void* h, uint32_t* out, uint32_t cap) {
  auto* r = static_cast<RefDg*>(h);
  const std::vector<uint32_t> v = r->core->residency();
  for (uint32_t i = 0; i < cap && i < v.size(); ++i) out[i] = v[i];
  return uint32_t(v.size());
}

void refdg_close(void* h) { delete static_cast<RefDg*>(h); }

}  // extern "C"
