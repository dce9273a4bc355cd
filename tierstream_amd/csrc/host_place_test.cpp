// Test hook over the host contract's placement alone (tsa_test_hostplace_run in tsa_test.h): HostPlacement driven by
// the engine's forward loop on a HostWork that does nothing and reports every copy as complete, so the tables, groups
// and counters can be compared with the reference CPU backend's on the CPU (the reference's own tests drive its
// runtime the same way: tests/test_runtime.cpp).
#include <cstring>
#include <vector>

#include "common.hpp"
#include "copy_runs.hpp"
#include "read_sched.hpp"
#include "host_place.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {
namespace {

class NoDevice final : public HostWork {
 public:
  void write_back(const WriteBackOrder&) override {}
  bool fetch(const FetchOrder&) override { return false; }
  void promote(int32_t) override {}
  void retire(int32_t) override {}
  bool settle(int32_t, bool) override { return true; }
};

}  // namespace
}  // namespace tsa

extern "C" {

ss_status tsa_test_hostplace_run(const char* desc_json, size_t len, const ss_budget* budget, const ss_options* opt,
                                 int steps, const int32_t* routes, const int32_t* prefetch, int max_ids, int mode,
                                 int max_units, int32_t* spot_kind, int32_t* spot_index, int32_t* group_of,
                                 ss_layer_stats* stats) {
  return tsa::guard([&] {
    using namespace tsa;
    require(desc_json && budget && opt && routes && steps >= 0 && max_ids > 0 && max_units > 0 && mode >= 0 &&
                mode <= 2,
            SS_E_INVALID, "tsa_test_hostplace_run: bad argument");
    const Desc d = desc_from_json(json_parse(std::string(desc_json, len)));
    const Plan p = plan_make(d, *budget, {});
    NoDevice dev;
    HostPlacement place(d, p, *opt);
    place.attach(&dev);
    place.place_residents();
    const int L = int(d.layers.size());
    std::vector<int32_t> ids(static_cast<size_t>(max_ids));
    for (int s = 0; s < steps; ++s) {
      place.begin(nullptr, 0);
      for (int l = 0; l < L; ++l) {
        const int nu = d.layers[size_t(l)].n_units;
        if (nu <= 0) continue;
        const int32_t* r = routes + (size_t(s) * L + l) * max_ids;
        int n = 0;
        while (n < max_ids && r[n] >= 0) ++n;
        if (mode == 1) place.routes_all(l);
        else place.routes(l, r, n);
        const HostPlacement::Acquire a = place.acquire(l, mode != 2);
        (void)a;
        const std::vector<DevSpot>& t = place.take_table(l);
        const size_t base = (size_t(s) * L + l) * max_units;
        for (int u = 0; u < nu && u < max_units; ++u) {
          spot_kind[base + u] = t[size_t(u)].kind;
          spot_index[base + u] = t[size_t(u)].index;
          group_of[base + u] = -1;
        }
        const auto& groups = place.groups(l);
        for (size_t gi = 0; gi < groups.size(); ++gi)
          for (int32_t u : groups[gi])
            if (u < max_units) group_of[base + size_t(u)] = int32_t(gi);
        // the next layer's prediction, made while this layer computes (CERTAIN on even steps, SPECULATIVE on odd)
        if (prefetch && l + 1 < L && d.layers[size_t(l + 1)].n_units > 0) {
          const int32_t* q = prefetch + (size_t(s) * L + l + 1) * max_ids;
          int m = 0;
          while (m < max_ids && q[m] >= 0) ++m;
          if (m) place.prefetch(l + 1, q, m, s % 2 == 1);
        }
        place.release(l);
      }
      place.end();
      stats[s] = ss_layer_stats{};
      for (const ss_layer_stats& x : place.forward_stats()) add_stats(stats[s], x);
    }
  });
}

ss_status tsa_test_copy_runs(const int32_t* layer, const int32_t* src_alloc, const int32_t* dst_alloc,
                             const uint64_t* src, const uint64_t* dst, size_t n, uint64_t unit_bytes, uint64_t cap,
                             uint32_t* run_of) {
  return tsa::guard([&] {
    using namespace tsa;
    require(n == 0 || (layer && src_alloc && dst_alloc && src && dst && run_of), SS_E_INVALID,
            "tsa_test_copy_runs: null argument");
    require(unit_bytes > 0, SS_E_INVALID, "tsa_test_copy_runs: unit_bytes is 0");
    std::vector<CopyRunItem> items(n);
    for (size_t k = 0; k < n; ++k) items[k] = CopyRunItem{layer[k], src_alloc[k], dst_alloc[k], src[k], dst[k]};
    uint32_t run = 0;
    for (size_t i = 0; i < n; ++run) {
      const size_t j = copy_run_end(items.data(), n, i, unit_bytes, std::max(cap, unit_bytes));
      for (size_t k = i; k < j; ++k) run_of[k] = run;
      i = j;
    }
  });
}

ss_status tsa_test_read_sched(const int32_t* ops, size_t n_ops, int readers, int32_t* taken, size_t* n_taken) {
  return tsa::guard([&] {
    using namespace tsa;
    require((n_ops == 0 || ops) && taken && n_taken, SS_E_INVALID, "tsa_test_read_sched: null argument");
    ReadScheduler<int32_t> q;
    q.set_readers(readers);
    size_t out = 0;
    for (size_t k = 0; k < n_ops; ++k) {
      const int32_t op = ops[3 * k], cls = ops[3 * k + 1], id = ops[3 * k + 2];
      require(cls >= 0 && cls < 3, SS_E_INVALID, "tsa_test_read_sched: class out of range");
      const ReadClass c = ReadClass(cls);
      switch (op) {
        case 0: q.push(c, id); break;
        case 1: q.raise(c, id); break;
        case 2: q.remove(c, id); break;
        case 3: {
          int32_t got = -1;
          ReadClass gc = ReadClass::kDemand;
          const bool ok = q.try_next(&got, &gc);
          taken[2 * out] = ok ? got : -1;
          taken[2 * out + 1] = ok ? int32_t(gc) : -1;
          ++out;
          break;
        }
        case 4: q.ended(c); break;
        case 5: q.hold(id != 0); break;
        case 6: q.stop(); break;
        default: fail(SS_E_INVALID, "tsa_test_read_sched: unknown op");
      }
    }
    *n_taken = out;
  });
}

ss_status tsa_test_cover_windows(uint64_t off, uint64_t n, uint64_t al, uint64_t cap, uint64_t* windows, size_t max_w,
                                 size_t* n_w) {
  return tsa::guard([&] {
    using namespace tsa;
    require(windows && n_w && al > 0 && cap >= al && cap % al == 0, SS_E_INVALID, "tsa_test_cover_windows: bad argument");
    size_t k = 0;
    for_each_cover_window(off, n, al, cap, [&](const CoverWindow& w) {
      require(k < max_w, SS_E_CAPACITY, "tsa_test_cover_windows: too many windows");
      uint64_t* o = windows + 5 * k++;
      o[0] = w.at, o[1] = w.len, o[2] = w.a0, o[3] = w.span, o[4] = w.lead;
    });
    *n_w = k;
  });
}

ss_status tsa_test_hostplace_exclusive(const char* desc_json, size_t len, const ss_budget* budget,
                                       const ss_options* opt, int steps, const int32_t* routes,
                                       const int32_t* prefetch, int max_ids, int mode, ss_exclusive_stats* out) {
  return tsa::guard([&] {
    using namespace tsa;
    require(desc_json && budget && opt && routes && out, SS_E_INVALID, "tsa_test_hostplace_exclusive: bad argument");
    const Desc d = desc_from_json(json_parse(std::string(desc_json, len)));
    const Plan p = plan_make(d, *budget, {});
    NoDevice dev;
    HostPlacement place(d, p, *opt);
    place.attach(&dev);
    place.place_residents();
    const int L = int(d.layers.size());
    for (int s = 0; s < steps; ++s) {
      place.begin(nullptr, 0);
      for (int l = 0; l < L; ++l) {
        if (d.layers[size_t(l)].n_units <= 0) continue;
        const int32_t* r = routes + (size_t(s) * L + l) * max_ids;
        int n = 0;
        while (n < max_ids && r[n] >= 0) ++n;
        if (mode == 1) place.routes_all(l);
        else place.routes(l, r, n);
        place.acquire(l, mode != 2);
        place.take_table(l);
        if (prefetch && l + 1 < L && d.layers[size_t(l + 1)].n_units > 0) {
          const int32_t* q = prefetch + (size_t(s) * L + l + 1) * max_ids;
          int m = 0;
          while (m < max_ids && q[m] >= 0) ++m;
          if (m) place.prefetch(l + 1, q, m, s % 2 == 1);
        }
        place.release(l);
      }
      place.end();
    }
    *out = place.exclusive_stats();
  });
}

}  // extern "C"

// ---- the device-gated geometry alone ----------------------------------------------------------------------------------
#include "dg_geometry.hpp"

extern "C" ss_status tsa_test_dg_geometry(const char* desc_json, size_t len, const ss_budget* budget,
                                          const uint8_t* tiers, size_t n_tiers, const ss_options* opt, uint32_t* out,
                                          uint32_t* residents, uint32_t res_cap) {
  return tsa::guard([&] {
    using namespace tsa;
    require(desc_json && budget && opt && out, SS_E_INVALID, "tsa_test_dg_geometry: null argument");
    const Desc d = desc_from_json(json_parse(std::string(desc_json, len)));
    const Plan p = tiers ? plan_from_tiers(d, *budget, std::vector<uint8_t>(tiers, tiers + n_tiers))
                         : plan_make(d, *budget, {});
    const DgGeometry x = dg_geometry(d, p, *opt);
    const uint32_t v[] = {x.keys, uint32_t(x.gated.size()), x.R, x.D, x.B, x.P, x.F, x.Q, x.I, x.S, x.disk_queue,
                          x.persistent_slots, x.slots, x.guard_slot, x.blocks, uint32_t(x.scored), x.w_trans,
                          x.w_freq, x.w_rec, x.L, x.landing_queued, x.landing_ttl, uint32_t(x.landing_chunk)};
    std::memcpy(out, v, sizeof v);
    for (uint32_t i = 0; residents && i < res_cap && i < x.residents.size(); ++i) residents[i] = x.residents[i];
  });
}
