// The device-gated decode context (SS_FORWARD_DEVICE_GATED) on one MI355X: the open-time layout and refusals
// (reference src/dg_layout.cpp:182-446, two-tier subset), the HBM arena (one array per part, slots = R + D + 2B + 1,
// the last one the zeroed guard), the fine-grained control area, the HIP transport, the service thread
// (reference src/dg_service.cpp:269-365) and the begin / end protocol (reference src/dg_ctx.cpp:429-567).
#pragma once

#include <memory>

#include "json.hpp"
#include "model.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {

class DgCtx {
 public:
  virtual ~DgCtx() = default;
  virtual bool poisoned() const = 0;
  virtual void poison() = 0;
  virtual int n_sources() const = 0;
  virtual bool source_direct(int i) const = 0;
  virtual void begin(const uint32_t* rows, int n_layers) = 0;
  virtual void end(uint32_t rows = 1) = 0;  // rows: the verify rows the token closed (ss_dg_end_rows)
  virtual void set_policy(ss_policy policy) = 0;
  virtual ss_dg_device_view device_view() const = 0;
  virtual int gated_index(int layer) const = 0;
  virtual void enqueue_begin(void* stream) = 0;
  virtual void enqueue_export(int g, const int32_t* ids_dev, int n, int n_pred, void* stream) = 0;
  virtual void enqueue_predict(int g, const int32_t* ids_dev, int n, void* stream) = 0;
  virtual void enqueue_wait(int g, void* stream) = 0;
  virtual void enqueue_end(void* stream) = 0;
  virtual uint32_t residency(ss_dg_unit* out, uint32_t cap) = 0;
  virtual void set_budgets(uint32_t spare_target, uint32_t per_layer, uint32_t per_token) = 0;
  // Between tokens: the units of gated layer g no later boundary may evict (replaces g's set; n = 0 releases it).
  virtual void keep(int g, const int32_t* ids, int n) = 0;
  // Between tokens: write-back deferral on / off, and dg_flush_ready (0 / 1 each).
  virtual void set_sched(uint32_t wb_defer, uint32_t flush_ready) = 0;
  // Between tokens: dg_clean_evict on / off from the next victim on (ss_dg_set_clean_evict).
  virtual void set_clean_evict(uint32_t on) = 0;
  // Test hooks (opened with dg_test_hooks = 1): the core's ownership invariants, between tokens; stop the service
  // thread (the next token fails closed).
  virtual void test_check() = 0;
  virtual void test_stop_service() = 0;
  virtual ss_dg_stats stats() const = 0;
  virtual ss_layer_stats layer_stats(int layer) const = 0;
  virtual ss_layer_stats total_stats() const = 0;
  virtual ss_exclusive_stats exclusive_stats() const = 0;
  virtual void stats_reset() = 0;
  virtual void set_hook(ss_stats_hook h, void* user) = 0;
  // The stats-v1 document of the counters now; the snapshot publication (as the host contract's)
  virtual Json stats_json() const = 0;
  virtual bool snapshot(ss_layer_stats* total, ss_snapshot_info* info) const = 0;
  virtual bool snapshot_json(Json* out) const = 0;
  virtual uint32_t host_table(int32_t* out, uint32_t cap) const = 0;
  virtual uint64_t verify_failures() const = 0;
  virtual bool hsa_copies() const = 0;  // unit copies through the HSA runtime (else the HIP streams)
  // measurement hooks (tsa_test.h)
  virtual void profile_enable(int on) = 0;
  virtual tsa_test_profile profile_read(bool wait) = 0;
  virtual uint32_t stamps(uint64_t* out, uint32_t cap) const = 0;
  virtual void timeline(int g, ss_dg_layer_timeline* out) const = 0;  // dg_diag (ss_dg_timeline_sized)
  virtual void boundary_timeline(ss_dg_boundary_timeline* out) const = 0;
  virtual void corrupt_block(int g, int unit, uint64_t offset) = 0;
};

std::unique_ptr<DgCtx> open_dg_ctx(const Desc& d, const Plan& p, const ss_options& o);

}  // namespace tsa
