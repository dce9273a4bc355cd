// The host contract on one MI355X (ss_begin / ss_layer_routes / ss_layer_all / ss_acquire[_groups] / ss_group_wait /
// ss_release / ss_end). Placement follows reference src/stream_ctx.cpp (init :69-272, jobs :433-706, forward
// :1194-1709) decision for decision, so hit / miss / evict sequences, groups and table slots are identical; the device
// side is this library's: slot pools and stream rings in HBM, a coarse-grained hipHostMalloc pinned tier, pinned-tier
// misses as SDMA copies issued at once on the copy stream, file misses staged through pinned buffers by reader
// threads, exclusive-mode write-backs on their own D2H stream, and (verify_hash = 2) every landed unit re-hashed in HBM
// by the checkpoint-parallel XXH64 kernel.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hip_rt.hpp"
#include "json.hpp"
#include "model.hpp"
#include "residency.hpp"
#include "source.hpp"
#include "tierstream_amd/tsa.h"

namespace tsa {

struct HostJob {
  enum State { Queued = 0, Running = 1, Done = 2, Cancelled = 3, Failed = 4 };
  int layer = 0, unit = 0;
  bool spec = false;
  bool from_pinned = false;
  bool host_dst = false;            // the pinned tier's own fill (file -> pinned host)
  void* dst = nullptr;
  const void* host_src = nullptr;   // pinned source
  hipEvent_t dst_release_ev = nullptr, dst_wb_ev = nullptr, src_wait_ev = nullptr;
  hipEvent_t done_ev = nullptr;
  std::atomic<int> state{Queued};
  ss_status err_status = SS_OK;
  std::string err;
  bool ran_as_demand = false;
};
using HostJobPtr = std::shared_ptr<HostJob>;

// Where a table address points (test hook for parity): kind 1 = layer pool (index = layer), 2 = ring class.
struct Region {
  int kind = 0, index = -1;
  uint64_t offset = 0;
};

class HostCtx {
 public:
  HostCtx(const Desc& d, const ss_budget& b, const Plan& p, const ss_options& o);
  ~HostCtx();

  void seed(int layer, const int32_t* units, int n);
  void begin(const uint32_t* rows, int n_layers);
  void routes(int layer, const int32_t* ids, int n);
  void routes_dev(int layer, const int32_t* ids_dev, int n, void* stream);
  void routes_all(int layer);
  void prefetch(int layer, const int32_t* ids, int n, bool speculative);
  void prefetch_layer(int layer);
  // Host-only read-ahead of file-backed units (ss_host_prefetch / ss_host_prefetch_layer): a no-op while
  // readahead_units is 0; the arguments are checked either way.
  void host_prefetch(int layer, const int32_t* ids, int n);
  void host_prefetch_layer(int layer);
  void acquire(int layer, void* stream, bool wait_all, ss_layer_view* out);
  void group_wait(int layer, int group, void* stream);
  void release(int layer, void* stream);
  void end();
  void check_unit(int layer, int unit);

  const ss_layer_stats& stats(int layer) const { return stats_[size_t(layer)]; }
  ss_layer_stats total() const;
  void stats_reset();
  void set_hook(ss_stats_hook h, void* user) {
    hook_ = h;
    hook_user_ = user;
  }
  ss_exclusive_stats exclusive_stats() const;
  int n_layers() const { return int(d_.layers.size()); }
  int n_sources() const { return int(files_.size()); }
  bool source_direct(int i) const { return files_[size_t(i)]->direct(); }
  void poison() noexcept { poisoned_ = true; }
  bool poisoned() const { return poisoned_; }
  Region region_of(uint64_t addr) const;
  uint64_t verify_failures() const { return verify_fail_total_; }
  // The stats-v1 document of the counters now; the snapshot publication (armed by the first snapshot call, published
  // at each ss_end that folds a forward and each reset between forwards; any thread).
  Json stats_json() const;
  bool snapshot(ss_layer_stats* total, ss_snapshot_info* info) const;
  bool snapshot_json(Json* out) const;

 private:
  enum Loc : int8_t { None = 0, Persistent = 1, Ring = 2 };
  struct RingSlot {
    void* dev = nullptr;
    uint64_t stride = 0;
    int owner = -1;
    HostJobPtr job;
  };
  struct RingClassState {
    uint64_t stride;
    size_t first, count, cursor;
    void* base;
  };
  struct Staging {
    void* host = nullptr;
    hipEvent_t ev = nullptr;
  };
  struct LayerState {
    std::unique_ptr<Residency> rs;
    void* pool = nullptr;
    hipEvent_t release_ev = nullptr, ready_ev = nullptr, ids_ev = nullptr;
    bool ready_wait = false;
    void* table_dev[2] = {nullptr, nullptr};
    uint64_t* table_host[2] = {nullptr, nullptr};
    hipEvent_t table_ev[2] = {nullptr, nullptr};
    int version = 0;
    std::vector<int8_t> loc;
    std::vector<int32_t> slot;
    std::vector<HostJobPtr> job;
    std::vector<char> spec_unclaimed;
    std::vector<int32_t> routed, pending, hits;
    std::vector<uint32_t> count;
    std::vector<std::vector<int32_t>> groups;
    std::vector<ss_group> group_view;
    bool routes_given = false, acquired = false, released = false, skip = false;
    int32_t* ids_host = nullptr;
    size_t ids_cap = 0;
    int ids_n = -1;
  };
  // verify_hash = 2: the device check of a landed unit (checkpoints of the unit, uploaded once per unit)
  struct UnitCheck {
    uint64_t* states_dev = nullptr;
    uint64_t n_states = 0;
  };

  void init();
  void cleanup() noexcept;
  void worker();
  void run_job(HostJob& j);
  void read_unit_host(int layer, int unit, void* dst, bool hash, uint64_t* digest);
  void read_unit_device(HostJob& j);
  void submit(const HostJobPtr& j);
  void fail_job(HostJob& j, ss_status st, const char* msg) noexcept;
  void promote(const HostJobPtr& j);
  void wait_job(HostJob& j);
  void wait_job_quiet(HostJob& j);
  HostJobPtr make_job(int layer, int unit, void* dst, bool spec);
  void fetch_into_persistent(int layer, int unit, int slot, bool spec, hipEvent_t dst_wb_ev = nullptr);
  bool fetch_into_ring(int layer, int unit, bool spec);
  void dispatch_pending();
  void ingest_routes(int layer, const int32_t* ids, int n);
  void ingest_dev_routes(int layer);
  void check_layer(int layer, const char* what) const;
  void check_stream(void* stream, const char* what);
  void* unit_addr(int layer, int unit) const;
  void open_forward();
  void retire_ring(int layer);
  hipEvent_t write_back(int layer, const Admission& a, bool speculative, size_t* n_wb);
  void fetch_admitted(int layer, const Admission& a, bool spec);
  uint64_t writeback_blocks(int layer, bool speculative) const;
  int eviction_cap(int layer, bool speculative) const;
  void free_block(int layer, int unit);
  int block_class(int layer) const { return excl_ ? layer_class_[size_t(layer)] : -1; }
  hipEvent_t pooled_event();
  int64_t gidx(int layer, int unit) const { return d_.unit_base[size_t(layer)] + unit; }
  void verify_landed(const HostJob& j);  // verify_hash = 2: the unit joins the pending check batch (copy_mu_ held)
  void flush_verify();                   // the pending batch: one launch on the verify stream behind its copies
  void collect_verify();

  Desc d_;
  Plan plan_;
  ss_options o_;
  std::unique_ptr<HipDevice> dev_;
  // Pinned -> HBM copies alternate between copy_ and copy2_ (two SDMA queues: one queue's per-copy gap is about 6 % of
  // a 9 MiB unit's copy time); the other copies use copy_. join_copies() makes copy_ follow copy2_'s work so far, so
  // an event recorded on copy_ after it stands for every copy before it.
  hipStream_t copy_ = nullptr, copy2_ = nullptr, wb_ = nullptr;
  hipEvent_t join_ev_ = nullptr;
  bool copy_alt_ = false;
  hipStream_t next_copy_stream() { return (copy_alt_ = !copy_alt_) ? copy2_ : copy_; }
  void join_copies();  // (copy_mu_ held)
  std::vector<std::unique_ptr<SourceFile>> files_;
  std::vector<LayerState> L_;
  std::vector<RingSlot> ring_;
  std::vector<hipEvent_t> ring_owner_ev_;
  std::vector<hipEvent_t> ev_pool_, all_events_;
  std::vector<RingClassState> ring_classes_;
  std::vector<void*> pinned_chunks_;
  std::vector<const void*> pinned_of_;

  bool excl_ = false;
  std::vector<uint64_t> block_bytes_;
  std::vector<int> layer_class_;
  std::vector<std::vector<void*>> free_blocks_;
  std::vector<void*> spare_chunks_;
  std::vector<hipEvent_t> wb_pending_;
  std::vector<int64_t> wb_units_;
  std::vector<hipEvent_t> wb_evs_;
  hipEvent_t blocks_ev_ = nullptr, wb_mark_ev_ = nullptr;
  bool wb_gate_ = false;
  std::vector<uint64_t> spares_of_;
  ss_exclusive_stats xst_{};

  std::vector<Staging> staging_;
  std::vector<size_t> staging_free_;
  std::mutex staging_mu_;
  std::condition_variable staging_cv_;
  std::mutex copy_mu_;

  std::mutex q_mu_;
  std::condition_variable q_cv_, done_cv_;
  std::deque<HostJobPtr> demand_q_, spec_q_;
  int demand_running_ = 0;
  bool stop_ = false;
  std::vector<std::thread> workers_;

  // verify_hash = 2
  bool dverify_ = false;
  uint64_t seg_bytes_ = 0;
  std::vector<UnitCheck> checks_;  // per global unit (with a descriptor hash)
  void* vtable_dev_ = nullptr;     // tsa_verify_unit slots, one per possible in-flight verify
  uint32_t* vfail_dev_ = nullptr;
  tsa_verify_unit* vtable_host_ = nullptr;
  uint32_t* vfail_host_ = nullptr;
  size_t vcap_ = 0, vused_ = 0, vflushed_ = 0;  // table slots used this forward; the ones already launched
  hipStream_t vstream_ = nullptr;                 // the checks (copies never queue behind them)
  hipEvent_t vready2_ev_ = nullptr;               // the second copy stream at a flush
  hipEvent_t vready_ev_ = nullptr;                // the copy stream at a flush: the batch's copies are done
  std::vector<std::pair<int, int>> vunits_;  // (layer, unit) of each verify slot this forward
  // A landed unit's check reads its slot until the check's launch completes, so the next copy into that slot waits for
  // it: the slot's pending entry (since the last collect), the flush that launched each entry, and per flush an event
  // on the verify stream after its launch.
  std::unordered_map<const void*, size_t> vdst_;
  std::vector<uint32_t> ventry_flush_;
  std::vector<hipEvent_t> vflush_ev_;
  uint32_t vflushes_ = 0;
  void wait_slot_check(hipStream_t s, const void* dst);  // (copy_mu_ held)
  hipEvent_t vdone_ev_ = nullptr;
  uint64_t verify_fail_total_ = 0;

  void* fwd_stream_ = nullptr;
  bool fwd_stream_set_ = false;
  bool poisoned_ = false, in_forward_ = false, fwd_open_ = false;
  uint64_t forward_ = 0;
  uint64_t n_blocks_ = 0;  // EXCLUSIVE: the pinned blocks (the homes of the pinned units and the spares)
  struct Published {
    uint64_t seq = 0, forwards = 0;
    std::vector<ss_layer_stats> layers;
    ss_exclusive_stats x{};
  };
  mutable std::atomic<bool> snap_armed_{false};
  mutable std::mutex snap_mu_;
  Published snap_;
  void publish();
  Json format_stats(uint64_t forwards, const ss_layer_stats* layers, const ss_exclusive_stats& x) const;
  std::vector<HostJobPtr> fwd_jobs_;
  std::vector<ss_layer_stats> stats_, fwd_stats_;
  ss_stats_hook hook_ = nullptr;
  void* hook_user_ = nullptr;
};

}  // namespace tsa
