// The host contract on one MI355X (ss_seed / ss_begin / ss_layer_routes[_dev] / ss_layer_all / ss_prefetch /
// ss_acquire[_groups] / ss_group_wait / ss_release / ss_end). HostPlacement decides every placement; this executor
// carries its orders out:
//  - layer pools and the stream ring in HBM, the pinned tier and exclusive-mode spare blocks in hipHostMalloc memory;
//  - copies from pinned blocks are issued when the engine call that ordered them returns, on two SDMA copy streams
//    (alternating per copy; neighbouring units into neighbouring slots go as one copy);
//  - a copy from a file is a job for the reader threads: direct-I/O reads into pinned staging, host XXH64, then the
//    copy stream;
//  - exclusive-mode write-backs run on their own device-to-host stream;
//  - with readahead_units, file-backed units a forward will need are read ahead into pinned read-ahead buffers by the
//    reader threads (below demand reads), and their copy later lands from the buffer;
//  - with verify_hash = 2 every landed unit is re-hashed in HBM (checkpoint-parallel XXH64, batched on a verify stream);
//  - every wait the reference expresses as an event (a slot's last reader, a victim's write-back, a block's write-back,
//    the copies of an earlier forward) is a device-side stream wait here.
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
#include "host_place.hpp"
#include "json.hpp"
#include "model.hpp"
#include "read_sched.hpp"
#include "source.hpp"
#include "stream_order.hpp"
#include "tierstream_amd/tsa.h"
#include "tierstream_amd/tsa_test.h"

namespace tsa {

// Where a table address points (test hook for parity): kind 1 = layer pool (index = layer), 2 = ring class.
struct Region {
  int kind = 0, index = -1;
  uint64_t offset = 0;
};

class HostCtx final : public HostWork {
 public:
  HostCtx(const Desc& d, const ss_budget& b, const Plan& p, const ss_options& o);
  ~HostCtx() override;

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

  const ss_layer_stats& stats(int layer) const { return place_.stats()[size_t(layer)]; }
  ss_layer_stats total() const;
  void stats_reset();
  void set_hook(ss_stats_hook h, void* user) {
    hook_ = h;
    hook_user_ = user;
  }
  ss_exclusive_stats exclusive_stats() const { return place_.exclusive_stats(); }
  int n_layers() const { return int(d_.layers.size()); }
  int n_sources() const { return int(files_.size()); }
  bool source_direct(int i) const { return files_[size_t(i)]->direct(); }
  void poison() noexcept { poisoned_ = true; }
  bool poisoned() const { return poisoned_; }
  Region region_of(uint64_t addr) const;
  uint64_t verify_failures() const { return verify_fail_total_; }
  // Test hooks: reader threads take no job while held (a stop still ends them); wait until every read-ahead read of
  // the forward has ended (readers not held).
  void test_hold_readers(bool hold);
  void test_ra_quiesce();
  void test_inject(int what);
  void check_exclusive() const { place_.check_blocks(); }
  void copy_counts(uint64_t* units, uint64_t* copies) const {
    std::lock_guard<std::mutex> lk(copy_mu_);
    *units = pinned_units_;
    *copies = pinned_copies_;
  }
  // Cross-stream waits given to the runtime and those skipped as implied by an earlier wait of the same stream.
  void wait_counts(uint64_t* issued, uint64_t* skipped) { ord_.counts(issued, skipped); }
  // Timing (a test hook, between forwards): each device-check launch bracketed by its dispatch's own begin and end
  // stamps when on & TSA_TEST_PROF_VERIFY (this context brackets nothing else); read sums the completed brackets.
  void profile_enable(int on);
  tsa_test_profile profile_read(bool wait);
  // The stats-v1 document of the counters now; the snapshot publication (armed by the first snapshot call, published
  // at each ss_end that folds a forward and each reset between forwards; any thread).
  Json stats_json() const;
  bool snapshot(ss_layer_stats* total, ss_snapshot_info* info) const;
  bool snapshot_json(Json* out) const;

 private:
  struct RaEntry;
  // One copy onto the device (or, to_host, a pinned block's fill from the file at open, or a read-ahead read).
  struct Copy {
    enum State : int { kQueued = 0, kRunning = 1, kDone = 2, kCancelled = 3, kFailed = 4 };
    int32_t layer = 0, unit = 0;
    bool speculative = false, to_host = false;
    bool reading = false;                   // a reader started it (its class counts it running until it ends)
    ReadClass ran_as = ReadClass::kDemand;  // (reading) the class it was started from
    RaEntry* ra = nullptr;      // a read-ahead read: its request
    uint64_t bytes_read = 0;    // a read-ahead read: the file bytes it read
    void* dst = nullptr;
    const void* src = nullptr;  // a pinned block, or null: the unit's file
    hipEvent_t after[3] = {nullptr, nullptr, nullptr};  // dst's last reader, dst's victim write-back, src's write-back
    hipEvent_t done_ev = nullptr;
    bool owns_ev = true;      // false: done_ev is the event of the run it was copied in (its first copy owns it)
    int32_t src_alloc = -1;   // a pinned block's allocation (-1: not a pinned block)
    int32_t dst_alloc = -1;   // the destination's allocation (a ring class, or a layer's pool)
    std::atomic<int> state{kQueued};
    ss_status status = SS_OK;
    std::string what;
  };
  using CopyPtr = std::shared_ptr<Copy>;
  struct ReadOutcome {
    int state = Copy::kDone;
    ss_status status = SS_OK;
    std::string what;
  };
  struct LayerDev {
    void* pool = nullptr;
    uint64_t stride = 0;
    hipEvent_t release_ev = nullptr, ready_ev = nullptr, ids_ev = nullptr;
    void* table_dev[2] = {nullptr, nullptr};
    uint64_t* table_host[2] = {nullptr, nullptr};
    hipEvent_t table_ev[2] = {nullptr, nullptr};
    int version = 0;
    std::vector<ss_group> group_view;
    int32_t* ids_host = nullptr;  // device routes copied back (ss_layer_routes_dev)
    size_t ids_cap = 0;
    int ids_n = -1;
  };
  struct Staging {
    void* host = nullptr;
    hipEvent_t ev = nullptr;  // the last copy out of it
  };
  // verify_hash = 2: a unit's checkpoints in HBM (uploaded once, the first time its bytes pass the host hash)
  struct UnitCheck {
    uint64_t* states_dev = nullptr;
    uint64_t n_states = 0;
  };

  // Host read-ahead: one request of this forward. Waiting (no buffer yet) -> Reading (its read queued or running) ->
  // Ready (read) -> Landing (a fetch takes it: the copy out of the buffer is issued when the read ends) -> Consumed;
  // Abandoned (not needed any more), Failed (its read failed: the fetch reads the file).
  struct RaEntry {
    enum State : uint8_t { kWaiting, kReading, kReady, kLanding, kConsumed, kAbandoned, kFailed };
    int32_t layer = 0, unit = 0;
    State st = kWaiting;
    int32_t buf = -1;
    std::shared_ptr<Copy> producer, child;
  };
  struct RaCounts {  // the reference's "readahead" counters: requests, reads ended, landed, unused, failed, fallback
    uint64_t requested = 0, read = 0, landed = 0, unused = 0, failed = 0, fallback = 0, bytes = 0;
  };

  // HostWork
  void write_back(const WriteBackOrder& w) override;
  bool fetch(const FetchOrder& f) override;
  void read_ahead(int layer, int unit) override;
  void promote(int32_t job) override;
  void retire(int32_t job) override;
  bool settle(int32_t job, bool speculative) override;

  void init();
  void cleanup() noexcept;
  void reader_loop();
  void read_file_unit(Copy& c);  // a reader thread: the unit's file bytes to its destination
  // got: + the file bytes read (null: not counted)
  void read_into_host(int layer, int unit, void* dst, bool hash, uint64_t* digest, uint64_t* got = nullptr);
  bool take_inject(int what);  // (one shot) the armed injection is `what`: disarm it and report true
  void issue_first_piece(Copy& c, const void* src);
  std::vector<uint64_t> checkpoint_buffer(const Layer& l, bool hash) const;
  void keep_checkpoints_locked(int64_t g, const std::vector<uint64_t>& states);
  const SourceFile& part_source(int layer, int unit, const Part& part, uint64_t* off) const;
  void stage_to_device(Copy& c);
  void submit(const CopyPtr& c);
  void issue_copy(Copy& c, const void* src, hipEvent_t after_ev);  // host memory -> c.dst now (copy_mu_ taken)
  void issue_copy_locked(Copy& c, const void* src, hipEvent_t after_ev);  // the same, copy_mu_ held
  // Copies from pinned blocks are held until the engine call that ordered them returns, then issued: a run of them
  // whose sources and destinations advance by the same stride inside one allocation each goes as one copy (the units
  // of a layer's misses are fetched in id order, so neighbours in a pinned layout often take neighbouring ring slots).
  void flush_copies();
  void issue_run(size_t first, size_t end, uint64_t span);  // pend_[first, end) as one copy of span bytes (copy_mu_)
  struct PendGuard {  // an engine call that throws part-way still issues what it ordered
    HostCtx* h;
    ~PendGuard() {
      if (h->pend_.empty()) return;
      try {
        h->flush_copies();
      } catch (...) {
      }
    }
  };
  void wait_jobs(const std::vector<int32_t>& jobs, hipStream_t es);
  void release_event(const Copy& c) {
    if (c.done_ev && c.owns_ev) ev_pool_.push_back(c.done_ev);
  }
  // read-ahead
  bool ra_on() const { return !ra_buf_.empty(); }
  void ra_pump();                                  // waiting requests take free buffers (engine thread)
  bool ra_land(RaEntry& e, const CopyPtr& child);  // a fetch of e's unit: true when it lands from the buffer
  void ra_issue_child(RaEntry& e, Copy& child);    // the copy out of e's buffer (e's read has ended)
  void ra_read_ended(Copy& p, int state, ss_status st, const std::string& what);  // a reader thread
  void ra_abandon_locked(RaEntry& e);              // q_mu_ held
  void ra_give_buf_locked(RaEntry& e);             // q_mu_ held
  void ra_end_forward();                           // ss_end: no more requests, reads ended, counts
  void finish(Copy& c, int state, ss_status st, const std::string& what) noexcept;
  void await(Copy& c);       // until it ends; throws its error if it failed
  void await_quiet(Copy& c);  // until it ends
  size_t take_staging();
  void give_staging(size_t i);
  void check_layer(int layer, const char* what) const;
  void check_stream(void* stream, const char* what);
  void ingest_dev_routes(int layer);
  void* spot_addr(int layer, const DevSpot& s) const;
  hipEvent_t pooled_event();
  int64_t gidx(int layer, int unit) const { return d_.gidx(layer, unit); }
  hipStream_t next_copy_stream() {
    copy_next_ = (copy_next_ + 1) % int(copyx_.size() + 1);
    return copy_next_ ? copyx_[size_t(copy_next_ - 1)] : copy_;
  }
  void join_copies();  // copy_ follows the other copy streams' work so far (copy_mu_ held)
  void sync_copies();  // every copy stream drained
  // verify_hash = 2
  void verify_landed(const Copy& c);  // the unit joins the pending check batch (copy_mu_ held)
  void flush_verify();                // the pending batch: one launch on the verify stream behind its copies
  void collect_verify();
  void wait_slot_check(hipStream_t s, const void* dst);  // a slot's next copy waits for its pending check
  void publish();
  Json format_stats(uint64_t forwards, const ss_layer_stats* layers, const ss_exclusive_stats& x,
                    const RaCounts& ra) const;

  Desc d_;
  Plan plan_;
  ss_options o_;
  HostPlacement place_;
  std::unique_ptr<HipDevice> dev_;
  std::vector<std::unique_ptr<SourceFile>> files_;
  std::vector<LayerDev> L_;
  // Pinned -> HBM copies rotate over copy_ and copyx_ (kCopyStreams SDMA queues); other copies use copy_. Measured
  // with neighbouring units merged: three queues gain under 1 % on 9 MiB units and cost 2 % on 224 MiB blobs, and every
  // extra queue slows the device checks beside it.
  static constexpr int kCopyStreams = 2;
  hipStream_t copy_ = nullptr, wb_ = nullptr;
  std::vector<hipStream_t> copyx_;  // the other copy streams
  std::vector<hipEvent_t> joinx_ev_, vreadyx_ev_;  // per other copy stream: its mark at a join / at a check flush
  int copy_next_ = 0;
  std::vector<void*> ring_base_;     // per ring class
  std::vector<void*> ring_addr_;     // per ring slot
  std::vector<void*> host_chunks_;   // the pinned tier and the spare blocks
  std::vector<void*> block_addr_;    // per pinned block
  uint64_t excl_blocks_ = 0;         // exclusive mode: blocks of the block classes (homes + spares)
  std::vector<hipEvent_t> wb_ev_;    // this forward's write-back batches
  hipEvent_t blocks_ev_ = nullptr, wb_mark_ev_ = nullptr;
  bool wb_gate_ = false;             // the next write-back waits for blocks_ev_ (the last forward's block readers)
  std::vector<hipEvent_t> ev_pool_, all_events_;
  std::vector<CopyPtr> jobs_;        // this forward's, by job id
  std::vector<CopyPtr> fills_;       // open and seed fills
  std::vector<CopyPtr> pend_;        // pinned-block copies ordered by the current engine call, not issued yet
  uint64_t pinned_units_ = 0, pinned_copies_ = 0;  // since open (copy_mu_)
  std::vector<int32_t> block_alloc_;  // per pinned block: its allocation (an index into host_chunks_)
  std::vector<int32_t> ring_alloc_;   // per ring slot: its ring class
  ss_status fwd_failed_ = SS_OK;     // the first failed job of the forward (settle)
  std::string fwd_error_;

  std::vector<Staging> staging_;
  std::vector<size_t> staging_free_;
  std::mutex staging_mu_;
  std::condition_variable staging_cv_;
  mutable std::mutex copy_mu_;
  StreamOrder ord_;  // every event record and cross-stream wait of this context

  // reader threads and the reads they start (read_sched.hpp); q_mu_ guards the scheduler, copy states and read-ahead
  // request states together
  std::mutex q_mu_;
  std::condition_variable done_cv_;
  ReadScheduler<CopyPtr> reads_;
  // read-ahead buffers (pinned, one unit each) and this forward's requests
  std::vector<void*> ra_buf_;
  std::vector<hipEvent_t> ra_ev_;                     // per buffer: its last copy out
  std::vector<int32_t> ra_free_;                      // q_mu_
  std::vector<std::unique_ptr<RaEntry>> ra_entries_;  // engine thread (their states under q_mu_)
  std::vector<std::vector<int32_t>> ra_index_;        // [layer][unit]: its entry this forward, -1
  std::deque<RaEntry*> ra_wait_;                      // engine thread
  bool ra_frozen_ = false;
  RaCounts ra_st_;                                    // since open or the last reset
  std::vector<std::thread> readers_;
  std::atomic<int> inject_{0};  // ss_test_inject

  // verify_hash = 2
  bool dverify_ = false;
  uint64_t seg_bytes_ = 0;
  std::vector<UnitCheck> checks_;  // per global unit (with a descriptor hash)
  void* vtable_dev_ = nullptr;     // tsa_verify_unit slots, one per possible in-flight check
  uint32_t* vfail_dev_ = nullptr;
  tsa_verify_unit* vtable_host_ = nullptr;
  uint32_t* vfail_host_ = nullptr;
  size_t vcap_ = 0, vused_ = 0, vflushed_ = 0;  // table slots used this forward; the ones already launched
  hipStream_t vstream_ = nullptr;                 // the checks (copies never queue behind them)
  hipEvent_t vready_ev_ = nullptr;  // copy_ at a flush (the other copy streams: vreadyx_ev_)
  std::vector<std::pair<int, int>> vunits_;  // (layer, unit) of each check slot this forward
  // a landed unit's check reads its slot until its launch completes: the slot's pending entry, the flush that launched
  // each entry, and per flush an event on the verify stream after its launch
  std::unordered_map<const void*, size_t> vdst_;
  std::vector<uint32_t> ventry_flush_;
  std::vector<hipEvent_t> vflush_ev_;
  uint32_t vflushes_ = 0;
  hipEvent_t vdone_ev_ = nullptr;
  uint64_t verify_fail_total_ = 0;
  // check launch timing (profile_enable): brackets in flight, recycled events, the sums so far (copy_mu_)
  struct TimedCheck {
    hipEvent_t start, stop;
    uint64_t bytes;
    uint32_t units;
  };
  bool prof_verify_ = false;
  std::vector<TimedCheck> prof_pending_;
  std::vector<hipEvent_t> prof_free_, prof_made_;
  tsa_test_profile prof_sum_{};
  void prof_drain(bool wait);  // copy_mu_ held

  void* fwd_stream_ = nullptr;
  bool fwd_stream_set_ = false;
  bool poisoned_ = false;
  struct Published {
    uint64_t seq = 0, forwards = 0;
    std::vector<ss_layer_stats> layers;
    ss_exclusive_stats x{};
    RaCounts ra;
  };
  mutable std::atomic<bool> snap_armed_{false};
  mutable std::mutex snap_mu_;
  Published snap_;
  ss_stats_hook hook_ = nullptr;
  void* hook_user_ = nullptr;
};

}  // namespace tsa
