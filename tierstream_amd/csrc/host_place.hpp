// The host contract's placement, with no device in it: which units of a forward are hits, which are admitted into a
// layer's pool of persistent slots (evicting whom), which stream through the ring of shared slots (and in which slot),
// which wait for a ring slot, which pinned block each copy reads and each exclusive-mode victim is written back to,
// how a layer's units are grouped, and every counter. It decides; a HostWork carries each decision out on a device as
// it is made (the MI355X executor in host_ctx.cpp, or nothing at all in the CPU placement tests).
//
// The rules are the reference's host contract (src/stream_ctx.cpp: routes :1303-1355, prefetch :1401-1439, acquire
// :1459-1521, release :1572-1590, end :1600-1709; slot admission in residency.hpp), so hit / miss / evict sequences,
// ring slots, groups and the address tables equal the reference's for the same call sequence. The structure is this
// library's: placement is a pure state machine driven by the ss_* calls; a layer's routes are sorted into hits, claims
// and asks in one pass; the ring, its wait line and the spare blocks are objects of their own (host_slots.hpp); each
// admission computes its victim budget once and carries it through; and the read-ahead rules ask one question, where
// a unit's bytes would come from now.
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

#include "host_slots.hpp"
#include "model.hpp"
#include "residency.hpp"

namespace tsa {

// Where a unit's bytes are on the device in this forward.
struct DevSpot {
  enum Kind : int8_t { kNone = 0, kPool = 1, kRing = 2 };
  Kind kind = kNone;
  int32_t index = -1;  // kPool: slot of the unit's layer pool; kRing: global ring slot (-1 while waiting for one)
};

// A copy of unit (layer, unit) into dst. Forward jobs are numbered from 0 in each forward; fills (open, seeds) use
// job -1.
struct FetchOrder {
  int32_t job = -1;
  int32_t layer = 0, unit = 0;
  bool speculative = false;
  DevSpot dst;
  int32_t after_release = -1;    // the copy waits for this layer's last ss_release (dst's previous reader), -1: none
  int32_t after_writeback = -1;  // dst held a victim written back by this batch of the forward, -1: none
  int32_t src_block = -1;        // the pinned block with the unit's bytes, -1: read them from the file
  int32_t src_writeback = -1;    // exclusive: the batch of this forward that writes src_block, -1: none
};

// Exclusive mode: victims of one admission leave their pool slots for free blocks (batch: numbered per forward).
struct WriteBackOrder {
  int32_t batch = 0, layer = 0;
  std::vector<int32_t> units, slots, blocks;  // parallel
};

// A pinned block: the pinned-tier home of a unit (home >= 0, its global index) or a spare of block class `cls`.
struct BlockHome {
  int64_t home = -1;
  int32_t cls = -1;
};

class HostWork {
 public:
  virtual ~HostWork() = default;
  virtual void write_back(const WriteBackOrder& w) = 0;
  // true: the copy lands from the unit's read-ahead buffer (its file bytes are counted when the read-ahead ends)
  virtual bool fetch(const FetchOrder& f) = 0;
  // Host read-ahead (readahead_units): read file-backed unit (layer, unit) into a host buffer now, for a later fetch
  // of it in this forward (default: nothing).
  virtual void read_ahead(int layer, int unit) { (void)layer, (void)unit; }
  virtual void promote(int32_t job) = 0;  // a speculative job was routed: it becomes a demand
  virtual void retire(int32_t job) = 0;   // its ring slot was released: cancel it if it never started, else wait
  // End of forward, in job order: cancel a speculative job that never started, else wait for it; true when it ran to
  // completion.
  virtual bool settle(int32_t job, bool speculative) = 0;
};

class HostPlacement {
 public:
  HostPlacement(const Desc& d, const Plan& p, const ss_options& o);
  void attach(HostWork* w) { w_ = w; }

  // ---- the layout the executor allocates
  bool exclusive() const { return excl_; }
  int pool_slots(int layer) const { return L_[size_t(layer)].pool ? L_[size_t(layer)].pool->capacity() : 0; }
  struct RingClassInfo {
    uint64_t stride;
    uint32_t first, count;
  };
  const std::vector<RingClassInfo>& ring_classes() const { return ring_cls_; }
  uint32_t ring_slots() const { return ring_.size(); }
  const std::vector<BlockHome>& blocks() const { return blocks_; }
  const std::vector<uint64_t>& block_class_bytes() const { return class_bytes_; }
  uint64_t block_count() const { return blocks_.size(); }

  // ---- open and between forwards
  // The planned residents' pool slots; with fill_residents, one fill copy each (job -1) through HostWork::fetch.
  void place_residents();
  // ss_seed: free slots only (seeds never evict); returns the units placed, each with its fill through fetch().
  std::vector<int32_t> seed(int layer, const int32_t* units, int n);
  void seed_landed(int layer, int32_t unit, bool ok);  // a failed fill is dropped; exclusive: a landed one's block frees

  // ---- a forward
  void begin(const uint32_t* rows, int n_layers);
  bool forward_open() const { return fwd_open_; }
  bool in_forward() const { return in_fwd_; }
  bool routes_given(int layer) const { return L_[size_t(layer)].routes_in; }
  void routes(int layer, const int32_t* ids, int n);
  void routes_all(int layer);
  void prefetch(int layer, const int32_t* ids, int n, bool speculative);
  // ss_host_prefetch: read-ahead requests for the eligible units (allowed between forwards: they belong to the next)
  void host_prefetch(int layer, const int32_t* ids, int n);
  bool ra_on() const { return ra_bytes_ > 0; }   // readahead_units > 0 and some unit can be read from its file
  uint64_t ra_bytes() const { return ra_bytes_; }  // a read-ahead buffer: the largest host stride read from a file
  void add_disk_bytes(int layer, uint64_t b) { fwd_[size_t(layer)].bytes_disk += b; }  // (read-ahead reads, at end)
  // A requested read-ahead is still of use: the unit is off the device with no copy of it, no pinned source.
  bool ra_wanted(int layer, int unit) const;
  struct Acquire {
    bool wait_ready = false;         // wait for the copies of earlier forwards into this layer's pool
    std::vector<int32_t> wait_jobs;  // (wait_all) every fetched routed unit's job, group order
  };
  // ss_acquire in two steps: the units waiting for a ring slot are placed (or SS_E_CAPACITY), the groups are formed
  // and the jobs to wait for listed; once those waits succeeded, take_table builds the layer's table and marks it
  // acquired.
  Acquire acquire(int layer, bool wait_all);
  const std::vector<DevSpot>& take_table(int layer);
  const std::vector<DevSpot>& table(int layer) const { return L_[size_t(layer)].table; }
  const std::vector<std::vector<int32_t>>& groups(int layer) const { return L_[size_t(layer)].groups; }
  std::vector<int32_t> group_jobs(int layer, int group) const;  // ss_group_wait's jobs (group 0: none)
  bool acquired(int layer) const { return L_[size_t(layer)].acquired; }
  bool released(int layer) const { return L_[size_t(layer)].released; }
  int32_t job_of(int layer, int unit) const { return L_[size_t(layer)].job[size_t(unit)]; }
  void release(int layer);
  struct Ended {
    std::vector<int> landed_layers;  // layers with a pool copy issued this forward (their next acquire waits)
    uint32_t writeback_batches = 0;
  };
  Ended end();  // every job settled (HostWork::settle); residency, blocks and counters of the forward folded
  void add_wait_ns(int layer, uint64_t ns) { fwd_[size_t(layer)].wait_ns += ns; }

  // ---- counters
  const std::vector<ss_layer_stats>& stats() const { return total_; }
  const std::vector<ss_layer_stats>& forward_stats() const { return fwd_; }
  void reset_stats();
  const ss_exclusive_stats& exclusive_stats() const { return xst_; }
  // Exclusive mode, between forwards: each pinned block belongs to exactly one unit off the device or to a free list,
  // and no write-back is pending (ss_test_check_exclusive; SS_E_INVALID naming the first rule broken).
  void check_blocks() const;
  uint64_t forwards() const { return forwards_; }

 private:
  struct LayerPlace {
    std::unique_ptr<SlotPool> pool;  // null: the layer has no units
    int32_t cls = -1;                // exclusive: its block class
    // this forward
    std::vector<DevSpot> spot;
    std::vector<int32_t> job;
    std::vector<uint8_t> spec_open;  // fetched speculatively and not routed (yet)
    std::vector<uint32_t> uses;      // occurrences in the routes
    std::vector<int32_t> routed, hits;  // this forward's routed units and its hits, ascending
    std::vector<std::vector<int32_t>> groups;
    std::vector<DevSpot> table;
    bool routes_in = false, acquired = false, released = false, skipped = false;
    bool ready_wait = false;  // across forwards: the next acquire waits for the pool copies of the last one
    std::vector<uint8_t> ra_asked;  // this forward: a read-ahead was requested (never twice)
  };
  struct Job {
    int32_t layer, unit;
    bool speculative, pool;
  };
  // A layer's routed units sorted in one pass: hits were resident before this forward, claims were placed earlier in
  // it (a prefetch), asks need admission; held marks the units an admission must not evict (routed, or placed).
  struct RouteSort {
    std::vector<int32_t> hits, claims, asks;
    std::vector<char> held;
  };
  // What one admission may evict: cap for SlotPool::admit (-1: none) and the blocks its victims may be written to.
  struct VictimBudget {
    int cap = -1;
    uint64_t blocks = 0;
  };
  // Where a unit's bytes would come from if it were fetched now.
  enum class Source { kDevice, kPinned, kFile, kPeer };

  void open_forward();
  LayerPlace& layer_with_units(int layer, const char* what);
  int32_t new_job(int layer, int unit, bool speculative, bool pool);
  FetchOrder order_for(int layer, int unit, bool speculative);
  void issue(const FetchOrder& f);  // records the copy's spot and job, hands it to the executor, counts its bytes
  RouteSort sort_routes(int layer) const;
  VictimBudget victim_budget(int layer, bool speculative) const;
  // Admission of `units` into the layer's pool: victims leave for blocks (exclusive), the admitted units are copied.
  Admission admit_units(int layer, const std::vector<int32_t>& units, const std::vector<char>& held, bool speculative);
  int32_t write_back_victims(int layer, const Admission& a, const VictimBudget& b);  // its batch, -1: none
  bool stream(int layer, int unit, bool speculative);  // a ring slot now (false: none free)
  void wait_for_ring(int layer, int unit);
  void serve_wait_line();
  void give_back_block(int layer, int unit);  // a promoted unit's block returns to its class's free list
  Source source_now(int layer, int unit) const;
  // A read-ahead request for a unit the forward will read from its file (see ra_wanted); waiting_ok: also while it
  // waits for a ring slot.
  void ra_request(int layer, int unit, bool waiting_ok);
  void take_routes(int layer, const int32_t* ids, int n);

  const Desc& d_;
  const Plan& p_;
  ss_options o_;
  HostWork* w_ = nullptr;
  bool excl_ = false;
  std::vector<LayerPlace> L_;
  std::vector<RingClassInfo> ring_cls_;
  RingPool ring_;
  WaitLine line_;
  // pinned blocks: the units' homes, then the spares; block_of_[g] the block a unit's bytes are in (-1: its file)
  std::vector<BlockHome> blocks_;
  std::vector<uint64_t> class_bytes_;
  std::vector<int32_t> block_of_;
  SpareBlocks spare_;
  std::vector<int32_t> wb_batch_of_;  // per global unit: this forward's write-back batch into its block, -1
  std::vector<int64_t> wb_touched_;
  int32_t wb_batches_ = 0;
  std::vector<Job> jobs_;
  uint64_t ra_bytes_ = 0;
  bool fwd_open_ = false, in_fwd_ = false;
  uint64_t forwards_ = 0;
  std::vector<ss_layer_stats> fwd_, total_;
  ss_exclusive_stats xst_{};
};

void add_stats(ss_layer_stats& a, const ss_layer_stats& b);

}  // namespace tsa
