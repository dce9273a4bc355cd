// Device-gated decode: the cache state machine, free of any device API (a transport does the copies, publications and
// events). The decisions - homes (Host / Device / Coming / Bank / Evicting), free-slot and bank-slot choice, cover,
// resurrection, recency, the boundary's admissions, victims from the recency tail to the spare target, deferred
// write-backs with a per-layer credit, the inclusive share of clean copies - are those of reference src/dg_core.cpp
// (place :769-858, fetch_impl :1146-1368, serve_demand / serve_use / serve_prediction :1415-1634, end_token
// :1636-1927, collect / write-back scheduling :961-1097) for its two- and three-tier configurations, with LRU or
// scored victims (score_history / select_scored / score_candidate :1929-2057, the boundary's one acceptance loop
// :1775-1840, set_policy :2059-2071; the score and its order: reference docs/design.md:284-354).
//
// Schedule: this core asks its transport for completion (collect) only through done(), which the MI355X transport
// answers after waiting for the event, and it never asks whether the device "ran ahead". Every decision is therefore
// the one the reference makes under its canonical (eager) schedule: placement is a function of the route stream alone,
// which is what makes slot tables comparable bit for bit with the CPU oracle.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <unordered_map>
#include <vector>

namespace tsa {

class DgTransport {
 public:
  enum Stream { kDem = 0, kPf = 1, kD2h = 2 };
  virtual ~DgTransport() = default;
  virtual void h2d(Stream s, int32_t slot, int32_t block) = 0;  // every part, host block -> slot
  virtual void d2h(int32_t slot, int32_t block) = 0;            // every part, slot -> block, on kD2h
  virtual void d2h_part(Stream s, int32_t slot, int32_t block, uint32_t part) = 0;
  virtual uint32_t parts() const = 0;
  virtual uint64_t part_bytes(uint32_t part) const = 0;
  virtual void write_entry(Stream s, uint32_t key, int32_t v) = 0;  // slot_of[key] = v after s's earlier work
  // True: the entry of a fetched unit (key -> its slot) is published by the transport with its landed() call, after
  // the unit's copies (the core then never calls write_entry for it).
  virtual bool publishes_landed() const { return false; }
  virtual void signal_ready(uint32_t g, uint32_t seq) = 0;  // ready[g] = seq after the layer's copies (and landed())
  virtual void* event_create() = 0;
  virtual void event_destroy(void* ev) = 0;
  virtual void record(void* ev, Stream s) = 0;
  virtual void wait(Stream s, void* ev) = 0;
  virtual bool done(void* ev) = 0;
  virtual void event_sync(void* ev) = 0;
  virtual void sync(Stream s) = 0;
  virtual bool query(void* ev) = 0;  // non-blocking: the event's last record has completed
  virtual void upload_table(const int32_t* table, uint32_t n) = 0;  // the whole table on kDem, then sync
  // Three-tier: the unit's bytes from its file into staging block `block` (blocks .. blocks + disk_staging - 1: the
  // host layout of a unit), synchronously; the core then copies it in from that block as from a pinned home.
  virtual void read_unit(uint32_t key, int32_t block);
  // Before h2d(s, slot, block): slot_ev / block_ev (either may be null) are the write-backs that may still read the
  // slot or write the block. The default makes s wait for both; a transport that tracks its copies per part may let
  // each part of the next h2d wait only for the same part of those write-backs.
  virtual void wait_copy_in(Stream s, int32_t slot, int32_t block, void* slot_ev, void* block_ev) {
    (void)slot, (void)block;
    if (slot_ev) wait(s, slot_ev);
    if (block_ev) wait(s, block_ev);
  }
  // A deferred write-back (slot -> block, every part) the core has just recorded at the boundary, with write-backs on
  // kD2h. It will submit it later, part by part (d2h_part on kD2h), by its credit or when it needs the slot; meanwhile
  // neither the slot nor the block is written by anything else. A transport may copy it now on kD2h and make the
  // later d2h_part calls of the same (slot, block, part) no-ops (default: nothing).
  virtual void prestage(int32_t slot, int32_t block) { (void)slot, (void)block; }
  // Units just copied in (key, slot) on stream s: one call per fetch, right after its copies (a demand's before the
  // layer's signal_ready). A transport that verifies landed bytes enqueues the check here (default: nothing).
  virtual void landed(Stream s, uint32_t g, const uint32_t* keys, const int32_t* slots, uint32_t n) {
    (void)s, (void)g, (void)keys, (void)slots, (void)n;
  }
};

struct DgConfig {
  std::vector<uint32_t> n_units;  // per gated layer
  uint32_t persistent_slots = 0;  // R + D
  uint32_t bank_slots = 0;        // per bank (dg_max_ids)
  uint32_t blocks = 0;            // P + Q
  uint32_t spare_target = 0;
  uint32_t prefetch_reserve = 0;
  bool prefetch_reserve_auto = false;
  uint32_t prefetch_per_layer = 4, prefetch_per_token = 48;
  bool wb_defer = true, wb_on_d2h = true;
  uint64_t wb_layer_bytes = 0, wb_max_outstanding = 0;
  uint32_t inclusive = 0;  // device units that may keep their block as a clean copy
  // Three-tier (SS_DG_DISK_TIER): keys off the device and without a pinned home live in their file (Home::File) and
  // a miss reads them through one of disk_staging staging buffers (round robin). home_blocks: the blocks that are
  // pinned homes at open (the plan's pinned units; the rest of `blocks` are spares). Pinned homes keep a recency list
  // (most recently homed first); a victim that needs a block while none is free takes the least recently homed pinned
  // unit's (that unit goes to its file, disk_drops), or with no pinned unit left goes to its file itself
  // (disk_discards). clean_evict: such a victim goes to its file at once, no pinned unit displaced. disk_prefetch:
  // a prefetch may read a file-homed unit.
  bool disk_tier = false, disk_prefetch = false, clean_evict = false;
  uint32_t home_blocks = 0, disk_staging = 0;
  // Scored eviction (SS_POLICY_SCORED / SCORED_AUTO): the boundary takes its victims lowest score first instead of
  // from the recency tail; every other decision is LRU's. Weights in thousandths (each 0..1000, sum 1000). max_ids:
  // the ids of one export (a union's upper bound), 1..64. scored_auto: learn every token, but rank only at a boundary
  // closing more than one verify row (end_token(rows > 1)); otherwise the recency tail.
  bool scored = false, scored_auto = false;
  uint32_t w_trans = 700, w_freq = 200, w_rec = 100;
  uint32_t max_ids = 0;
};

struct DgCounts {  // the subset of ss_dg_stats this core counts
  uint64_t tokens = 0, lookups = 0, misses = 0, covered = 0, fetched = 0, prefetched = 0, prefetch_used = 0;
  uint64_t pred_invalid = 0, resurrected = 0, bank_serves = 0, collected_mid = 0, evicted = 0, evict_short = 0;
  uint64_t writebacks_done = 0, stalled = 0, predicted = 0, predicted_true = 0, miss_layers = 0, covered_waits = 0;
  uint64_t wb_deferred = 0, wb_cancelled = 0, wb_forced = 0, wb_boundary_flushed = 0;
  uint64_t wb_issued_bytes = 0, wb_completed_bytes = 0, wb_cancelled_bytes = 0, wb_boundary_flushed_bytes = 0;
  uint64_t wb_forced_wait_ns = 0, inclusive_kept = 0, inclusive_drops = 0;
  uint64_t disk_reads = 0, disk_read_bytes = 0, disk_stage_waits = 0, disk_drops = 0, disk_discards = 0;
  uint64_t clean_drops = 0, clean_drop_bytes = 0;
  // scored eviction: boundaries that had to use the recency order (a gated layer not served this token: never expected
  // under this core's one-export-per-layer service); victims taken in score order; layers and eligible keys the
  // selection considered; transition increments lost to a saturated cell; selection time.
  uint64_t score_fallbacks = 0, scored_victims = 0, score_layers = 0, score_candidates = 0, score_saturated = 0;
  uint64_t score_ns = 0;
};
struct DgLayerCounts {
  uint64_t lookups = 0, misses = 0, fetched = 0, bank_serves = 0, prefetched = 0, prefetch_used = 0, evicted = 0;
};

class DgCore {
 public:
  enum class Home : uint8_t { Host, Device, Coming, Bank, Evicting, File };

  DgCore(const DgConfig& cfg, DgTransport* t);
  ~DgCore();
  DgCore(const DgCore&) = delete;
  DgCore& operator=(const DgCore&) = delete;

  // Open: the first persistent_slots - spare_target distinct keys of `priority` take slots 0.. (the first one most
  // recent); every other key takes a block, in key order; free slots are a stack with the lowest on top. Three-tier:
  // `disk` flags the plan's file-tier keys; of the keys off the device, the plan-pinned ones and then the file-tier
  // ones, each in `priority` order, take pinned homes up to home_blocks (blocks in key order; the recency list in
  // priority order, the first most recent), every other key lives in its file.
  void place(const std::vector<uint32_t>& priority, const std::vector<uint8_t>* disk = nullptr);
  uint32_t keys() const { return keys_; }
  uint32_t gated() const { return uint32_t(base_.size() - 1); }
  uint32_t units(uint32_t g) const { return base_[g + 1] - base_[g]; }
  uint32_t key(uint32_t g, uint32_t u) const { return base_[g] + u; }
  uint32_t gated_of(uint32_t k) const;
  const std::vector<uint32_t>& unit_base() const { return base_; }
  const std::vector<int32_t>& table() const { return table_; }
  Home home(uint32_t k) const { return e_[k].home; }
  int32_t slot_of(uint32_t k) const { return e_[k].slot; }
  int32_t block_of(uint32_t k) const { return e_[k].block; }
  uint32_t free_slots() const { return uint32_t(free_slots_.size()); }
  uint32_t free_blocks() const { return uint32_t(free_blocks_.size()); }
  const std::vector<int32_t>& free_block_ids() const { return free_blocks_; }  // the free stack, top last
  uint32_t on_device() const { return on_device_; }
  uint32_t file_units() const { return on_file_; }
  std::vector<uint32_t> host_order() const;  // three-tier: the pinned homes, most recently homed first
  uint32_t backed_units() const { return backed_; }
  uint64_t outstanding_bytes() const { return outstanding_; }
  uint32_t deferred() const { return uint32_t(deferred_.size()); }
  const DgCounts& counts() const { return st_; }
  const std::vector<DgLayerCounts>& layer_counts() const { return lc_; }
  std::vector<uint32_t> residency() const;  // device keys, most recent first

  // run: the gated layers this token exports (null: all); a layer left out keeps its score history unchanged
  void begin_token(uint32_t seq, const std::vector<uint8_t>* run = nullptr);
  // mask: the ids whose entry the canonical schedule sees absent (the host mirror before this layer's service), which
  // every count and fetch follows; dev_mask (default: mask): the ids the export kernel saw absent in the device table,
  // whose readers wait for the layer's ready word. A device-only bit is an entry still in flight (a prefetch that had
  // not landed when the layer exported): its readers wait for that copy, and nothing is counted for it.
  void serve_demand(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask, uint64_t dev_mask);
  void serve_demand(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask) { serve_demand(g, ids, n, mask, mask); }
  // The canonical mask of layer g's export: the ids in range whose mirror entry is absent.
  uint64_t canonical_mask(uint32_t g, const uint32_t* ids, uint32_t n) const;
  void serve_use(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask);
  void serve_prediction(uint32_t g_next, const uint32_t* pred, uint32_t n);
  void issue_writebacks(uint32_t g);  // the deferred write-back slice after layer g's service
  // rows: the verify rows the token closed (scored_auto ranks only above one); keep: keys this boundary must not
  // evict (every gated layer's ss_dg_keep set), out-of-range keys ignored
  void end_token(uint32_t rows = 1, const std::vector<uint32_t>& keep = {});
  // Between tokens: deferral of write-backs on or off; turning it off first submits every deferred write-back. The
  // per-token credit and carry restart as after open. Placement and submission only: the same bytes.
  void set_wb_defer(bool on);
  bool wb_defer() const { return c_.wb_defer; }
  void drain();  // between tokens: every deferred write-back submitted, every stream synchronized
  void set_spare_target(uint32_t n);
  void set_prefetch_budget(uint32_t per_layer, uint32_t per_token);
  uint32_t spare_target() const { return c_.spare_target; }
  void check() const;  // ownership invariants (tests); throws SS_E_BACKEND naming the first broken rule

  // ---- scored eviction ----
  static constexpr uint32_t kScoreWindow = 16;       // unions in each layer's frequency ring
  static constexpr uint32_t kScoreMaxUnits = 65536;  // units per gated layer (the integer bounds rest on it)
  // Starting transition counts, at open (after place, before the first token): per gated layer units^2 uint32
  // little-endian cells row-major [previous unit][unit], layers concatenated. They are also the state set_policy
  // restores.
  void load_counts(const unsigned char* cells);
  // Between tokens: drains every write-back, switches LRU (0) / SCORED (1) / SCORED_AUTO (2), resets the learned
  // state to the open counts (or zero) and every demand epoch, and renumbers the recency stamps in list order.
  // Switching to scoring needs the tables, so an open under LRU refuses it.
  void set_policy(uint32_t policy);
  uint32_t policy() const { return c_.scored ? (c_.scored_auto ? 2u : 1u) : 0u; }
  uint64_t epoch() const { return epoch_; }
  uint64_t stamp_counter() const { return stamp_; }
  void set_stamp_counter(uint64_t v) { stamp_ = v; }  // tests: start near the limit
  // Past this the next token fails before it changes anything, so the stamp counter never wraps.
  static constexpr uint64_t kStampLimit = UINT64_MAX - (uint64_t(1) << 40);

 private:
  static constexpr uint32_t kNone = 0xffffffffu;
  struct Entry {
    Home home = Home::Host;
    int32_t slot = -1, block = -1;
    uint32_t prev = kNone, next = kNone;
    bool in_list = false, wb_pending = false, via_prefetch = false, used = false, backed = false;
    void* pf_done = nullptr;
    uint32_t hprev = kNone, hnext = kNone;  // three-tier: the pinned homes' recency list
    bool in_hlist = false;
    uint64_t demand_epoch = 0;  // scored: the token of its last demand use (0: none since open or a policy switch)
    uint64_t stamp = 0;         // scored: its last push to the recency list (unique; larger = more recent)
  };
  // Scored eviction, per gated layer: transition counts T[r][e] (saturating uint32, row-major) with exact row sums,
  // the ring of the last kScoreWindow unions with per-unit counts over it, the previous and this token's union.
  struct LayerScore {
    std::vector<uint32_t> T, open_T;
    std::vector<uint64_t> rowsum;
    std::vector<uint16_t> cnt;
    std::vector<uint32_t> ring;  // kScoreWindow rows of max_ids
    std::vector<uint8_t> ring_len;
    uint32_t ring_head = 0, ring_n = 0;
    std::vector<uint32_t> prev, cur;
    uint64_t served = 0;  // the token whose union cur holds
  };
  struct Cand {
    uint64_t s, epoch, stamp;
    uint32_t key;
  };
  static bool cand_less(const Cand& a, const Cand& b) {
    if (a.s != b.s) return a.s < b.s;
    if (a.epoch != b.epoch) return a.epoch < b.epoch;
    return a.stamp < b.stamp;
  }
  struct Writeback {
    uint32_t key;
    int32_t slot, block;
    void* done;
    bool discard;
    uint64_t bytes;
  };
  struct Deferred {
    uint32_t key;
    int32_t slot, block;
    uint32_t parts_done;
    uint64_t bytes;
  };

  void unlink(uint32_t k);
  void push_front(uint32_t k);
  void* event();
  uint32_t collect();
  void submit_part(Deferred& d);
  void* record_deferred_front(bool discard);
  void* finish_deferred_front();
  void force_free_slot();
  int32_t take_bank_slot(uint32_t g);
  void write_entry(DgTransport::Stream s, uint32_t k, int32_t v, bool landing = false);
  bool fetch(uint32_t g, uint32_t unit, bool prefetch);
  void cover(uint32_t g, uint32_t unit);
  void use(uint32_t g, uint32_t unit, bool was_miss);
  // Leaves the device (or a bank) without a write-back: its block is its home again (the recency head), else
  // (three-tier, no block) its file.
  void to_lower(uint32_t k);
  void hpush(uint32_t k);    // a pinned home now (three-tier: at the recency head)
  void hunlink(uint32_t k);  // no longer a pinned home
  bool drop_host_lru();      // three-tier: the least recently homed pinned unit to its file, its block free
  int32_t take_stage();      // three-tier: the next staging buffer, its last copy out of it landed
  bool clean_now() const { return c_.clean_evict && c_.disk_tier && free_blocks_.empty(); }
  void attach(std::vector<void*>& where, int32_t i, void* ev);
  void detach(std::vector<void*>& where, int32_t i);
  void sweep_events();
  void score_history(uint32_t g);  // serve_use: layer g's union into the counts, the ring and the previous union
  // The `need` smallest eligible candidates of every gated layer, ascending, into heap_.
  void select_scored(size_t need);
  Cand score_of(uint32_t g, uint32_t u, uint64_t denom, const Cand* cutoff) const;
  void reset_score();
  bool eligible(uint32_t k) const {
    return e_[k].home == Home::Device && !e_[k].wb_pending && (keep_.empty() || !keep_[k]);
  }
  void apply_wb_defer();  // the write-back stream, layer credit and outstanding cap of c_.wb_defer
  bool accept_victim(uint32_t k);  // the boundary's acceptance of one victim; false: no block for it (evict_short)
  bool on_device_or_coming(uint32_t g, uint32_t unit) const {
    const Home h = e_[key(g, unit)].home;
    return h == Home::Device || h == Home::Coming || h == Home::Bank;
  }

  DgConfig c_;
  DgTransport* t_;
  std::vector<uint32_t> base_;
  uint32_t keys_ = 0, slots_ = 0, bank_first_ = 0;
  std::vector<Entry> e_;
  std::vector<int32_t> table_;
  std::vector<int32_t> free_slots_, free_blocks_;
  uint32_t head_ = kNone, tail_ = kNone, on_device_ = 0, on_host_ = 0, backed_ = 0;
  uint32_t hhead_ = kNone, htail_ = kNone, on_file_ = 0, stage_next_ = 0;
  std::vector<void*> stage_ev_;  // [disk_staging]: the last copy out of each staging buffer
  std::vector<uint32_t> coming_, banked_, bank_key_;
  uint32_t bank_seq_[2] = {0, 0}, bank_layer_[2] = {kNone, kNone}, bank_next_[2] = {0, 0};
  std::deque<Writeback> wbs_;
  std::deque<Deferred> deferred_;
  uint64_t unit_bytes_ = 0, outstanding_ = 0, layer_bytes_ = 0, max_outstanding_ = 0;
  int64_t credit_ = 0;
  size_t prev_evict_ = 0;
  DgTransport::Stream wb_stream_ = DgTransport::kDem;
  void* post_ready_ev_ = nullptr;
  std::vector<uint32_t> pf_layer_;
  uint32_t pf_token_ = 0, seq_ = 0, pred_layer_ = kNone;
  std::vector<uint8_t> layer_missed_, run_;
  std::vector<uint32_t> pred_, uniq_, victims_;
  std::vector<void*> event_pool_, all_events_;
  std::vector<void*> slot_ev_, block_ev_;        // a write-back still copying out of the slot / into the block
  std::unordered_map<void*, int> ev_refs_;      // attachments of each such event
  DgCounts st_;
  std::vector<DgLayerCounts> lc_;
  std::vector<LayerScore> sc_;  // scored: one per gated layer (empty under an LRU open)
  std::vector<Cand> heap_;
  std::vector<uint8_t> keep_;  // during end_token: the keys its keep list protects (empty: none)
  uint64_t epoch_ = 0, stamp_ = 0, open_stamp_ = 0;
};

}  // namespace tsa
