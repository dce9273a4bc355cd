// Device-gated decode: where every unit of every gated layer lives, and what moves when, with no device API in it (a
// DgTransport does the copies, table writes and events). The MI355X context drives it once per exported layer from
// its service thread and once per token boundary; the CPU test hook drives it on a transport that completes
// everything at once.
//
// Parity: the decisions are the reference core's (src/dg_core.cpp: open placement :769-858, a miss's fetch
// :1146-1368, a layer's service :1415-1634, the boundary :1636-1927, write-back scheduling :961-1097, scored victims
// :1929-2071 with the score of docs/design.md:284-354), so slot tables, homes and counters compare bit for bit with the
// reference's under its eager schedule. The structure is this library's own:
//   - KeyOrder: one intrusive order over keys (two index arrays), used twice - the device recency order (victims come
//     from its back) and, with the file tier, the pinned homes' order (the back one gives up its block first);
//   - one FIFO of write-backs: a sealed prefix (event recorded, complete at the next retire) and a queued tail (parts
//     still to submit, by a per-layer byte credit or when a slot is needed);
//   - EventLedger: the transport's events, pooled, and the write-back events still tied to a slot or a block;
//   - BankSlots: the two per-token banks of dg_max_ids slots that a miss borrows when no persistent slot is free;
//   - LayerHistory: scored eviction's per-layer transition counts and window of recent unions.
//
// Completion: the core only learns that a write-back finished by retiring it (retire_writebacks), which the MI355X
// transport makes true by waiting for the event; it never asks whether the device ran ahead. Placement is therefore a
// function of the route stream alone.
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
  virtual void h2d(Stream s, int32_t slot, int32_t block, uint32_t key) = 0;  // every part of key's unit, block -> slot
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
  // slot: where the copy that follows puts it (a bank slot when the read went into a kept pinned block).
  virtual void read_unit(uint32_t key, int32_t block, int32_t slot);
  // Landings (dg_landing_blocks): the unit's file read into landing block `block` (blocks + disk_staging + l), queued
  // behind the demand reads. The core may copy out of the block (h2d) right after this call: the transport orders
  // that copy after the read, and this read after the block's previous read and its last copy out. Default:
  // read_unit.
  virtual void read_landing(uint32_t key, int32_t block) { read_unit(key, block, -1); }
  // The landing in `block` will never be copied out (it expired): a read not started yet may be dropped (default:
  // nothing).
  virtual void drop_landing(int32_t block) { (void)block; }
  // Before h2d(s, slot, block): slot_ev / block_ev (either may be null) are the write-backs that may still read the
  // slot or write the block. The default makes s wait for both; a transport that tracks its copies per part may let
  // each part of the next h2d wait only for the same part of those write-backs.
  virtual void wait_copy_in(Stream s, int32_t slot, int32_t block, void* slot_ev, void* block_ev) {
    (void)slot, (void)block;
    if (slot_ev) wait(s, slot_ev);
    if (block_ev) wait(s, block_ev);
  }
  // A queued write-back (slot -> block, every part) the core has just chosen at the boundary, with write-backs on
  // kD2h. It will submit it later, part by part (d2h_part on kD2h), by its credit or when it needs the slot; meanwhile
  // neither the slot nor the block is written by anything else. A transport may copy it now on kD2h and make the
  // later d2h_part calls of the same (slot, block, part) no-ops (default: nothing).
  virtual void prestage(int32_t slot, int32_t block) { (void)slot, (void)block; }
  // The core dropped a queued write-back (slot -> block) before submitting any part of it (its unit came back). A
  // transport that prestaged it forgets it; its copy may still run: the core then ties the slot and the block to an
  // event recorded on the write-back stream, so that the block's next user (a file read, a copy into the slot) waits
  // for it (default: nothing).
  virtual void unqueue(int32_t slot, int32_t block) { (void)slot, (void)block; }
  // Units just copied in (key, slot) on stream s: one call per fetch, right after its copies (a demand's before the
  // layer's signal_ready). A transport that verifies landed bytes enqueues the check here (default: nothing).
  virtual void landed(Stream s, uint32_t g, const uint32_t* keys, const int32_t* slots, uint32_t n) {
    (void)s, (void)g, (void)keys, (void)slots, (void)n;
  }
  // dg_diag timing marks (default: nothing): which 0 = before layer g's first copy, 2 = after its first miss's copies,
  // 1 = after its ready word; the boundary begins; the boundary has issued its write-backs.
  virtual void diag_mark(uint32_t g, int which) { (void)g, (void)which; }
  virtual void diag_boundary() {}
  virtual void diag_writebacks_issued() {}
};

struct DgBoundaryTimes {  // the last boundary's host microseconds by phase, its write-back victims, boundaries so far
  uint64_t boundaries = 0;
  uint32_t writebacks = 0;
  double sync_us = 0, select_us = 0, upload_us = 0, issue_us = 0;
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
  // Three-tier (SS_DG_DISK_TIER): keys off the device and without a pinned home live in their file and a miss reads
  // them through one of disk_staging staging buffers (round robin). home_blocks: the blocks that are pinned homes at
  // open (the plan's pinned units; the rest of `blocks` are spares). A victim that needs a block while none is free
  // takes the block of the pinned home that was homed longest ago (that unit goes to its file: disk_drops), or with no
  // pinned home left goes to its file itself (disk_discards). clean_evict: such a victim goes to its file at once.
  // disk_prefetch: a prefetch may read a file-homed unit.
  bool disk_tier = false, disk_prefetch = false, clean_evict = false;
  uint32_t home_blocks = 0, disk_staging = 0;
  // dg_bank_keep (three-tier): a demand file miss served through a bank slot is read into a pinned block - a free one,
  // else the longest-homed pinned unit's (that unit to its file) - which becomes its pinned home when the bank releases
  // it: at the front of the homes' order (1) or behind its front half (2). 0: read through a staging buffer.
  uint32_t bank_keep = 0;
  // dg_landing_blocks (three-tier): a prediction of a file-homed unit reads it into one of landing_blocks landing
  // blocks (never a slot): a demand then copies it from there, as from a pinned block. landing_ttl 0: a landing its
  // target layer did not demand goes back to its file right after that layer's demand (and a prediction for a layer
  // already served this token lands nothing); N >= 1: one not demanded for N boundaries goes back to its file.
  uint32_t landing_blocks = 0, landing_ttl = 0;
  // Scored eviction (SS_POLICY_SCORED / SCORED_AUTO): the boundary takes its victims lowest score first instead of
  // from the back of the recency order; every other decision stays LRU's. Weights in thousandths (each 0..1000, sum
  // 1000). max_ids: the ids of one export (a union's upper bound), 1..64. scored_auto: learn every token, but rank
  // only at a boundary closing more than one verify row; otherwise the recency order.
  bool scored = false, scored_auto = false;
  uint32_t w_trans = 700, w_freq = 200, w_rec = 100;
  uint32_t max_ids = 0;
};

struct DgCounts {  // the subset of ss_dg_stats this core counts (the ABI's field names)
  uint64_t tokens = 0, lookups = 0, misses = 0, covered = 0, fetched = 0, prefetched = 0, prefetch_used = 0;
  uint64_t pred_invalid = 0, resurrected = 0, bank_serves = 0, collected_mid = 0, evicted = 0, evict_short = 0;
  uint64_t writebacks_done = 0, stalled = 0, predicted = 0, predicted_true = 0, miss_layers = 0, covered_waits = 0;
  uint64_t wb_deferred = 0, wb_cancelled = 0, wb_forced = 0, wb_boundary_flushed = 0;
  uint64_t wb_issued_bytes = 0, wb_completed_bytes = 0, wb_cancelled_bytes = 0, wb_boundary_flushed_bytes = 0;
  uint64_t wb_forced_wait_ns = 0, inclusive_kept = 0, inclusive_drops = 0;
  uint64_t disk_reads = 0, disk_read_bytes = 0, disk_stage_waits = 0, disk_drops = 0, disk_discards = 0;
  uint64_t clean_drops = 0, clean_drop_bytes = 0;
  // dg_bank_keep: reads kept in a pinned block; pinned units dropped to their file for one; such a dropped unit read
  // from its file again within 8 tokens
  uint64_t bank_kept = 0, bank_keep_drops = 0, bank_keep_rereads = 0;
  // dg_landing_blocks: landing reads issued; demands served from a landing block; landings back to their file at a
  // boundary (TTL) and right after their target layer (TTL 0); advice dropped with no free landing block; predictions
  // for a layer already served (TTL 0); the bytes of the reads issued
  uint64_t landing_issued = 0, landing_promoted = 0, landing_expired = 0, landing_expired_layer = 0;
  uint64_t landing_dropped_full = 0, landing_skipped_passed = 0, landing_read_bytes = 0;
  // the physical side of landings, which the core never sees (the context adds its transport's): demands of a landing
  // whose read still ran, host waits for a landing block's reuse, reads dropped before they started, demand reads a
  // part-way landing read gave its readers to, bytes not read of reads dropped part-way, failed landing reads
  uint64_t landing_late = 0, landing_wait_ns = 0, landing_cancelled = 0, landing_yields = 0;
  uint64_t landing_aborted_bytes = 0, landing_failed = 0;
  // scored eviction: boundaries that fell back to the recency order (an exported gated layer whose union is not this
  // token's); victims taken in score order; layers and eligible keys the selection considered; transition increments
  // lost to a saturated cell; selection time.
  uint64_t score_fallbacks = 0, scored_victims = 0, score_layers = 0, score_candidates = 0, score_saturated = 0;
  uint64_t score_ns = 0;
};
struct DgLayerCounts {
  uint64_t lookups = 0, misses = 0, fetched = 0, bank_serves = 0, prefetched = 0, prefetch_used = 0, evicted = 0;
};

// An order over keys 0..n-1 (each in it at most once) with constant-time insertion and removal. It also keeps the
// boundary after its first size() / 2 keys (the front half), so a key can go in at the middle in constant time.
class KeyOrder {
 public:
  static constexpr uint32_t kEnd = 0xffffffffu;
  void reset(uint32_t n);
  bool has(uint32_t k) const { return member_[k] != 0; }
  void put_front(uint32_t k);
  void put_middle(uint32_t k);  // right behind the front half (as it was before k joined)
  void remove(uint32_t k);
  uint32_t front() const { return front_; }
  uint32_t back() const { return back_; }
  uint32_t toward_back(uint32_t k) const { return link_[2 * size_t(k)]; }
  uint32_t toward_front(uint32_t k) const { return link_[2 * size_t(k) + 1]; }
  uint32_t size() const { return n_; }
  bool half_consistent() const;  // the front half is exactly the first size() / 2 keys (tests)

 private:
  void link_after(uint32_t k, uint32_t prev);  // prev kEnd: at the front
  void rebalance();
  std::vector<uint32_t> link_;  // per key: [toward the back, toward the front]
  std::vector<uint8_t> member_;  // 0: out; 1: in the back half; 2: in the front half
  uint32_t front_ = kEnd, back_ = kEnd, n_ = 0;
  uint32_t half_last_ = kEnd, half_n_ = 0;  // the front half's last key and its size
};

class DgCore {
 public:
  // Pinned: its host block is its home. Resident: a persistent slot. Arriving: copied into a persistent slot this
  // token (resident from the boundary on). InBank: copied into a bank slot for this token only. Draining: chosen at a
  // boundary, its write-back into a block not yet retired (the slot still holds its bytes). File: three-tier only.
  // Landed: its home is still its file, and its read into a landing block was issued (no slot, block or entry); a
  // demand copies it from there.
  enum class Where : uint8_t { Pinned, Resident, Arriving, InBank, Draining, File, Landed };

  DgCore(const DgConfig& cfg, DgTransport* t);
  ~DgCore();
  DgCore(const DgCore&) = delete;
  DgCore& operator=(const DgCore&) = delete;

  // Open: the first persistent_slots - spare_target distinct keys of `priority` take slots 0.. (the first one the most
  // recent); every other key takes a block, in key order; free slots are a stack with the lowest on top. Three-tier:
  // `disk` flags the plan's file-tier keys; of the keys off the device, the plan-pinned ones and then the file-tier
  // ones, each in `priority` order, take pinned homes up to home_blocks (blocks in key order; the first by priority
  // the most recently homed), every other key lives in its file.
  void seat(const std::vector<uint32_t>& priority, const std::vector<uint8_t>* disk = nullptr);
  uint32_t keys() const { return keys_; }
  uint32_t gated() const { return uint32_t(first_key_.size() - 1); }
  uint32_t units(uint32_t g) const { return first_key_[g + 1] - first_key_[g]; }
  uint32_t key(uint32_t g, uint32_t u) const { return first_key_[g] + u; }
  uint32_t gated_of(uint32_t k) const;
  const std::vector<uint32_t>& unit_base() const { return first_key_; }
  const std::vector<int32_t>& table() const { return mirror_; }
  Where where(uint32_t k) const { return st_[k].where; }
  int32_t slot_of(uint32_t k) const { return st_[k].slot; }
  int32_t block_of(uint32_t k) const { return st_[k].block; }
  uint32_t free_slots() const { return uint32_t(free_slot_.size()); }
  uint32_t free_blocks() const { return uint32_t(free_block_.size()); }
  const std::vector<int32_t>& free_block_ids() const { return free_block_; }  // the free stack, top last
  uint32_t on_device() const { return n_device_; }
  uint32_t file_units() const { return n_file_; }  // three-tier: file-homed keys (landings included)
  uint32_t landing_units() const { return n_land_; }
  uint32_t landing_free() const { return uint32_t(free_land_.size() + land_busy_.size()); }
  const std::vector<uint32_t>& landing_owners() const { return land_owner_; }  // per landing block: its key, or ~0
  std::vector<uint32_t> pinned_order() const;  // three-tier: the pinned homes, most recently homed first
  uint32_t clean_copies() const { return n_clean_; }
  uint64_t outstanding_bytes() const { return in_flight_bytes_; }
  uint32_t queued_writebacks() const { return uint32_t(wb_.size() - sealed_); }
  const DgCounts& counts() const { return n_; }
  const DgBoundaryTimes& boundary_times() const { return bt_; }
  const std::vector<DgLayerCounts>& layer_counts() const { return per_layer_; }
  std::vector<uint32_t> device_order() const;  // device keys, most recent first

  // run: the gated layers this token exports (null: all); a layer left out keeps its score history unchanged
  void open_token(uint32_t seq, const std::vector<uint8_t>* run = nullptr);
  // The ids of layer g's export whose mirror entry is absent (in range only): the misses the eager schedule sees.
  uint64_t absent_mask(uint32_t g, const uint32_t* ids, uint32_t n) const;
  // Layer g exported `ids`. mask: the misses every count and fetch follows (absent_mask before this call). dev_mask
  // (default: mask): the ids the export kernel saw absent in the device table, whose readers wait for the layer's
  // ready word. A device-only bit is an entry still in flight (a prefetch that had not landed when the layer
  // exported): its readers wait for that copy, and nothing is counted for it.
  void serve_misses(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask, uint64_t dev_mask);
  void serve_misses(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask) { serve_misses(g, ids, n, mask, mask); }
  // Layer g computed with `ids` (after serve_misses): lookups, misses, recency, the prediction's hits, the history.
  void note_uses(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask);
  // A prediction of gated layer g_next's ids, made while an earlier layer computes: prefetched in list order within
  // the per-layer and per-token budgets.
  void prefetch_next(uint32_t g_next, const uint32_t* pred, uint32_t n);
  void spend_wb_credit(uint32_t g);  // the queued write-backs' slice after layer g's service
  // rows: the verify rows the token closed (scored_auto ranks only above one); keep: keys this boundary must not
  // choose (every gated layer's ss_dg_keep set), out-of-range keys ignored
  void close_token(uint32_t rows = 1, const std::vector<uint32_t>& keep = {});
  // Between tokens: queueing of write-backs on or off; turning it off first submits every queued write-back. The
  // per-token credit and carry restart as after open. Placement and submission only: the same bytes.
  void defer_writebacks(bool on);
  bool wb_defer() const { return c_.wb_defer; }
  void quiesce();  // between tokens: every queued write-back submitted, every stream synchronized
  void set_spare_target(uint32_t n);
  void set_clean_evict(bool on) { c_.clean_evict = on; }  // (only a file tier has a victim to drop to its file)
  void set_prefetch_budget(uint32_t per_layer, uint32_t per_token);
  uint32_t spare_target() const { return c_.spare_target; }
  void audit() const;  // ownership invariants (tests); throws SS_E_BACKEND naming the first broken rule

  // ---- scored eviction ----
  static constexpr uint32_t kWindow = 16;             // unions in each layer's frequency window
  static constexpr uint32_t kMaxScoredUnits = 65536;  // units per gated layer (the integer bounds rest on it)
  // Starting transition counts, at open (after seat, before the first token): per gated layer units^2 uint32
  // little-endian cells row-major [previous unit][unit], layers concatenated. A policy switch restores them.
  void seed_transitions(const unsigned char* cells);
  // Between tokens: quiesces, switches LRU (0) / SCORED (1) / SCORED_AUTO (2), restores the learned state to the open
  // counts (or zero) and every demand token, and renumbers the recency stamps in the order's sequence. Switching to
  // scoring needs the tables, so an open under LRU refuses it.
  void set_policy(uint32_t policy);
  uint32_t policy() const { return c_.scored ? (c_.scored_auto ? 2u : 1u) : 0u; }
  // Past this the next token fails before it changes anything, so the stamp counter never wraps.
  static constexpr uint64_t kStampLimit = UINT64_MAX - (uint64_t(1) << 40);

 private:
  static constexpr uint32_t kNoKey = 0xffffffffu;

  struct KeyState {
    Where where = Where::Pinned;
    int32_t slot = -1, block = -1;
    bool wb_open = false;    // a write-back record of this key is not retired yet
    bool ahead = false;      // copied in by a prefetch this token
    bool ahead_hit = false;  // ... and since used
    bool clean = false;      // resident with its block kept as a clean copy
    bool home_middle = false;  // dg_bank_keep 2: its kept block becomes its home behind the front half of the order
    void* ahead_ev = nullptr;  // the prefetch's copy
    uint64_t demand_token = 0;  // scored: the token of its last demand use (0: none since open or a policy switch)
    uint64_t dropped_for_keep = 0;  // dg_bank_keep: 1 + the tokens closed when a kept read took its block (0: none)
    int32_t land = -1;              // Landed: its landing block (0 .. landing_blocks - 1)
    uint32_t land_age = 0;          // Landed: boundaries since it landed
  };

  // A victim's copy into its block. Sealed: its event recorded after its last submitted part; it completes in the
  // bookkeeping at the next retire (dropped: the key came back before it finished, so only the block returns).
  struct WriteBack {
    uint32_t key;
    int32_t slot, block;
    uint32_t parts_sent;
    uint64_t bytes_sent;
    void* ev;
    bool dropped;
  };

  // The transport's events: a pool, and the write-back events still tied to a slot or a block (a copy into that slot,
  // or out of that block, waits for them first; a tie ends when the event has completed or is replaced).
  class EventLedger {
   public:
    void init(DgTransport* t, uint32_t slots, uint32_t blocks);
    void destroy_all();
    void* take();
    void give(void* ev) { pool_.push_back(ev); }
    void* on_slot(int32_t s) const { return slot_[size_t(s)]; }
    void* on_block(int32_t b) const { return block_[size_t(b)]; }
    void tie_slot(int32_t s, void* ev) { tie(slot_, s, ev); }
    void tie_block(int32_t b, void* ev) { tie(block_, b, ev); }
    void untie_slot(int32_t s) { untie(slot_, s); }
    void untie_block(int32_t b) { untie(block_, b); }
    void release_if_loose(void* ev);  // back to the pool unless tied somewhere
    void sweep();                     // untie every completed event

   private:
    void tie(std::vector<void*>& at, int32_t i, void* ev);
    void untie(std::vector<void*>& at, int32_t i);
    DgTransport* t_ = nullptr;
    std::vector<void*> pool_, made_, slot_, block_;
    std::unordered_map<void*, uint32_t> ties_;
  };

  // Two banks of B slots after the persistent ones; layer g borrows from bank g & 1, which restarts for each new
  // (token, layer) pair, so a layer's bank slots stay untouched while the next gated layer borrows from the other.
  class BankSlots {
   public:
    void init(uint32_t first_slot, uint32_t per_bank);
    // The next slot of layer g's bank in token seq (-1: the bank is used up); *held: the key last copied into it.
    int32_t borrow(uint32_t g, uint32_t seq, uint32_t* held);
    void hold(int32_t slot, uint32_t k) { holder_[size_t(slot) - first_] = k; }
    void clear();

   private:
    uint32_t first_ = 0, per_ = 0;
    uint32_t seq_[2] = {0, 0}, layer_[2] = {kNoKey, kNoKey}, used_[2] = {0, 0};
    std::vector<uint32_t> holder_;
  };

  // Scored eviction, one per gated layer: transition counts T[r][e] (saturating uint32, row-major) with exact row sums,
  // a window of the last kWindow unions with per-unit occurrence counts over it, and the previous and current union.
  class LayerHistory {
   public:
    void init(uint32_t units, uint32_t max_ids);
    void set_open(const unsigned char* le_cells);  // the open counts (little-endian uint32)
    void restore();                                // the open counts, an empty window and no unions
    // The token's sorted unique union: one saturating increment per cell (previous union x this one); returns the
    // increments lost to saturation.
    uint64_t learn(const std::vector<uint32_t>& uni, uint64_t token);
    uint64_t served() const { return served_; }
    uint64_t denominator() const;        // sum of the row sums over the current union
    uint64_t pull(uint32_t u) const;     // sum over the current union r of T[r][u]
    uint32_t cur_size() const { return uint32_t(cur_.size()); }
    uint32_t seen(uint32_t u) const { return occ_[u]; }
    bool consistent() const;

   private:
    uint32_t n_ = 0, max_ids_ = 0;
    std::vector<uint32_t> T_, open_T_;
    std::vector<uint64_t> row_sum_;
    std::vector<uint16_t> occ_;
    std::vector<uint32_t> win_;     // kWindow rows of max_ids
    std::vector<uint8_t> win_len_;
    uint32_t win_first_ = 0, win_n_ = 0;
    std::vector<uint32_t> prev_, cur_;
    uint64_t served_ = 0;  // the token whose union cur_ holds
  };

  // A victim candidate in score order: (score, demand token, stamp), a total order since stamps are unique.
  struct Ranked {
    uint64_t score, demand, stamp;
    uint32_t key;
    bool operator<(const Ranked& o) const {
      if (score != o.score) return score < o.score;
      if (demand != o.demand) return demand < o.demand;
      return stamp < o.stamp;
    }
  };

  // recency
  void touch(uint32_t k);   // to the front of the device order (and, scored, a new stamp)
  void make_pinned(uint32_t k);   // its block is its home now (three-tier: the most recently homed)
  void leave_pinned(uint32_t k);  // copied in (its block stays its until the boundary)
  // to its block, else (three-tier, none) its file; no copy
  void fall_back(uint32_t k);
  bool give_up_oldest_home();  // three-tier: the longest-homed pinned unit to its file, its block free
  int32_t block_to_keep();     // dg_bank_keep: a free block, else the longest-homed unit's; -1: none (stage it)
  int32_t next_stage();        // three-tier: the next staging buffer, its last copy out of it landed

  // write-backs
  void send_part(WriteBack& w);
  void seal_first_queued(bool dropped);
  void finish_first_queued();
  uint32_t retire_writebacks();
  void free_a_slot();  // a demand miss with no free slot: submit and retire until one is free
  void apply_wb_mode();  // the write-back stream, layer credit and in-flight cap of the current mode

  // service
  void publish(DgTransport::Stream s, uint32_t k, int32_t v, bool from_copy = false);
  bool bring_in(uint32_t g, uint32_t u, bool ahead);
  bool resurrect(uint32_t k);
  bool on_device_or_arriving(uint32_t k) const {
    const Where w = st_[k].where;
    return w == Where::Resident || w == Where::Arriving || w == Where::InBank;
  }

  // landings
  int32_t land_block(int32_t l) const { return int32_t(c_.blocks + c_.disk_staging) + l; }
  bool advise_land(uint32_t g, uint32_t u);  // true: the landing path took the prediction (a bring_in must not)
  void land(uint32_t k);
  void unland(uint32_t k);       // back to its file, its landing block free
  void reclaim_lands();          // landing blocks copied out of since the last reclaim: free
  void expire_layer_landings(uint32_t g, const uint32_t* ids, uint32_t n);

  // boundary
  bool choose(uint32_t k);  // one victim; false: no block to write it into (evict_short)
  bool choosable(uint32_t k) const {
    return st_[k].where == Where::Resident && !st_[k].wb_open && (kept_.empty() || !kept_[k]);
  }
  void rank_by_score(size_t want);  // the `want` lowest-ranked choosable keys, ascending, into ranked_
  Ranked rank_of(uint32_t g, uint32_t u, uint64_t denom, const Ranked* bar) const;
  bool clean_evict_now() const { return c_.clean_evict && c_.disk_tier && free_block_.empty(); }

  DgConfig c_;
  DgTransport* t_;
  std::vector<uint32_t> first_key_;  // per gated layer, and the total last
  uint32_t keys_ = 0, slots_ = 0;
  std::vector<KeyState> st_;
  std::vector<uint64_t> stamp_of_;  // scored: each key's last move to the front (unique; larger = more recent)
  std::vector<int32_t> mirror_;     // the host copy of the device table
  std::vector<int32_t> free_slot_, free_block_;
  KeyOrder recent_, homed_;
  uint32_t n_device_ = 0, n_pinned_ = 0, n_clean_ = 0, n_file_ = 0;
  uint32_t stage_cursor_ = 0;
  std::vector<void*> stage_ev_;  // [disk_staging]: the last copy out of each staging buffer
  std::vector<uint32_t> arriving_, in_bank_;
  std::vector<int32_t> free_land_, land_busy_;  // free landing blocks (a stack, block 0 on top at open); copied out of
  std::vector<uint32_t> land_owner_;            // per landing block: its key (kNoKey: free)
  uint32_t n_land_ = 0;
  std::vector<uint8_t> served_;                 // landing_ttl 0: the gated layers whose demand this token served
  BankSlots banks_;
  std::deque<WriteBack> wb_;  // sealed prefix, then the queued tail
  size_t sealed_ = 0;
  uint64_t unit_bytes_ = 0, in_flight_bytes_ = 0, layer_grant_ = 0, in_flight_cap_ = 0;
  int64_t credit_ = 0;
  size_t last_chosen_ = 0;  // write-back victims of the previous boundary
  DgTransport::Stream wb_stream_ = DgTransport::kDem;
  void* after_ready_ev_ = nullptr;
  EventLedger ev_;
  std::vector<uint32_t> ahead_in_layer_;
  uint32_t ahead_in_token_ = 0, seq_ = 0, predicted_layer_ = kNoKey;
  std::vector<uint8_t> layer_missed_, exported_;
  std::vector<uint32_t> predicted_, scratch_ids_, chosen_;
  DgCounts n_;
  std::vector<DgLayerCounts> per_layer_;
  std::vector<LayerHistory> hist_;  // scored: one per gated layer (empty under an LRU open)
  std::vector<Ranked> ranked_;
  std::vector<uint8_t> kept_;  // during close_token: the keys its keep list protects (empty: none)
  uint64_t token_ = 0, stamp_ = 0;
  DgBoundaryTimes bt_;
};

}  // namespace tsa
