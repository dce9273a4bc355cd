#include "dg_core.hpp"

#include <algorithm>
#include <chrono>
#include <string>

#include "common.hpp"

namespace tsa {
namespace {
[[noreturn]] void broken(const std::string& what) { fail(SS_E_BACKEND, "device-gated cache invariant: " + what); }
}  // namespace

DgCore::DgCore(const DgConfig& cfg, DgTransport* t) : c_(cfg), t_(t) {
  base_.assign(1, 0);
  uint64_t n = 0;
  for (uint32_t u : c_.n_units) {
    n += u;
    require(n < 0x7fffffffull, SS_E_INVALID, "device-gated: more than 2^31 - 1 gated units");
    base_.push_back(uint32_t(n));
  }
  keys_ = uint32_t(n);
  require(c_.persistent_slots >= 1 && c_.spare_target <= c_.persistent_slots, SS_E_INVALID,
          "device-gated: spare target above the persistent slots");
  const uint64_t slots = uint64_t(c_.persistent_slots) + 2ull * c_.bank_slots;
  require(slots < 0x7fffffffull, SS_E_INVALID, "device-gated: more than 2^31 - 1 slots");
  slots_ = uint32_t(slots);
  bank_first_ = c_.persistent_slots;
  e_.assign(keys_, Entry{});
  table_.assign(keys_, -1);
  bank_key_.assign(2u * size_t(c_.bank_slots), kNone);
  pf_layer_.assign(gated(), 0);
  layer_missed_.assign(gated(), 0);
  run_.assign(gated(), 1);
  lc_.assign(gated(), DgLayerCounts{});
  slot_ev_.assign(slots_, nullptr);
  block_ev_.assign(c_.blocks, nullptr);
  if (c_.prefetch_reserve_auto) c_.prefetch_reserve = std::min<uint32_t>(24, c_.spare_target / 4);
  require(t_->parts() >= 1, SS_E_INVALID, "device-gated: a unit without parts");
  for (uint32_t p = 0; p < t_->parts(); ++p) unit_bytes_ += t_->part_bytes(p);
  require(c_.inclusive < c_.blocks || c_.inclusive == 0, SS_E_INVALID,
          "device-gated: the inclusive share must leave a block for write-backs");
  require(!c_.disk_tier || c_.disk_staging >= 1, SS_E_INVALID, "device-gated: the disk tier needs staging buffers");
  require(c_.disk_tier || (!c_.disk_prefetch && !c_.disk_staging && !c_.home_blocks && !c_.clean_evict), SS_E_INVALID,
          "device-gated: disk options without the disk tier");
  if (c_.disk_tier) stage_ev_.assign(c_.disk_staging, nullptr);
  apply_wb_defer();
  if (c_.scored) {  // every table now: the service never allocates
    require(c_.w_trans <= 1000 && c_.w_freq <= 1000 && c_.w_rec <= 1000 && c_.w_trans + c_.w_freq + c_.w_rec == 1000,
            SS_E_INVALID, "device-gated: score weights must each be 0..1000 and sum to 1000");
    require(c_.max_ids >= 1 && c_.max_ids <= 64, SS_E_INVALID, "device-gated: score unions need max ids 1..64");
    sc_.resize(gated());
    for (uint32_t g = 0; g < gated(); ++g) {
      const size_t n = units(g);
      require(n <= kScoreMaxUnits, SS_E_INVALID,
              "device-gated: scored eviction needs at most 65536 units per gated layer (gated layer " +
                  std::to_string(g) + " has " + std::to_string(n) + ")");
      LayerScore& l = sc_[g];
      l.T.assign(n * n, 0u);
      l.rowsum.assign(n, 0);
      l.cnt.assign(n, 0);
      l.ring.assign(size_t(kScoreWindow) * c_.max_ids, 0u);
      l.ring_len.assign(kScoreWindow, 0);
      l.prev.reserve(c_.max_ids);
      l.cur.reserve(c_.max_ids);
    }
    heap_.reserve(c_.persistent_slots);
  }
  victims_.reserve(c_.persistent_slots);
}

DgCore::~DgCore() {
  for (void* ev : all_events_) t_->event_destroy(ev);
}

uint32_t DgCore::gated_of(uint32_t k) const {
  return uint32_t(std::upper_bound(base_.begin(), base_.end(), k) - base_.begin()) - 1;
}

void* DgCore::event() {
  if (!event_pool_.empty()) {
    void* ev = event_pool_.back();
    event_pool_.pop_back();
    return ev;
  }
  void* ev = t_->event_create();
  all_events_.push_back(ev);
  return ev;
}

// ---- write-back events attached to slots and blocks ----
// A write-back is collected in bookkeeping when the canonical schedule says so (see the header); until its D2H has
// really finished, its event stays attached to the slot it reads and the block it writes, and any copy into that slot
// or out of that block first makes its stream wait for it (device side).
void DgCore::attach(std::vector<void*>& where, int32_t i, void* ev) {
  if (where[size_t(i)]) detach(where, i);
  where[size_t(i)] = ev;
  ++ev_refs_[ev];
}

void DgCore::detach(std::vector<void*>& where, int32_t i) {
  void* ev = where[size_t(i)];
  if (!ev) return;
  where[size_t(i)] = nullptr;
  auto it = ev_refs_.find(ev);
  if (it == ev_refs_.end()) broken("a write-back event without references");
  if (--it->second == 0) {
    ev_refs_.erase(it);
    event_pool_.push_back(ev);
  }
}

void DgCore::sweep_events() {
  for (uint32_t s = 0; s < slots_; ++s)
    if (slot_ev_[s] && t_->query(slot_ev_[s])) detach(slot_ev_, int32_t(s));
  for (uint32_t b = 0; b < c_.blocks; ++b)
    if (block_ev_[b] && t_->query(block_ev_[b])) detach(block_ev_, int32_t(b));
}

void DgTransport::read_unit(uint32_t, int32_t) {
  fail(SS_E_UNSUPPORTED, "device-gated: this transport cannot read a unit from its file");
}

void DgCore::place(const std::vector<uint32_t>& priority, const std::vector<uint8_t>* disk) {
  const uint32_t dev_max = c_.persistent_slots - c_.spare_target;
  std::vector<uint8_t> placed(keys_, 0);
  std::vector<uint32_t> order;
  for (uint32_t k : priority) {
    require(k < keys_, SS_E_INVALID, "device-gated: resident key out of range");
    if (!placed[k] && order.size() < dev_max) {
      placed[k] = 1;
      order.push_back(k);
    }
  }
  const uint32_t dev0 = uint32_t(order.size());
  const bool three = c_.disk_tier;
  const std::vector<uint8_t> none(three && !disk ? keys_ : 0, 0);
  if (three && !disk) disk = &none;
  require(!three || disk->size() == keys_, SS_E_INVALID, "device-gated: the disk flags do not cover the keys");
  // three-tier: the keys off the device that get a pinned home, plan-pinned first, then file-tier, each in priority
  // order (the priority list, duplicates dropped, then any key it missed), up to home_blocks
  std::vector<uint8_t> blocked(keys_, 0);
  std::vector<uint32_t> host_rank;
  if (three) {
    std::vector<uint8_t> seen(keys_, 0);
    std::vector<uint32_t> prio;
    for (uint32_t k : priority)
      if (!seen[k]) {
        seen[k] = 1;
        prio.push_back(k);
      }
    for (uint32_t k = 0; k < keys_; ++k)
      if (!seen[k]) prio.push_back(k);
    const uint32_t cap = std::min(c_.home_blocks, c_.blocks);
    for (int pass = 0; pass < 2; ++pass)
      for (uint32_t k : prio)
        if (!placed[k] && (*disk)[k] == uint8_t(pass) && host_rank.size() < cap) {
          blocked[k] = 1;
          host_rank.push_back(k);
        }
  } else {
    require(uint64_t(keys_) - dev0 <= c_.blocks, SS_E_CAPACITY,
            "device-gated: fewer host blocks than non-resident units");
  }
  int32_t next_block = 0;
  on_host_ = on_file_ = backed_ = 0;
  hhead_ = htail_ = kNone;
  for (uint32_t k = 0; k < keys_; ++k) {
    Entry& x = e_[k];
    x = Entry{};
    if (!placed[k] && (!three || blocked[k])) {
      x.home = Home::Host;
      x.block = next_block++;
      if (!three) ++on_host_;
    } else if (!placed[k]) {
      x.home = Home::File;
      ++on_file_;
    }
  }
  for (size_t i = host_rank.size(); i-- > 0;) hpush(host_rank[i]);  // the first by priority most recent
  for (uint32_t i = 0; i < dev0; ++i) {
    Entry& x = e_[order[i]];
    x.home = Home::Device;
    x.slot = int32_t(i);
    table_[order[i]] = x.slot;
  }
  head_ = tail_ = kNone;
  for (uint32_t i = dev0; i-- > 0;) push_front(order[i]);  // the first of the priority list is the most recent
  on_device_ = dev0;
  free_slots_.clear();
  free_blocks_.clear();
  for (uint32_t s = c_.persistent_slots; s-- > dev0;) free_slots_.push_back(int32_t(s));  // lowest on top
  for (int32_t b = int32_t(c_.blocks); b-- > next_block;) free_blocks_.push_back(b);
  open_stamp_ = stamp_;
}

void DgCore::unlink(uint32_t k) {
  Entry& x = e_[k];
  if (!x.in_list) return;
  if (x.prev != kNone) e_[x.prev].next = x.next;
  else head_ = x.next;
  if (x.next != kNone) e_[x.next].prev = x.prev;
  else tail_ = x.prev;
  x.prev = x.next = kNone;
  x.in_list = false;
}

void DgCore::push_front(uint32_t k) {
  Entry& x = e_[k];
  x.prev = kNone;
  x.next = head_;
  if (head_ != kNone) e_[head_].prev = k;
  else tail_ = k;
  head_ = k;
  x.in_list = true;
  if (c_.scored) {  // begin_token keeps the counter below kStampLimit, so this never wraps
    if (stamp_ == UINT64_MAX) broken("the recency stamp counter wrapped");
    x.stamp = ++stamp_;
  }
}

std::vector<uint32_t> DgCore::residency() const {
  std::vector<uint32_t> out;
  for (uint32_t k = head_; k != kNone; k = e_[k].next)
    if (e_[k].home == Home::Device) out.push_back(k);
  return out;
}

void DgCore::write_entry(DgTransport::Stream s, uint32_t k, int32_t v, bool landing) {
  table_[k] = v;
  if (!(landing && t_->publishes_landed())) t_->write_entry(s, k, v);
}

// Every recorded write-back is complete in bookkeeping: the key's block is its home and its slot is free (a discarded
// one - the key was resurrected - only returns its block). The events stay attached until the copies really ended.
uint32_t DgCore::collect() {
  uint32_t n = 0;
  while (!wbs_.empty()) {
    Writeback& w = wbs_.front();
    Entry& x = e_[w.key];
    x.wb_pending = false;
    if (w.discard) {
      free_blocks_.push_back(w.block);
      attach(block_ev_, w.block, w.done);
    } else {
      x.home = Home::Host;
      x.block = w.block;
      x.slot = -1;
      hpush(w.key);
      free_slots_.push_back(w.slot);
      attach(slot_ev_, w.slot, w.done);
      attach(block_ev_, w.block, w.done);
    }
    ++n;
    outstanding_ -= w.bytes;
    st_.wb_completed_bytes += w.bytes;
    auto it = ev_refs_.find(w.done);
    if (it == ev_refs_.end()) event_pool_.push_back(w.done);  // (attached to nothing: a discard of a zero-part record)
    wbs_.pop_front();
  }
  st_.writebacks_done += n;
  return n;
}

void DgCore::submit_part(Deferred& d) {
  const uint32_t p = d.parts_done;
  t_->d2h_part(wb_stream_, d.slot, d.block, p);
  ++d.parts_done;
  const uint64_t b = t_->part_bytes(p);
  d.bytes += b;
  outstanding_ += b;
  st_.wb_issued_bytes += b;
}

void* DgCore::record_deferred_front(bool discard) {
  Deferred& d = deferred_.front();
  void* ev = event();
  t_->record(ev, wb_stream_);
  wbs_.push_back({d.key, d.slot, d.block, ev, discard, d.bytes});
  deferred_.pop_front();
  return ev;
}

void* DgCore::finish_deferred_front() {
  Deferred& d = deferred_.front();
  while (d.parts_done < t_->parts()) submit_part(d);
  return record_deferred_front(false);
}

void DgCore::issue_writebacks(uint32_t g) {
  if (deferred_.empty()) {
    credit_ = 0;
    return;
  }
  if (g + 1 >= gated()) return;  // nothing after the last gated layer
  const int64_t grant = int64_t(layer_bytes_);
  credit_ = std::min(credit_ + grant, grant);  // a debt carries over, unused credit does not
  st_.collected_mid += collect();
  bool after_ready = false;
  while (credit_ > 0 && !deferred_.empty() && outstanding_ < max_outstanding_) {
    if (wb_stream_ == DgTransport::kD2h && !after_ready) {  // behind the ready already on the demand stream
      t_->record(post_ready_ev_, DgTransport::kDem);
      t_->wait(DgTransport::kD2h, post_ready_ev_);
      after_ready = true;
    }
    Deferred& d = deferred_.front();
    credit_ -= int64_t(t_->part_bytes(d.parts_done));
    if (d.parts_done + 1 == t_->parts()) finish_deferred_front();
    else submit_part(d);
  }
}

// A demand without a free slot while victims are deferred: finish the deferred front (its remaining parts), collect,
// until a persistent slot is free.
void DgCore::force_free_slot() {
  while (free_slots_.empty() && !deferred_.empty()) {
    bool live = false;
    for (const Writeback& w : wbs_) live = live || !w.discard;
    if (!live) finish_deferred_front();
    ++st_.wb_forced;
    st_.collected_mid += collect();
  }
}

// A demand bank slot of gated layer g: bank g & 1, reused two gated layers later; its previous alias is unpublished.
int32_t DgCore::take_bank_slot(uint32_t g) {
  const uint32_t b = g & 1u;
  if (bank_seq_[b] != seq_ || bank_layer_[b] != g) {
    bank_seq_[b] = seq_;
    bank_layer_[b] = g;
    bank_next_[b] = 0;
  }
  if (bank_next_[b] >= c_.bank_slots) return -1;
  const uint32_t idx = b * c_.bank_slots + bank_next_[b]++;
  const int32_t slot = int32_t(bank_first_ + idx);
  const uint32_t old = bank_key_[idx];
  if (old != kNone && e_[old].home == Home::Bank && e_[old].slot == slot) {
    to_lower(old);  // its block, or (read from its file) its file
    write_entry(DgTransport::kDem, old, -1);
  }
  bank_key_[idx] = kNone;
  return slot;
}

void DgCore::to_lower(uint32_t k) {
  Entry& x = e_[k];
  x.slot = -1;
  if (x.backed) {
    x.backed = false;
    --backed_;
  }
  if (x.block >= 0) {
    x.home = Home::Host;
    hpush(k);
  } else {
    if (!c_.disk_tier) broken("a key without a block left the device without a write-back");
    x.home = Home::File;
    ++on_file_;
  }
}

// ---- three-tier: the pinned homes' recency list (most recently homed at the head) ----
void DgCore::hpush(uint32_t k) {
  ++on_host_;
  if (!c_.disk_tier) return;
  Entry& x = e_[k];
  x.hprev = kNone;
  x.hnext = hhead_;
  if (hhead_ != kNone) e_[hhead_].hprev = k;
  else htail_ = k;
  hhead_ = k;
  x.in_hlist = true;
}

void DgCore::hunlink(uint32_t k) {
  --on_host_;
  if (!c_.disk_tier) return;
  Entry& x = e_[k];
  if (!x.in_hlist) broken("a pinned home outside the recency list");
  if (x.hprev != kNone) e_[x.hprev].hnext = x.hnext;
  else hhead_ = x.hnext;
  if (x.hnext != kNone) e_[x.hnext].hprev = x.hprev;
  else htail_ = x.hprev;
  x.hprev = x.hnext = kNone;
  x.in_hlist = false;
}

std::vector<uint32_t> DgCore::host_order() const {
  std::vector<uint32_t> out;
  for (uint32_t k = hhead_; k != kNone; k = e_[k].hnext) out.push_back(k);
  return out;
}

// The least recently homed pinned unit goes to its file (no copy: the file holds its bytes) and its block is free at
// once (a pinned home's block is quiescent: nothing copies into or out of it).
bool DgCore::drop_host_lru() {
  if (!c_.disk_tier || htail_ == kNone) return false;
  const uint32_t k = htail_;
  Entry& x = e_[k];
  hunlink(k);
  free_blocks_.push_back(x.block);
  x.block = -1;
  x.home = Home::File;
  ++on_file_;
  ++st_.disk_drops;
  return true;
}

// The next staging buffer (round robin); the copy that last read it must have landed before a read overwrites it.
int32_t DgCore::take_stage() {
  const uint32_t i = stage_next_;
  stage_next_ = (i + 1) % c_.disk_staging;
  if (stage_ev_[i] && !t_->query(stage_ev_[i])) {
    t_->event_sync(stage_ev_[i]);
    ++st_.disk_stage_waits;
  }
  return int32_t(c_.blocks + i);
}

void DgCore::begin_token(uint32_t seq, const std::vector<uint8_t>* run) {
  require(!run || run->size() == gated(), SS_E_INVALID, "device-gated: the exported layers do not cover the gated layers");
  if (c_.scored) {  // this token's epoch (the first is 1); one token pushes far fewer than 2^40 stamps
    require(stamp_ <= kStampLimit, SS_E_BACKEND,
            "device-gated: the scored eviction's recency stamp counter is exhausted (reopen the context)");
    require(epoch_ < (uint64_t(1) << 63), SS_E_BACKEND, "device-gated: the scored eviction's epoch counter is exhausted");
    ++epoch_;
  }
  if (run) std::copy(run->begin(), run->end(), run_.begin());
  else std::fill(run_.begin(), run_.end(), uint8_t(1));
  seq_ = seq;
  pf_token_ = 0;
  std::fill(pf_layer_.begin(), pf_layer_.end(), 0u);
  std::fill(layer_missed_.begin(), layer_missed_.end(), uint8_t(0));
  pred_.clear();
  pred_layer_ = kNone;
}

bool DgCore::fetch(uint32_t g, uint32_t unit, bool prefetch) {
  const uint32_t k = key(g, unit);
  Entry& x = e_[k];
  if (prefetch && (pf_layer_[g] >= c_.prefetch_per_layer || pf_token_ >= c_.prefetch_per_token)) return false;
  switch (x.home) {
    case Home::Coming:
    case Home::Device:
    case Home::Bank:
      return false;
    case Home::Evicting: {  // resurrection: the slot still holds the bytes (the write-back only reads them)
      bool done = false;
      for (auto it = deferred_.begin(); it != deferred_.end() && !done; ++it) {
        if (it->key != k) continue;
        done = true;
        if (it->parts_done == 0) {  // nothing submitted: the record goes, its block returns unread
          const int32_t b = it->block;
          deferred_.erase(it);
          free_blocks_.push_back(b);
          x.wb_pending = false;
          ++st_.wb_cancelled;
          st_.wb_cancelled_bytes += unit_bytes_;
        } else {  // partly submitted (only the front): its event after the sent parts, discarded
          if (it != deferred_.begin()) broken("parts submitted behind the deferred front");
          st_.wb_cancelled_bytes += unit_bytes_ - it->bytes;
          record_deferred_front(true);
        }
        break;
      }
      if (!done)
        for (Writeback& w : wbs_)
          if (w.key == k && !w.discard) {
            w.discard = true;
            break;
          }
      x.home = Home::Device;
      x.block = -1;
      write_entry(DgTransport::kDem, k, x.slot);
      push_front(k);
      ++on_device_;
      ++st_.resurrected;
      return true;
    }
    case Home::Host:
      break;
    case Home::File:  // three-tier: read from its file below; a prefetch only with disk_prefetch
      if (prefetch && !c_.disk_prefetch) return false;
      break;
  }
  int32_t slot = -1;
  bool bank = false;
  const size_t reserve = prefetch ? c_.prefetch_reserve : 0u;
  if (free_slots_.size() <= reserve) st_.collected_mid += collect();
  if (!prefetch && free_slots_.empty()) force_free_slot();
  if (free_slots_.size() > reserve) {
    slot = free_slots_.back();
    free_slots_.pop_back();
  } else if (prefetch) {
    return false;
  } else {
    slot = take_bank_slot(g);
    if (slot >= 0) {
      bank = true;
    } else {  // a layer has at most bank_slots distinct misses: only an internal error reaches here
      force_free_slot();
      while (free_slots_.empty() && !wbs_.empty()) {
        collect();
        ++st_.stalled;
      }
      if (free_slots_.empty()) fail(SS_E_BACKEND, "device-gated: no free slot, no bank slot, no write-back to wait for");
      slot = free_slots_.back();
      free_slots_.pop_back();
    }
  }
  const DgTransport::Stream s = prefetch ? DgTransport::kPf : DgTransport::kDem;
  if (x.home == Home::File) {  // its bytes from its file into a staging buffer, then the same copy from there
    const int32_t stage = take_stage();
    t_->read_unit(k, stage);
    ++st_.disk_reads;
    st_.disk_read_bytes += unit_bytes_;
    t_->wait_copy_in(s, slot, stage, slot_ev_[size_t(slot)], nullptr);  // (no write-back touches a staging buffer)
    detach(slot_ev_, slot);
    t_->h2d(s, slot, stage);
    void*& ev = stage_ev_[uint32_t(stage) - c_.blocks];  // the buffer is reusable once this copy landed
    if (!ev) ev = event();
    t_->record(ev, s);
    --on_file_;
  } else {
    // the slot's last write-back and the block's incoming write-back (if still copying) come first
    t_->wait_copy_in(s, slot, x.block, slot_ev_[size_t(slot)], block_ev_[size_t(x.block)]);
    detach(slot_ev_, slot);
    detach(block_ev_, x.block);
    t_->h2d(s, slot, x.block);
    hunlink(k);
  }
  write_entry(s, k, slot, true);
  x.slot = slot;
  x.via_prefetch = prefetch;
  x.used = false;
  if (prefetch) {
    x.pf_done = event();
    t_->record(x.pf_done, s);
  }
  if (bank) {
    x.home = Home::Bank;
    bank_key_[size_t(slot) - bank_first_] = k;
    banked_.push_back(k);
    ++st_.bank_serves;
    ++lc_[g].bank_serves;
  } else {
    x.home = Home::Coming;
    coming_.push_back(k);
    push_front(k);
    ++on_device_;
  }
  if (prefetch) {
    ++st_.prefetched;
    ++lc_[g].prefetched;
    ++pf_layer_[g];
    ++pf_token_;
  } else {
    ++st_.fetched;
    ++lc_[g].fetched;
  }
  // each unit as soon as its copies are issued: a transport that checks landed bytes checks this unit while the
  // layer's next miss is still copying
  t_->landed(s, g, &k, &slot, 1);
  return true;
}

void DgCore::cover(uint32_t g, uint32_t unit) {
  Entry& x = e_[key(g, unit)];
  if (x.home == Home::Coming && x.via_prefetch && x.pf_done) {  // the layer's readers wait for the prefetch's copies
    t_->wait(DgTransport::kDem, x.pf_done);
    ++st_.covered_waits;
  }
}

void DgCore::use(uint32_t g, uint32_t unit, bool was_miss) {
  const uint32_t k = key(g, unit);
  Entry& x = e_[k];
  ++st_.lookups;
  ++lc_[g].lookups;
  if (was_miss) {
    ++st_.misses;
    ++lc_[g].misses;
    if (!layer_missed_[g]) {
      layer_missed_[g] = 1;
      ++st_.miss_layers;
    }
  }
  if (c_.scored) x.demand_epoch = epoch_;  // demand uses only: prefetches and resurrections leave it
  if (x.via_prefetch && !x.used) {
    x.used = true;
    ++st_.prefetch_used;
    ++lc_[g].prefetch_used;
  }
  if (x.in_list) {
    unlink(k);
    push_front(k);
  }
}

uint64_t DgCore::canonical_mask(uint32_t g, const uint32_t* ids, uint32_t n) const {
  uint64_t m = 0;
  for (uint32_t i = 0; i < n && i < 64; ++i)
    if (ids[i] < units(g) && table_[key(g, ids[i])] < 0) m |= uint64_t(1) << i;
  return m;
}

void DgCore::serve_demand(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask, uint64_t dev_mask) {
  const uint32_t nu = units(g);
  for (uint32_t i = 0; i < n; ++i)
    require(ids[i] < nu, SS_E_INVALID,
            "device-gated: layer " + std::to_string(g) + " exported id " + std::to_string(ids[i]) + " of " +
                std::to_string(nu));
  // per masked occurrence in export order: a repeated id is fetched at its first occurrence, covered at the others
  for (uint32_t i = 0; i < n; ++i) {
    if (!(mask >> i & 1u)) {
      const Entry& x = e_[key(g, ids[i])];
      if ((dev_mask >> i & 1u) && x.home == Home::Coming && x.via_prefetch && x.pf_done)
        t_->wait(DgTransport::kDem, x.pf_done);  // in flight when the layer exported: its readers wait for it
      continue;
    }
    if (on_device_or_coming(g, ids[i])) {
      cover(g, ids[i]);
      ++st_.covered;
    } else {
      fetch(g, ids[i], false);
    }
  }
  // after every fetch's landed(): a transport that checks landed units orders the ready word behind the checks
  if (mask | dev_mask) t_->signal_ready(g, seq_);
}

void DgCore::serve_use(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask) {
  const bool have_pred = pred_layer_ == g;
  uniq_.assign(ids, ids + n);
  std::sort(uniq_.begin(), uniq_.end());
  uniq_.erase(std::unique(uniq_.begin(), uniq_.end()), uniq_.end());
  if (c_.scored) score_history(g);
  for (uint32_t id : uniq_) {
    bool miss = false;
    for (uint32_t i = 0; i < n; ++i)
      if (ids[i] == id && (mask >> i & 1u)) miss = true;
    use(g, id, miss);
    if (have_pred && std::find(pred_.begin(), pred_.end(), id) != pred_.end()) ++st_.predicted_true;
  }
  pred_.clear();
  pred_layer_ = kNone;
}

void DgCore::serve_prediction(uint32_t g_next, const uint32_t* pred, uint32_t n) {
  if (g_next >= gated()) return;
  const uint32_t nu = units(g_next);
  uniq_.clear();
  for (uint32_t i = 0; i < n; ++i) {  // order kept: the budget keeps the head of the list
    if (pred[i] >= nu) {
      ++st_.pred_invalid;
      continue;
    }
    if (std::find(uniq_.begin(), uniq_.end(), pred[i]) == uniq_.end()) uniq_.push_back(pred[i]);
  }
  st_.predicted += uniq_.size();
  pred_.assign(uniq_.begin(), uniq_.end());
  pred_layer_ = g_next;
  for (uint32_t id : pred_) fetch(g_next, id, true);
}

void DgCore::end_token(uint32_t rows, const std::vector<uint32_t>& keep) {
  keep_.clear();
  if (!keep.empty()) {
    keep_.assign(keys_, 0);
    for (uint32_t k : keep)
      if (k < keys_) keep_[k] = 1;
  }
  struct ClearKeep {
    std::vector<uint8_t>& v;
    ~ClearKeep() { v.clear(); }
  } clear_keep{keep_};
  // every copy and entry write of the token has landed before anything changes home
  t_->sync(DgTransport::kDem);
  t_->sync(DgTransport::kPf);
  for (uint32_t k : coming_) {  // admitted: device homes now; their source blocks are free (or kept clean)
    Entry& x = e_[k];
    if (x.home != Home::Coming) continue;
    x.home = Home::Device;
    x.via_prefetch = false;
    if (x.pf_done) {
      event_pool_.push_back(x.pf_done);
      x.pf_done = nullptr;
    }
    if (x.block >= 0) {
      if (backed_ < c_.inclusive) {
        x.backed = true;
        ++backed_;
        ++st_.inclusive_kept;
      } else {
        free_blocks_.push_back(x.block);
        x.block = -1;
      }
    }
  }
  coming_.clear();
  for (uint32_t k : banked_) {  // bank units: back to their blocks (three-tier: read from their file, to it)
    Entry& x = e_[k];
    if (x.home == Home::Bank) {
      to_lower(k);
      table_[k] = -1;
    }
    if (x.pf_done) {
      event_pool_.push_back(x.pf_done);
      x.pf_done = nullptr;
    }
    x.via_prefetch = false;
  }
  banked_.clear();
  std::fill(bank_key_.begin(), bank_key_.end(), kNone);
  bank_seq_[0] = bank_seq_[1] = 0;
  bank_layer_[0] = bank_layer_[1] = kNone;
  collect();
  // victims until free + pending + accepted = the spare target, from the recency tail or (scored) lowest score
  // first; the first victim without a free block ends the acceptance (it stays on the device)
  size_t pending = deferred_.size();
  for (const Writeback& w : wbs_) pending += w.discard ? 0u : 1u;
  const size_t base = free_slots_.size() + pending;
  victims_.clear();
  size_t got = 0;
  bool by_score = c_.scored && (!c_.scored_auto || rows > 1);
  if (by_score) {  // every exported layer's union is this token's (a layer left out scores from its older history)
    bool fresh = true;
    for (uint32_t g = 0; g < gated(); ++g) fresh = fresh && (!run_[g] || sc_[g].served == epoch_);
    if (!fresh) {
      ++st_.score_fallbacks;
      by_score = false;
    }
  }
  if (by_score) {
    const auto t0 = std::chrono::steady_clock::now();
    select_scored(c_.spare_target > base ? c_.spare_target - base : 0);
    for (const Cand& cd : heap_) {
      if (!accept_victim(cd.key)) break;
      ++got;
      ++st_.scored_victims;
    }
    st_.score_ns += uint64_t(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
  } else {
    for (uint32_t k = tail_; k != kNone && base + got < c_.spare_target;) {
      const uint32_t prev = e_[k].prev;
      if (eligible(k)) {
        if (!accept_victim(k)) break;
        ++got;
      }
      k = prev;
    }
  }
  const size_t n_evict = victims_.size();
  t_->upload_table(table_.data(), keys_);  // the device table = the mirror, before any write-back is enqueued
  const size_t n_old = deferred_.size(), carry = std::max(n_evict, prev_evict_);
  const size_t n_flush = n_old > carry ? n_old - carry : 0;
  prev_evict_ = n_evict;
  credit_ = 0;
  for (size_t i = 0; c_.wb_defer && i < n_evict; ++i) {
    const uint32_t k = victims_[i];
    deferred_.push_back({k, e_[k].slot, e_[k].block, 0, 0});
    // (only on the D2H stream: the write-back events this core records on wb_stream_ then follow the copies)
    if (wb_stream_ == DgTransport::kD2h) t_->prestage(e_[k].slot, e_[k].block);
    ++st_.wb_deferred;
    ++st_.evicted;
    ++lc_[gated_of(k)].evicted;
  }
  const uint64_t issued0 = st_.wb_issued_bytes;
  size_t n_issued = 0;
  for (; n_issued < n_flush; ++n_issued) finish_deferred_front();
  st_.wb_boundary_flushed += n_issued;
  st_.wb_boundary_flushed_bytes += st_.wb_issued_bytes - issued0;
  for (size_t i = 0; !c_.wb_defer && i < n_evict; ++i) {
    const uint32_t k = victims_[i];
    const Entry& x = e_[k];
    t_->d2h(x.slot, x.block);
    void* ev = event();
    t_->record(ev, DgTransport::kD2h);
    wbs_.push_back({k, x.slot, x.block, ev, false, unit_bytes_});
    outstanding_ += unit_bytes_;
    st_.wb_issued_bytes += unit_bytes_;
    ++st_.evicted;
    ++lc_[gated_of(k)].evicted;
  }
  sweep_events();
  ++st_.tokens;
}

bool DgCore::accept_victim(uint32_t k) {
  Entry& x = e_[k];
  // a clean copy (its block is its home again), or three-tier with no block to write into after the least recently
  // homed pinned unit was offered (clean_evict: not even that): its file. No copy either way.
  const bool clean = !x.backed && clean_now();
  if (x.backed || clean || (free_blocks_.empty() && !drop_host_lru() && c_.disk_tier)) {
    if (x.backed) ++st_.inclusive_drops;
    else ++st_.disk_discards;
    if (clean) {
      ++st_.clean_drops;
      st_.clean_drop_bytes += unit_bytes_;
    }
    unlink(k);
    --on_device_;
    free_slots_.push_back(x.slot);
    to_lower(k);
    table_[k] = -1;
    ++st_.evicted;
    ++lc_[gated_of(k)].evicted;
    return true;
  }
  if (free_blocks_.empty()) {
    ++st_.evict_short;
    return false;
  }
  const int32_t b = free_blocks_.back();
  free_blocks_.pop_back();
  unlink(k);
  --on_device_;
  x.home = Home::Evicting;
  x.block = b;
  x.wb_pending = true;
  table_[k] = -1;
  victims_.push_back(k);
  return true;
}

// Layer g's sorted unique union (uniq_) becomes this token's: every cell (r in the previous token's union, e in this
// one) takes one saturating increment and its row sum with it; the union enters the ring of the last kScoreWindow
// unions (the oldest leaves it, the per-unit counts follow) and becomes the previous one.
void DgCore::score_history(uint32_t g) {
  LayerScore& l = sc_[g];
  const uint32_t n = units(g);
  require(uniq_.size() <= c_.max_ids, SS_E_BACKEND, "device-gated: a score union above max ids");
  l.cur.assign(uniq_.begin(), uniq_.end());
  l.served = epoch_;
  for (uint32_t r : l.prev) {
    uint32_t* row = l.T.data() + size_t(r) * n;
    uint64_t added = 0;
    for (uint32_t e : l.cur) {
      if (row[e] == UINT32_MAX) {
        ++st_.score_saturated;
      } else {
        ++row[e];
        ++added;
      }
    }
    l.rowsum[r] += added;
  }
  if (l.ring_n == kScoreWindow) {
    const uint32_t* old = l.ring.data() + size_t(l.ring_head) * c_.max_ids;
    for (uint32_t i = 0; i < l.ring_len[l.ring_head]; ++i) --l.cnt[old[i]];
    l.ring_head = (l.ring_head + 1) % kScoreWindow;
    --l.ring_n;
  }
  const uint32_t at = (l.ring_head + l.ring_n) % kScoreWindow;
  std::copy(l.cur.begin(), l.cur.end(), l.ring.begin() + ptrdiff_t(size_t(at) * c_.max_ids));
  l.ring_len[at] = uint8_t(l.cur.size());
  ++l.ring_n;
  for (uint32_t e : l.cur) ++l.cnt[e];
  l.prev.assign(l.cur.begin(), l.cur.end());
}

// Unit u of layer g, with cur = this token's union of g and denom = the sum of its rows' sums:
//   N = sum_{r in cur} T[r][u], P = ((|cur| N) << 16) / max(1, denom), F = (cnt[u] << 16) / kScoreWindow,
//   Rec = (1 << 16) / (1 + epoch - demand_epoch), S = w_t P + w_f F + w_r Rec
// in unsigned integers with floor division. With at most 65536 units and 64 ids, N < 2^38 and denom < 2^54, so
// (|cur| N) << 16 < 2^60; N <= denom bounds P by 2^22 and S below 2^33. Every term is nonnegative: when the F + Rec part alone does not order before
// `cutoff` the transition rows are not read (the result then orders after the cutoff anyway).
DgCore::Cand DgCore::score_of(uint32_t g, uint32_t u, uint64_t denom, const Cand* cutoff) const {
  const LayerScore& l = sc_[g];
  const Entry& x = e_[base_[g] + u];
  const uint64_t F = (uint64_t(l.cnt[u]) << 16) / kScoreWindow;
  const uint64_t R = (uint64_t(1) << 16) / (1 + (epoch_ - x.demand_epoch));
  Cand cd{uint64_t(c_.w_freq) * F + uint64_t(c_.w_rec) * R, x.demand_epoch, x.stamp, base_[g] + u};
  if (cutoff && !cand_less(cd, *cutoff)) return cd;
  const uint32_t n = units(g);
  uint64_t N = 0;
  for (uint32_t r : l.cur) N += l.T[size_t(r) * n + u];
  const uint64_t P = ((uint64_t(l.cur.size()) * N) << 16) / std::max<uint64_t>(1, denom);
  cd.s += uint64_t(c_.w_trans) * P;
  return cd;
}

// A max-heap (by the public order) of at most `need` candidates over every eligible key, then sorted ascending: the
// victims are the `need` smallest (score, demand epoch, stamp), a total order since stamps are unique.
void DgCore::select_scored(size_t need) {
  heap_.clear();
  for (uint32_t g = 0; need && g < gated(); ++g) {
    const LayerScore& l = sc_[g];
    uint64_t denom = 0;
    for (uint32_t r : l.cur) denom += l.rowsum[r];
    ++st_.score_layers;
    for (uint32_t u = 0; u < units(g); ++u) {
      if (!eligible(base_[g] + u)) continue;
      ++st_.score_candidates;
      const bool full = heap_.size() == need;
      const Cand cd = score_of(g, u, denom, full ? &heap_.front() : nullptr);
      if (!full) {
        heap_.push_back(cd);
        std::push_heap(heap_.begin(), heap_.end(), cand_less);
      } else if (cand_less(cd, heap_.front())) {
        std::pop_heap(heap_.begin(), heap_.end(), cand_less);
        heap_.back() = cd;
        std::push_heap(heap_.begin(), heap_.end(), cand_less);
      }
    }
  }
  std::sort_heap(heap_.begin(), heap_.end(), cand_less);
}

void DgCore::reset_score() {
  for (uint32_t g = 0; g < uint32_t(sc_.size()); ++g) {
    LayerScore& l = sc_[g];
    const uint32_t n = units(g);
    if (l.open_T.empty()) std::fill(l.T.begin(), l.T.end(), 0u);
    else std::copy(l.open_T.begin(), l.open_T.end(), l.T.begin());
    for (uint32_t r = 0; r < n; ++r) {
      uint64_t sum = 0;
      for (uint32_t e = 0; e < n && !l.open_T.empty(); ++e) sum += l.T[size_t(r) * n + e];
      l.rowsum[r] = sum;
    }
    std::fill(l.cnt.begin(), l.cnt.end(), uint16_t(0));
    std::fill(l.ring.begin(), l.ring.end(), 0u);
    std::fill(l.ring_len.begin(), l.ring_len.end(), uint8_t(0));
    l.ring_head = l.ring_n = 0;
    l.prev.clear();
    l.cur.clear();
    l.served = 0;
  }
  epoch_ = 0;
}

void DgCore::load_counts(const unsigned char* p) {
  require(c_.scored, SS_E_INVALID, "device-gated: starting score counts need policy SCORED or SCORED_AUTO");
  for (uint32_t g = 0; g < gated(); ++g) {
    LayerScore& l = sc_[g];
    for (size_t i = 0; i < l.T.size(); ++i, p += 4)
      l.T[i] = uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
    l.open_T = l.T;
  }
  reset_score();
}

void DgCore::set_policy(uint32_t policy) {
  require(policy <= 2, SS_E_INVALID, "device-gated: policy must be LRU, SCORED or SCORED_AUTO");
  require(!policy || !sc_.empty(), SS_E_INVALID, "device-gated: scoring must be provisioned at open");
  drain();
  collect();
  c_.scored = policy != 0;
  c_.scored_auto = policy == 2;
  reset_score();
  for (Entry& x : e_) x.demand_epoch = x.stamp = 0;
  stamp_ = 0;
  for (uint32_t k = tail_; k != kNone; k = e_[k].prev) e_[k].stamp = ++stamp_;  // the list's order, the head largest
}

void DgCore::apply_wb_defer() {
  if (!c_.wb_defer) {
    wb_stream_ = DgTransport::kDem;
    layer_bytes_ = max_outstanding_ = 0;
    return;
  }
  wb_stream_ = c_.wb_on_d2h ? DgTransport::kD2h : DgTransport::kDem;
  layer_bytes_ = c_.wb_layer_bytes ? c_.wb_layer_bytes : t_->part_bytes(0);
  max_outstanding_ = c_.wb_max_outstanding ? c_.wb_max_outstanding : 2 * unit_bytes_;
  if (c_.wb_on_d2h && !post_ready_ev_) post_ready_ev_ = event();
}

void DgCore::set_wb_defer(bool on) {
  if (on == c_.wb_defer) return;
  if (!on)
    while (!deferred_.empty()) finish_deferred_front();  // recorded write-backs now, collected as any other
  c_.wb_defer = on;
  apply_wb_defer();
  credit_ = 0;
  prev_evict_ = 0;
}

void DgCore::drain() {
  while (!deferred_.empty()) finish_deferred_front();
  t_->sync(DgTransport::kDem);
  t_->sync(DgTransport::kPf);
  t_->sync(DgTransport::kD2h);
  sweep_events();
}

void DgCore::set_spare_target(uint32_t n) {
  require(n <= c_.persistent_slots, SS_E_INVALID, "device-gated: spare target above the persistent slots");
  c_.spare_target = n;
  if (c_.prefetch_reserve_auto) c_.prefetch_reserve = std::min<uint32_t>(24, n / 4);
}

void DgCore::set_prefetch_budget(uint32_t per_layer, uint32_t per_token) {
  c_.prefetch_per_layer = per_layer;
  c_.prefetch_per_token = per_token;
}

void DgCore::check() const {
  std::vector<uint8_t> slot_used(slots_, 0), block_used(c_.blocks, 0);
  uint32_t dev = 0, host = 0, file = 0;
  for (uint32_t k = 0; k < keys_; ++k) {
    const Entry& x = e_[k];
    switch (x.home) {
      case Home::Device:
      case Home::Coming:
        ++dev;
        [[fallthrough]];
      case Home::Bank:
      case Home::Evicting:
        if (x.slot < 0 || uint32_t(x.slot) >= slots_ || slot_used[size_t(x.slot)]++)
          broken("slot of key " + std::to_string(k) + " missing or shared");
        break;
      case Home::Host:
        ++host;
        if (x.slot != -1) broken("a pinned home with a slot");
        if (c_.disk_tier && !x.in_hlist) broken("a pinned home outside the recency list");
        break;
      case Home::File:
        ++file;
        if (!c_.disk_tier || x.slot != -1 || x.block != -1 || table_[k] >= 0)
          broken("file home of key " + std::to_string(k) + " with a slot, a block or an entry");
        break;
    }
    if (x.home != Home::Host && x.in_hlist) broken("key " + std::to_string(k) + " in the recency list off its block");
    if (x.block >= 0 && (uint32_t(x.block) >= c_.blocks || block_used[size_t(x.block)]++))
      broken("block of key " + std::to_string(k) + " shared");
    if ((x.home == Home::Host || x.home == Home::Evicting || (x.home == Home::Bank && !c_.disk_tier)) && x.block < 0)
      broken("key " + std::to_string(k) + " has no block in a home that needs one");
    if (x.home == Home::Device && table_[k] != x.slot) broken("device key " + std::to_string(k) + " unpublished");
    if ((x.home == Home::Host || x.home == Home::Evicting) && table_[k] >= 0)
      broken("key " + std::to_string(k) + " published while off the device");
  }
  for (int32_t s : free_slots_)
    if (slot_used[size_t(s)]++) broken("free slot " + std::to_string(s) + " also owned");
  for (int32_t b : free_blocks_)
    if (block_used[size_t(b)]++) broken("free block " + std::to_string(b) + " also owned");
  for (const Writeback& w : wbs_)
    if (w.discard && block_used[size_t(w.block)]++) broken("a discarded write-back's block also owned");
  if (dev != on_device_) broken("device count");
  if (host != on_host_) broken("pinned count");
  if (file != on_file_) broken("file count");
  if (c_.disk_tier) {
    uint32_t n = 0;
    for (uint32_t k = hhead_; k != kNone; k = e_[k].hnext)
      if (++n > keys_ || e_[k].home != Home::Host) broken("the pinned recency list");
    if (n != on_host_) broken("the pinned recency list's length");
  }
  if (c_.scored) {  // stamps fall strictly from the recency head; no epoch lies ahead of the token's
    uint64_t last = UINT64_MAX;
    for (uint32_t k = head_; k != kNone; k = e_[k].next) {
      if (e_[k].stamp >= last || e_[k].stamp == 0 || e_[k].stamp > stamp_) broken("recency stamps");
      last = e_[k].stamp;
    }
    for (uint32_t k = 0; k < keys_; ++k)
      if (e_[k].demand_epoch > epoch_) broken("a demand epoch in the future");
    for (const LayerScore& l : sc_) {
      uint32_t in_ring = 0, counted = 0;
      for (uint32_t i = 0; i < l.ring_n; ++i) in_ring += l.ring_len[(l.ring_head + i) % kScoreWindow];
      for (uint16_t c : l.cnt) counted += c;
      if (l.ring_n > kScoreWindow || in_ring != counted) broken("the score ring's counts");
    }
  }
}

}  // namespace tsa
