#include "dg_core.hpp"

#include <algorithm>
#include <chrono>
#include <string>

#include "common.hpp"

namespace tsa {
namespace {
[[noreturn]] void broken(const std::string& what) { fail(SS_E_BACKEND, "device-gated state broken: " + what); }
std::string str(uint64_t v) { return std::to_string(v); }
}  // namespace

void DgTransport::read_unit(uint32_t, int32_t, int32_t) {
  fail(SS_E_UNSUPPORTED, "device-gated: this transport has no file tier");
}

// ---- KeyOrder ---------------------------------------------------------------------------------------------------------
void KeyOrder::reset(uint32_t n) {
  link_.assign(2 * size_t(n), kEnd);
  member_.assign(n, 0);
  front_ = back_ = half_last_ = kEnd;
  n_ = half_n_ = 0;
}

void KeyOrder::link_after(uint32_t k, uint32_t prev) {
  const uint32_t next = prev == kEnd ? front_ : link_[2 * size_t(prev)];
  link_[2 * size_t(k)] = next;
  link_[2 * size_t(k) + 1] = prev;
  if (prev == kEnd) front_ = k;
  else link_[2 * size_t(prev)] = k;
  if (next == kEnd) back_ = k;
  else link_[2 * size_t(next) + 1] = k;
  ++n_;
}

void KeyOrder::put_front(uint32_t k) {
  link_after(k, kEnd);
  member_[k] = 2;  // ahead of every key: the front half grows by it
  if (half_n_++ == 0) half_last_ = k;
  rebalance();
}

void KeyOrder::put_middle(uint32_t k) {
  link_after(k, half_last_);
  member_[k] = 1;
  rebalance();
}

void KeyOrder::remove(uint32_t k) {
  if (member_[k] == 2) {
    --half_n_;
    if (half_last_ == k) half_last_ = toward_front(k);
  }
  const uint32_t behind = link_[2 * size_t(k)], ahead = link_[2 * size_t(k) + 1];
  if (ahead == kEnd) front_ = behind;
  else link_[2 * size_t(ahead)] = behind;
  if (behind == kEnd) back_ = ahead;
  else link_[2 * size_t(behind) + 1] = ahead;
  link_[2 * size_t(k)] = link_[2 * size_t(k) + 1] = kEnd;
  member_[k] = 0;
  --n_;
  rebalance();
}

// Each insertion or removal moves the half's boundary by one key at most.
void KeyOrder::rebalance() {
  const uint32_t want = n_ / 2;
  for (; half_n_ > want; --half_n_) {
    member_[half_last_] = 1;
    half_last_ = toward_front(half_last_);
  }
  for (; half_n_ < want; ++half_n_) {
    half_last_ = half_last_ == kEnd ? front_ : toward_back(half_last_);
    member_[half_last_] = 2;
  }
}

bool KeyOrder::half_consistent() const {
  uint32_t i = 0, last = kEnd;
  for (uint32_t k = front_; k != kEnd; k = toward_back(k), ++i) {
    if (member_[k] != (i < n_ / 2 ? 2 : 1)) return false;
    if (i + 1 == n_ / 2) last = k;
  }
  return i == n_ && half_n_ == n_ / 2 && half_last_ == last;
}

// ---- EventLedger ------------------------------------------------------------------------------------------------------
void DgCore::EventLedger::init(DgTransport* t, uint32_t slots, uint32_t blocks) {
  t_ = t;
  slot_.assign(slots, nullptr);
  block_.assign(blocks, nullptr);
}

void DgCore::EventLedger::destroy_all() {
  for (void* ev : made_) t_->event_destroy(ev);
  made_.clear();
  pool_.clear();
}

void* DgCore::EventLedger::take() {
  if (pool_.empty()) {
    made_.push_back(t_->event_create());
    return made_.back();
  }
  void* ev = pool_.back();
  pool_.pop_back();
  return ev;
}

void DgCore::EventLedger::tie(std::vector<void*>& at, int32_t i, void* ev) {
  untie(at, i);
  at[size_t(i)] = ev;
  ++ties_[ev];
}

void DgCore::EventLedger::untie(std::vector<void*>& at, int32_t i) {
  void* ev = at[size_t(i)];
  if (!ev) return;
  at[size_t(i)] = nullptr;
  const auto it = ties_.find(ev);
  if (it == ties_.end()) broken("a tied write-back event with no count");
  if (--it->second == 0) {
    ties_.erase(it);
    pool_.push_back(ev);
  }
}

void DgCore::EventLedger::release_if_loose(void* ev) {
  if (ties_.find(ev) == ties_.end()) pool_.push_back(ev);
}

void DgCore::EventLedger::sweep() {
  for (size_t s = 0; s < slot_.size(); ++s)
    if (slot_[s] && t_->query(slot_[s])) untie(slot_, int32_t(s));
  for (size_t b = 0; b < block_.size(); ++b)
    if (block_[b] && t_->query(block_[b])) untie(block_, int32_t(b));
}

// ---- BankSlots --------------------------------------------------------------------------------------------------------
void DgCore::BankSlots::init(uint32_t first_slot, uint32_t per_bank) {
  first_ = first_slot;
  per_ = per_bank;
  holder_.assign(2 * size_t(per_bank), kNoKey);
  clear();
}

void DgCore::BankSlots::clear() {
  std::fill(holder_.begin(), holder_.end(), kNoKey);
  for (int b = 0; b < 2; ++b) {
    seq_[b] = 0;
    layer_[b] = kNoKey;
    used_[b] = 0;
  }
}

int32_t DgCore::BankSlots::borrow(uint32_t g, uint32_t seq, uint32_t* held) {
  const uint32_t b = g % 2;
  if (layer_[b] != g || seq_[b] != seq) {  // a new (token, layer): the bank starts over
    seq_[b] = seq;
    layer_[b] = g;
    used_[b] = 0;
  }
  *held = kNoKey;
  if (used_[b] >= per_) return -1;
  const size_t i = size_t(b) * per_ + used_[b]++;
  *held = holder_[i];
  holder_[i] = kNoKey;
  return int32_t(first_ + i);
}

// ---- LayerHistory -----------------------------------------------------------------------------------------------------
void DgCore::LayerHistory::init(uint32_t units, uint32_t max_ids) {
  n_ = units;
  max_ids_ = max_ids;
  T_.assign(size_t(units) * units, 0u);
  row_sum_.assign(units, 0);
  occ_.assign(units, 0);
  win_.assign(size_t(kWindow) * max_ids, 0u);
  win_len_.assign(kWindow, 0);
  prev_.reserve(max_ids);
  cur_.reserve(max_ids);
}

void DgCore::LayerHistory::set_open(const unsigned char* le) {
  open_T_.resize(T_.size());
  for (size_t i = 0; i < open_T_.size(); ++i, le += 4)
    open_T_[i] = uint32_t(le[0]) | uint32_t(le[1]) << 8 | uint32_t(le[2]) << 16 | uint32_t(le[3]) << 24;
}

void DgCore::LayerHistory::restore() {
  if (open_T_.empty()) {
    std::fill(T_.begin(), T_.end(), 0u);
    std::fill(row_sum_.begin(), row_sum_.end(), 0);
  } else {
    T_ = open_T_;
    for (uint32_t r = 0; r < n_; ++r) {
      const uint32_t* row = T_.data() + size_t(r) * n_;
      uint64_t s = 0;
      for (uint32_t e = 0; e < n_; ++e) s += row[e];
      row_sum_[r] = s;
    }
  }
  std::fill(occ_.begin(), occ_.end(), uint16_t(0));
  std::fill(win_.begin(), win_.end(), 0u);
  std::fill(win_len_.begin(), win_len_.end(), uint8_t(0));
  win_first_ = win_n_ = 0;
  prev_.clear();
  cur_.clear();
  served_ = 0;
}

uint64_t DgCore::LayerHistory::learn(const std::vector<uint32_t>& uni, uint64_t token) {
  cur_.assign(uni.begin(), uni.end());
  served_ = token;
  uint64_t lost = 0;
  for (uint32_t r : prev_) {  // the cells (previous union x this union)
    uint32_t* row = T_.data() + size_t(r) * n_;
    for (uint32_t e : cur_) {
      if (row[e] == UINT32_MAX) {
        ++lost;
        continue;
      }
      ++row[e];
      ++row_sum_[r];
    }
  }
  if (win_n_ == kWindow) {  // the oldest union leaves the window
    const uint32_t* old = win_.data() + size_t(win_first_) * max_ids_;
    for (uint32_t i = 0; i < win_len_[win_first_]; ++i) --occ_[old[i]];
    win_first_ = (win_first_ + 1) % kWindow;
    --win_n_;
  }
  const uint32_t at = (win_first_ + win_n_++) % kWindow;
  std::copy(cur_.begin(), cur_.end(), win_.begin() + ptrdiff_t(size_t(at) * max_ids_));
  win_len_[at] = uint8_t(cur_.size());
  for (uint32_t e : cur_) ++occ_[e];
  prev_.assign(cur_.begin(), cur_.end());
  return lost;
}

uint64_t DgCore::LayerHistory::denominator() const {
  uint64_t d = 0;
  for (uint32_t r : cur_) d += row_sum_[r];
  return d;
}

uint64_t DgCore::LayerHistory::pull(uint32_t u) const {
  uint64_t s = 0;
  for (uint32_t r : cur_) s += T_[size_t(r) * n_ + u];
  return s;
}

bool DgCore::LayerHistory::consistent() const {
  if (win_n_ > kWindow) return false;
  uint64_t in_window = 0, counted = 0;
  for (uint32_t i = 0; i < win_n_; ++i) in_window += win_len_[(win_first_ + i) % kWindow];
  for (uint16_t c : occ_) counted += c;
  return in_window == counted;
}

// ---- construction -----------------------------------------------------------------------------------------------------
DgCore::DgCore(const DgConfig& cfg, DgTransport* t) : c_(cfg), t_(t) {
  first_key_.assign(1, 0);
  uint64_t total = 0;
  for (uint32_t u : c_.n_units) {
    total += u;
    require(total < 0x7fffffffull, SS_E_INVALID, "device-gated: the gated layers hold 2^31 - 1 units or more");
    first_key_.push_back(uint32_t(total));
  }
  keys_ = uint32_t(total);
  require(c_.persistent_slots > 0, SS_E_INVALID, "device-gated: no persistent slot");
  require(c_.spare_target <= c_.persistent_slots, SS_E_INVALID,
          "device-gated: spare target " + str(c_.spare_target) + " exceeds the " + str(c_.persistent_slots) +
              " persistent slots");
  const uint64_t slots = uint64_t(c_.persistent_slots) + 2ull * c_.bank_slots;
  require(slots < 0x7fffffffull, SS_E_INVALID, "device-gated: 2^31 - 1 slots or more");
  slots_ = uint32_t(slots);
  require(t_->parts() > 0, SS_E_INVALID, "device-gated: a unit needs at least one part");
  for (uint32_t p = 0; p < t_->parts(); ++p) unit_bytes_ += t_->part_bytes(p);
  require(c_.inclusive == 0 || c_.inclusive < c_.blocks, SS_E_INVALID,
          "device-gated: clean copies may not take every block (write-backs need one)");
  if (c_.disk_tier) {
    require(c_.disk_staging > 0, SS_E_INVALID, "device-gated: the file tier reads through staging buffers; none given");
  } else {
    require(!c_.disk_prefetch && c_.disk_staging == 0 && c_.home_blocks == 0 && !c_.clean_evict, SS_E_INVALID,
            "device-gated: file-tier options given without the file tier");
  }
  require(c_.bank_keep <= 2, SS_E_INVALID, "device-gated: dg_bank_keep is 0, 1 or 2");
  require(c_.disk_tier || !c_.landing_blocks, SS_E_INVALID, "device-gated: landing blocks without the file tier");
  require(uint64_t(c_.blocks) + c_.disk_staging + c_.landing_blocks < 0x7fffffffull, SS_E_INVALID,
          "device-gated: 2^31 - 1 host blocks or more");
  if (c_.prefetch_reserve_auto) c_.prefetch_reserve = std::min<uint32_t>(24, c_.spare_target / 4);

  st_.assign(keys_, KeyState{});
  mirror_.assign(keys_, -1);
  recent_.reset(keys_);
  homed_.reset(keys_);
  ev_.init(t_, slots_, c_.blocks);
  banks_.init(c_.persistent_slots, c_.bank_slots);
  ahead_in_layer_.assign(gated(), 0);
  layer_missed_.assign(gated(), 0);
  exported_.assign(gated(), 1);
  per_layer_.assign(gated(), DgLayerCounts{});
  if (c_.disk_tier) stage_ev_.assign(c_.disk_staging, nullptr);
  served_.assign(gated(), 0);
  free_land_.reserve(c_.landing_blocks);
  land_busy_.reserve(c_.landing_blocks);
  land_owner_.assign(c_.landing_blocks, kNoKey);
  chosen_.reserve(c_.persistent_slots);
  apply_wb_mode();
  if (c_.scored) {  // every table now, so the service never allocates
    require(c_.w_trans <= 1000 && c_.w_freq <= 1000 && c_.w_rec <= 1000, SS_E_INVALID,
            "device-gated: a score weight above 1000");
    require(c_.w_trans + c_.w_freq + c_.w_rec == 1000, SS_E_INVALID,
            "device-gated: the score weights do not add up to 1000");
    require(c_.max_ids >= 1 && c_.max_ids <= 64, SS_E_INVALID, "device-gated: scoring needs 1..64 ids per export");
    hist_.resize(gated());
    for (uint32_t g = 0; g < gated(); ++g) {
      require(units(g) <= kMaxScoredUnits, SS_E_INVALID,
              "device-gated: gated layer " + str(g) + " has " + str(units(g)) + " units; scoring takes at most " +
                  str(kMaxScoredUnits));
      hist_[g].init(units(g), c_.max_ids);
    }
    stamp_of_.assign(keys_, 0);
    ranked_.reserve(c_.persistent_slots);
  }
}

DgCore::~DgCore() { ev_.destroy_all(); }

uint32_t DgCore::gated_of(uint32_t k) const {
  return uint32_t(std::upper_bound(first_key_.begin(), first_key_.end(), k) - first_key_.begin() - 1);
}

// ---- open placement ---------------------------------------------------------------------------------------------------
void DgCore::seat(const std::vector<uint32_t>& priority, const std::vector<uint8_t>* disk) {
  const bool files = c_.disk_tier;
  require(!files || !disk || disk->size() == keys_, SS_E_INVALID, "device-gated: file-tier flags for the wrong keys");
  // each key's first position in the priority list (absent keys after it, in key order)
  std::vector<uint64_t> rank(keys_, UINT64_MAX);
  for (size_t i = 0; i < priority.size(); ++i) {
    require(priority[i] < keys_, SS_E_INVALID, "device-gated: resident key " + str(priority[i]) + " out of range");
    if (rank[priority[i]] == UINT64_MAX) rank[priority[i]] = i;
  }
  for (uint32_t k = 0; k < keys_; ++k)
    if (rank[k] == UINT64_MAX) rank[k] = priority.size() + k;
  // the device keys: the first persistent_slots - spare_target distinct ones of the list
  std::vector<uint32_t> dev;
  std::vector<uint8_t> is_dev(keys_, 0);
  const size_t dev_cap = c_.persistent_slots - c_.spare_target;
  for (uint32_t k : priority)
    if (dev.size() < dev_cap && !is_dev[k]) {
      is_dev[k] = 1;
      dev.push_back(k);
    }
  // the keys with a block: every other one; three tiers: up to home_blocks of them, plan-pinned before file-tier,
  // each by rank
  std::vector<uint8_t> has_block(keys_, 0);
  std::vector<uint32_t> homes;
  if (files) {
    for (uint32_t k = 0; k < keys_; ++k)
      if (!is_dev[k]) homes.push_back(k);
    const auto tier = [&](uint32_t k) { return disk ? (*disk)[k] != 0 : false; };
    std::stable_sort(homes.begin(), homes.end(), [&](uint32_t a, uint32_t b) {
      if (tier(a) != tier(b)) return !tier(a);
      return rank[a] < rank[b];
    });
    // (only flags 0 and 1 compete; any other flag value never takes a home)
    homes.erase(std::remove_if(homes.begin(), homes.end(), [&](uint32_t k) { return disk && (*disk)[k] > 1; }),
                homes.end());
    homes.resize(std::min<size_t>(homes.size(), std::min(c_.home_blocks, c_.blocks)));
    for (uint32_t k : homes) has_block[k] = 1;
  } else {
    require(keys_ - dev.size() <= c_.blocks, SS_E_CAPACITY,
            "device-gated: " + str(keys_ - dev.size()) + " units off the device but only " + str(c_.blocks) +
                " host blocks");
    for (uint32_t k = 0; k < keys_; ++k) has_block[k] = !is_dev[k];
  }

  std::fill(st_.begin(), st_.end(), KeyState{});
  std::fill(mirror_.begin(), mirror_.end(), -1);
  free_land_.clear();
  for (uint32_t l = c_.landing_blocks; l-- > 0;) free_land_.push_back(int32_t(l));  // block 0 taken first
  land_busy_.clear();
  std::fill(land_owner_.begin(), land_owner_.end(), kNoKey);
  n_land_ = 0;
  recent_.reset(keys_);
  homed_.reset(keys_);
  n_device_ = n_pinned_ = n_clean_ = n_file_ = 0;
  int32_t blocks_used = 0;
  for (uint32_t k = 0; k < keys_; ++k) {
    KeyState& x = st_[k];
    if (has_block[k]) {
      x.where = Where::Pinned;
      x.block = blocks_used++;
    } else if (!is_dev[k]) {
      x.where = Where::File;
      ++n_file_;
    }
  }
  if (files) {
    for (size_t i = homes.size(); i-- > 0;) make_pinned(homes[i]);  // the first by rank the most recently homed
  } else {
    n_pinned_ = uint32_t(blocks_used);
  }
  for (size_t i = 0; i < dev.size(); ++i) {
    KeyState& x = st_[dev[i]];
    x.where = Where::Resident;
    x.slot = int32_t(i);
    mirror_[dev[i]] = x.slot;
  }
  for (size_t i = dev.size(); i-- > 0;) touch(dev[i]);  // the first of the list the most recent
  n_device_ = uint32_t(dev.size());
  free_slot_.clear();
  for (uint32_t s = c_.persistent_slots; s > dev.size(); --s) free_slot_.push_back(int32_t(s - 1));
  free_block_.clear();
  for (int32_t b = int32_t(c_.blocks); b > blocks_used; --b) free_block_.push_back(b - 1);
}

// ---- recency and homes ------------------------------------------------------------------------------------------------
void DgCore::touch(uint32_t k) {
  if (recent_.has(k)) recent_.remove(k);
  recent_.put_front(k);
  if (c_.scored) {
    if (stamp_ == UINT64_MAX) broken("recency stamps ran out");  // open_token keeps them below kStampLimit
    stamp_of_[k] = ++stamp_;
  }
}

void DgCore::make_pinned(uint32_t k) {
  ++n_pinned_;
  if (c_.disk_tier) homed_.put_front(k);
}

void DgCore::leave_pinned(uint32_t k) {
  --n_pinned_;
  if (!c_.disk_tier) return;
  if (!homed_.has(k)) broken("pinned key " + str(k) + " missing from the homes' order");
  homed_.remove(k);
}

void DgCore::fall_back(uint32_t k) {
  KeyState& x = st_[k];
  x.slot = -1;
  if (x.clean) {
    x.clean = false;
    --n_clean_;
  }
  if (x.block < 0) {
    if (!c_.disk_tier) broken("key " + str(k) + " left the device with no block and no write-back");
    x.where = Where::File;
    ++n_file_;
    return;
  }
  x.where = Where::Pinned;
  if (x.home_middle && c_.disk_tier) {  // (dg_bank_keep 2: a one-off read does not displace the recently homed)
    ++n_pinned_;
    homed_.put_middle(k);
  } else {
    make_pinned(k);
  }
  x.home_middle = false;
}

// The pinned unit homed longest ago goes to its file (its bytes are there already) and gives up its block, which no
// copy is using (a pinned home is only ever read, by a fetch that has since landed or not yet started).
// dg_bank_keep: the block a bank-served demand file miss is read into, its pinned home once the bank releases it.
int32_t DgCore::block_to_keep() {
  if (!c_.bank_keep || !c_.disk_tier) return -1;
  if (free_block_.empty()) {
    const uint32_t oldest = homed_.back();
    if (!give_up_oldest_home()) return -1;
    st_[oldest].dropped_for_keep = n_.tokens + 1;
    ++n_.bank_keep_drops;
  }
  const int32_t b = free_block_.back();
  free_block_.pop_back();
  return b;
}

bool DgCore::give_up_oldest_home() {
  if (!c_.disk_tier || homed_.size() == 0) return false;
  const uint32_t k = homed_.back();
  KeyState& x = st_[k];
  leave_pinned(k);
  free_block_.push_back(x.block);
  x.block = -1;
  x.where = Where::File;
  ++n_file_;
  ++n_.disk_drops;
  return true;
}

int32_t DgCore::next_stage() {
  const uint32_t i = stage_cursor_;
  stage_cursor_ = (stage_cursor_ + 1) % c_.disk_staging;
  void* last = stage_ev_[i];
  if (last && !t_->query(last)) {  // the buffer's previous unit is still being copied out of it
    t_->event_sync(last);
    ++n_.disk_stage_waits;
  }
  return int32_t(c_.blocks + i);
}

std::vector<uint32_t> DgCore::device_order() const {
  std::vector<uint32_t> out;
  for (uint32_t k = recent_.front(); k != KeyOrder::kEnd; k = recent_.toward_back(k))
    if (st_[k].where == Where::Resident) out.push_back(k);
  return out;
}

std::vector<uint32_t> DgCore::pinned_order() const {
  std::vector<uint32_t> out;
  for (uint32_t k = homed_.front(); k != KeyOrder::kEnd; k = homed_.toward_back(k)) out.push_back(k);
  return out;
}

void DgCore::publish(DgTransport::Stream s, uint32_t k, int32_t v, bool from_copy) {
  mirror_[k] = v;
  if (from_copy && t_->publishes_landed()) return;  // the transport publishes it with landed()
  t_->write_entry(s, k, v);
}

// ---- write-backs ------------------------------------------------------------------------------------------------------
void DgCore::apply_wb_mode() {
  if (!c_.wb_defer) {  // every victim copied whole at its boundary on kD2h
    wb_stream_ = DgTransport::kDem;
    layer_grant_ = in_flight_cap_ = 0;
    return;
  }
  wb_stream_ = c_.wb_on_d2h ? DgTransport::kD2h : DgTransport::kDem;
  layer_grant_ = c_.wb_layer_bytes ? c_.wb_layer_bytes : t_->part_bytes(0);
  in_flight_cap_ = c_.wb_max_outstanding ? c_.wb_max_outstanding : 2 * unit_bytes_;
  if (c_.wb_on_d2h && !after_ready_ev_) after_ready_ev_ = ev_.take();
}

void DgCore::send_part(WriteBack& w) {
  const uint32_t p = w.parts_sent++;
  t_->d2h_part(wb_stream_, w.slot, w.block, p);
  const uint64_t b = t_->part_bytes(p);
  w.bytes_sent += b;
  in_flight_bytes_ += b;
  n_.wb_issued_bytes += b;
}

void DgCore::seal_first_queued(bool dropped) {
  WriteBack& w = wb_[sealed_++];
  w.ev = ev_.take();
  t_->record(w.ev, wb_stream_);
  w.dropped = dropped;
}

void DgCore::finish_first_queued() {
  WriteBack& w = wb_[sealed_];
  while (w.parts_sent < t_->parts()) send_part(w);
  seal_first_queued(false);
}

// Every sealed write-back completes in the bookkeeping, oldest first: its key is pinned in its block and its slot is
// free (a dropped one only returns its block). Its event stays tied to the slot and the block until the copy has
// really ended, so a later copy into the slot or out of the block waits for it.
uint32_t DgCore::retire_writebacks() {
  const uint32_t n = uint32_t(sealed_);
  for (; sealed_ > 0; --sealed_) {
    const WriteBack w = wb_.front();
    wb_.pop_front();
    KeyState& x = st_[w.key];
    x.wb_open = false;
    if (w.dropped) {  // (its unit is resident again in the slot, which a copy in must not overwrite before w ends)
      free_block_.push_back(w.block);
      ev_.tie_slot(w.slot, w.ev);
      ev_.tie_block(w.block, w.ev);
    } else {
      x.where = Where::Pinned;
      x.slot = -1;
      x.block = w.block;
      make_pinned(w.key);
      free_slot_.push_back(w.slot);
      ev_.tie_slot(w.slot, w.ev);
      ev_.tie_block(w.block, w.ev);
    }
    ev_.release_if_loose(w.ev);
    in_flight_bytes_ -= w.bytes_sent;
    n_.wb_completed_bytes += w.bytes_sent;
  }
  n_.writebacks_done += n;
  return n;
}

void DgCore::free_a_slot() {
  while (free_slot_.empty() && queued_writebacks() > 0) {
    const bool slot_coming = std::any_of(wb_.begin(), wb_.begin() + ptrdiff_t(sealed_),
                                         [](const WriteBack& w) { return !w.dropped; });
    if (!slot_coming) finish_first_queued();
    ++n_.wb_forced;
    n_.collected_mid += retire_writebacks();
  }
}

void DgCore::spend_wb_credit(uint32_t g) {
  if (queued_writebacks() == 0) {
    credit_ = 0;
    return;
  }
  if (g + 1 >= gated()) return;  // no layer after the last gated one to overlap with
  // one grant per layer; an overdraft carries into the next layer, unused credit does not
  credit_ = std::min<int64_t>(credit_ + int64_t(layer_grant_), int64_t(layer_grant_));
  n_.collected_mid += retire_writebacks();
  bool behind_ready = false;
  while (credit_ > 0 && queued_writebacks() > 0 && in_flight_bytes_ < in_flight_cap_) {
    if (wb_stream_ == DgTransport::kD2h && !behind_ready) {  // after the ready word already on the demand stream
      t_->record(after_ready_ev_, DgTransport::kDem);
      t_->wait(DgTransport::kD2h, after_ready_ev_);
      behind_ready = true;
    }
    WriteBack& w = wb_[sealed_];
    credit_ -= int64_t(t_->part_bytes(w.parts_sent));
    if (w.parts_sent + 1 < t_->parts()) send_part(w);
    else finish_first_queued();
  }
}

// ---- a token's service ------------------------------------------------------------------------------------------------
void DgCore::open_token(uint32_t seq, const std::vector<uint8_t>* run) {
  require(!run || run->size() == gated(), SS_E_INVALID, "device-gated: the exported-layer flags do not match the gated layers");
  if (c_.scored) {  // one token moves far fewer than 2^40 keys to the front
    require(stamp_ <= kStampLimit, SS_E_BACKEND, "device-gated: scoring's recency stamps are used up (reopen)");
    require(token_ < (uint64_t(1) << 63), SS_E_BACKEND, "device-gated: scoring's token counter is used up (reopen)");
    ++token_;
  }
  if (run) exported_.assign(run->begin(), run->end());
  else std::fill(exported_.begin(), exported_.end(), uint8_t(1));
  seq_ = seq;
  ahead_in_token_ = 0;
  std::fill(ahead_in_layer_.begin(), ahead_in_layer_.end(), 0u);
  std::fill(layer_missed_.begin(), layer_missed_.end(), uint8_t(0));
  std::fill(served_.begin(), served_.end(), uint8_t(0));
  predicted_.clear();
  predicted_layer_ = kNoKey;
}

uint64_t DgCore::absent_mask(uint32_t g, const uint32_t* ids, uint32_t n) const {
  uint64_t m = 0;
  const uint32_t nu = units(g);
  for (uint32_t i = 0; i < std::min<uint32_t>(n, 64); ++i)
    if (ids[i] < nu && mirror_[key(g, ids[i])] < 0) m |= uint64_t(1) << i;
  return m;
}

// A unit chosen at a boundary whose write-back has not completed still has its bytes in its slot: it becomes resident
// again at once and the write-back goes (not started: dropped from the queue, its block free; partly submitted:
// sealed after its sent parts and dropped, so only its block returns at the retire).
bool DgCore::resurrect(uint32_t k) {
  KeyState& x = st_[k];
  bool found = false;
  for (size_t i = sealed_; i < wb_.size() && !found; ++i) {
    if (wb_[i].key != k) continue;
    found = true;
    if (wb_[i].parts_sent == 0) {
      // (a transport may have copied it already, at the boundary: the slot and the block wait for that copy)
      t_->unqueue(wb_[i].slot, wb_[i].block);
      void* ev = ev_.take();
      t_->record(ev, wb_stream_);
      ev_.tie_slot(wb_[i].slot, ev);
      ev_.tie_block(wb_[i].block, ev);
      free_block_.push_back(wb_[i].block);
      wb_.erase(wb_.begin() + ptrdiff_t(i));
      x.wb_open = false;
      ++n_.wb_cancelled;
      n_.wb_cancelled_bytes += unit_bytes_;
    } else {
      if (i != sealed_) broken("a queued write-back behind the first has parts submitted");
      n_.wb_cancelled_bytes += unit_bytes_ - wb_[i].bytes_sent;
      seal_first_queued(true);
    }
  }
  for (size_t i = 0; i < sealed_ && !found; ++i)
    if (wb_[i].key == k && !wb_[i].dropped) {
      wb_[i].dropped = true;
      found = true;
    }
  x.where = Where::Resident;
  x.block = -1;
  publish(DgTransport::kDem, k, x.slot);
  touch(k);
  ++n_device_;
  ++n_.resurrected;
  return true;
}

bool DgCore::bring_in(uint32_t g, uint32_t u, bool ahead) {
  const uint32_t k = key(g, u);
  KeyState& x = st_[k];
  if (ahead && (ahead_in_layer_[g] >= c_.prefetch_per_layer || ahead_in_token_ >= c_.prefetch_per_token)) return false;
  if (on_device_or_arriving(k)) return false;
  if (x.where == Where::Draining) return resurrect(k);
  if (x.where == Where::Landed && ahead) return false;  // a landing is copied in by a demand only
  if (x.where == Where::File && ahead && !c_.disk_prefetch) return false;

  // a persistent slot above the prefetch reserve, else (a demand) a bank slot
  const size_t reserve = ahead ? c_.prefetch_reserve : 0;
  if (free_slot_.size() <= reserve) n_.collected_mid += retire_writebacks();
  if (!ahead && free_slot_.empty()) free_a_slot();
  int32_t slot = -1;
  bool banked = false;
  if (free_slot_.size() > reserve) {
    slot = free_slot_.back();
    free_slot_.pop_back();
  } else if (ahead) {
    return false;
  } else {
    uint32_t held = kNoKey;
    slot = banks_.borrow(g, seq_, &held);
    if (slot >= 0) {
      banked = true;
      if (held != kNoKey && st_[held].where == Where::InBank && st_[held].slot == slot) {  // an earlier layer's alias
        fall_back(held);
        publish(DgTransport::kDem, held, -1);
      }
    } else {  // more distinct misses than a bank holds: not reachable through a service that checks its exports
      free_a_slot();
      for (; free_slot_.empty() && sealed_ > 0; ++n_.stalled) retire_writebacks();
      if (free_slot_.empty()) fail(SS_E_BACKEND, "device-gated: a miss found no slot, no bank slot and no write-back");
      slot = free_slot_.back();
      free_slot_.pop_back();
    }
  }

  const DgTransport::Stream s = ahead ? DgTransport::kPf : DgTransport::kDem;
  if (x.where == Where::File) {  // read into a staging buffer (or a kept block), then copied in from there
    const int32_t kept = banked ? block_to_keep() : -1;
    const int32_t src = kept >= 0 ? kept : next_stage();
    if (kept >= 0) {
      if (void* wb = ev_.on_block(kept)) t_->event_sync(wb);  // a write-back may still be copying into it
      try {
        t_->read_unit(k, src, slot);
      } catch (...) {  // nothing begun for the key: the block is free again
        free_block_.push_back(kept);
        throw;
      }
    } else {
      t_->read_unit(k, src, slot);
    }
    ++n_.disk_reads;
    n_.disk_read_bytes += unit_bytes_;
    t_->wait_copy_in(s, slot, src, ev_.on_slot(slot), nullptr);  // (the block's own write-back ended above)
    ev_.untie_slot(slot);
    if (kept >= 0) ev_.untie_block(kept);
    t_->h2d(s, slot, src, k);
    if (kept >= 0) {  // the block is the key's: its pinned home when the bank releases it
      x.block = kept;
      x.home_middle = c_.bank_keep == 2;
      ++n_.bank_kept;
    } else {
      void*& last = stage_ev_[size_t(src) - c_.blocks];
      if (!last) last = ev_.take();
      t_->record(last, s);
    }
    --n_file_;
    if (x.dropped_for_keep) {  // dropped for a kept read, and read back from its file
      if (n_.tokens + 1 - x.dropped_for_keep <= 8) ++n_.bank_keep_rereads;
      x.dropped_for_keep = 0;
    }
  } else if (x.where == Where::Landed) {  // from its landing block, as from a pinned block
    const int32_t lb = land_block(x.land);
    t_->wait_copy_in(s, slot, lb, ev_.on_slot(slot), nullptr);
    ev_.untie_slot(slot);
    t_->h2d(s, slot, lb, k);
    land_busy_.push_back(x.land);  // free at the next landing or boundary (the transport orders the reuse)
    land_owner_[size_t(x.land)] = kNoKey;
    x.land = -1;
    x.land_age = 0;
    --n_land_;
    --n_file_;
    ++n_.landing_promoted;
  } else {  // after the slot's last write-back and any write-back still copying into this block
    t_->wait_copy_in(s, slot, x.block, ev_.on_slot(slot), ev_.on_block(x.block));
    ev_.untie_slot(slot);
    ev_.untie_block(x.block);
    t_->h2d(s, slot, x.block, k);
    leave_pinned(k);
  }
  publish(s, k, slot, true);
  x.slot = slot;
  x.ahead = ahead;
  x.ahead_hit = false;
  if (ahead) {
    x.ahead_ev = ev_.take();
    t_->record(x.ahead_ev, s);
  }
  DgLayerCounts& lc = per_layer_[g];
  if (banked) {
    x.where = Where::InBank;
    banks_.hold(slot, k);
    in_bank_.push_back(k);
    ++n_.bank_serves;
    ++lc.bank_serves;
  } else {
    x.where = Where::Arriving;
    arriving_.push_back(k);
    touch(k);
    ++n_device_;
  }
  if (ahead) {
    ++n_.prefetched;
    ++lc.prefetched;
    ++ahead_in_layer_[g];
    ++ahead_in_token_;
  } else {
    ++n_.fetched;
    ++lc.fetched;
  }
  t_->landed(s, g, &k, &slot, 1);  // per unit, so a verifying transport checks it while the next miss copies
  return true;
}

void DgCore::serve_misses(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask, uint64_t dev_mask) {
  const uint32_t nu = units(g);
  for (uint32_t i = 0; i < n; ++i)
    require(ids[i] < nu, SS_E_INVALID,
            "device-gated: gated layer " + str(g) + " exported unit " + str(ids[i]) + " (it has " + str(nu) + ")");
  const bool any = (mask | dev_mask) != 0;
  if (any) t_->diag_mark(g, 0);
  bool first_miss = true;
  for (uint32_t i = 0; i < n; ++i) {  // a repeated id: fetched at its first miss, covered at the next
    const uint32_t k = key(g, ids[i]);
    const KeyState& x = st_[k];
    const bool prefetch_in_flight = x.where == Where::Arriving && x.ahead && x.ahead_ev;
    if (!(mask >> i & 1u)) {
      if ((dev_mask >> i & 1u) && prefetch_in_flight) t_->wait(DgTransport::kDem, x.ahead_ev);
      continue;
    }
    if (!on_device_or_arriving(k)) {
      bring_in(g, ids[i], false);
      if (first_miss) t_->diag_mark(g, 2);
      first_miss = false;
      continue;
    }
    if (prefetch_in_flight) {  // the layer's readers wait for the prefetch's copy
      t_->wait(DgTransport::kDem, x.ahead_ev);
      ++n_.covered_waits;
    }
    ++n_.covered;
  }
  if (c_.landing_blocks && c_.landing_ttl == 0) {  // nothing demands layer g again this token
    served_[g] = 1;
    expire_layer_landings(g, ids, n);
  }
  if (any) {
    t_->signal_ready(g, seq_);  // after every fetch's landed()
    t_->diag_mark(g, 1);
  }
}

void DgCore::note_uses(uint32_t g, const uint32_t* ids, uint32_t n, uint64_t mask) {
  std::vector<uint32_t>& uni = scratch_ids_;
  uni.assign(ids, ids + n);
  std::sort(uni.begin(), uni.end());
  uni.erase(std::unique(uni.begin(), uni.end()), uni.end());
  if (c_.scored) {
    require(uni.size() <= c_.max_ids, SS_E_BACKEND, "device-gated: an export's union exceeds its max ids");
    n_.score_saturated += hist_[g].learn(uni, token_);
  }
  const bool judge = predicted_layer_ == g;
  DgLayerCounts& lc = per_layer_[g];
  for (uint32_t id : uni) {
    bool missed = false;
    for (uint32_t i = 0; i < n && !missed; ++i) missed = ids[i] == id && (mask >> i & 1u);
    const uint32_t k = key(g, id);
    KeyState& x = st_[k];
    ++n_.lookups;
    ++lc.lookups;
    if (missed) {
      ++n_.misses;
      ++lc.misses;
      if (!layer_missed_[g]) ++n_.miss_layers;
      layer_missed_[g] = 1;
    }
    if (c_.scored) x.demand_token = token_;  // demand uses only: prefetches and resurrections leave it
    if (x.ahead && !x.ahead_hit) {
      x.ahead_hit = true;
      ++n_.prefetch_used;
      ++lc.prefetch_used;
    }
    if (recent_.has(k)) touch(k);
    if (judge && std::find(predicted_.begin(), predicted_.end(), id) != predicted_.end()) ++n_.predicted_true;
  }
  predicted_.clear();
  predicted_layer_ = kNoKey;
}

void DgCore::prefetch_next(uint32_t g_next, const uint32_t* pred, uint32_t n) {
  if (g_next >= gated()) return;
  const uint32_t nu = units(g_next);
  predicted_.clear();
  for (uint32_t i = 0; i < n; ++i) {  // first occurrences in list order: the budget keeps the head of the list
    if (pred[i] >= nu) ++n_.pred_invalid;
    else if (std::find(predicted_.begin(), predicted_.end(), pred[i]) == predicted_.end()) predicted_.push_back(pred[i]);
  }
  n_.predicted += predicted_.size();
  predicted_layer_ = g_next;
  for (uint32_t id : predicted_)
    if (!advise_land(g_next, id)) bring_in(g_next, id, true);  // (landings on: a file-homed unit lands instead)
}

// ---- landings (dg_landing_blocks) -------------------------------------------------------------------------------------
// A prediction of a file-homed unit reads it into a landing block of its own pool: no slot is taken and nothing is
// evicted or written back for it, outside the prefetch budgets. It stays file-homed (Landed: no slot, block or entry)
// until a demand copies it from its landing block into the slot a file miss would have taken; no free landing block
// drops the advice, and a landing is never displaced. In this schedule a landing read has landed when its layer is
// served: the transport orders every copy out of a landing block after its read on the device.
bool DgCore::advise_land(uint32_t g, uint32_t u) {
  if (!c_.landing_blocks) return false;
  const uint32_t k = key(g, u);
  const Where w = st_[k].where;
  if (w == Where::Landed) return true;  // (already landing: left as it is)
  if (w != Where::File) return false;
  if (c_.landing_ttl == 0 && served_[g]) {  // its layer's demand has passed: it could never be used
    ++n_.landing_skipped_passed;
    return true;
  }
  land(k);
  return true;
}

void DgCore::land(uint32_t k) {
  reclaim_lands();
  if (free_land_.empty()) {
    ++n_.landing_dropped_full;
    return;
  }
  const int32_t l = free_land_.back();
  t_->read_landing(k, land_block(l));
  free_land_.pop_back();
  KeyState& x = st_[k];
  land_owner_[size_t(l)] = k;
  x.where = Where::Landed;
  x.land = l;
  x.land_age = 0;
  ++n_land_;
  ++n_.landing_issued;
  n_.landing_read_bytes += unit_bytes_;
}

void DgCore::unland(uint32_t k) {
  KeyState& x = st_[k];
  const int32_t l = x.land;
  free_land_.push_back(l);
  land_owner_[size_t(l)] = kNoKey;
  x.land = -1;
  x.land_age = 0;
  x.where = Where::File;
  --n_land_;
  t_->drop_landing(land_block(l));
}

void DgCore::reclaim_lands() {
  free_land_.insert(free_land_.end(), land_busy_.begin(), land_busy_.end());
  land_busy_.clear();
}

// landing_ttl 0, after layer g's demand: its landings it did not route go back to their file (in block order).
void DgCore::expire_layer_landings(uint32_t g, const uint32_t* ids, uint32_t n) {
  for (uint32_t l = 0; l < c_.landing_blocks; ++l) {
    const uint32_t k = land_owner_[l];
    if (k == kNoKey || k < first_key_[g] || k >= first_key_[g + 1]) continue;
    if (std::find(ids, ids + n, k - first_key_[g]) != ids + n) continue;
    unland(k);
    ++n_.landing_expired_layer;
  }
}

// ---- the boundary -----------------------------------------------------------------------------------------------------
void DgCore::close_token(uint32_t rows, const std::vector<uint32_t>& keep) {
  if (!keep.empty()) {
    kept_.assign(keys_, 0);
    for (uint32_t k : keep)
      if (k < keys_) kept_[k] = 1;
  }
  struct Unkeep {
    std::vector<uint8_t>& v;
    ~Unkeep() { v.clear(); }
  } unkeep{kept_};
  using Clock = std::chrono::steady_clock;
  const auto us = [](Clock::time_point a, Clock::time_point b) {
    return double(std::chrono::duration_cast<std::chrono::nanoseconds>(b - a).count()) / 1e3;
  };
  DgBoundaryTimes bt = bt_;
  const auto t_sync = Clock::now();
  t_->diag_boundary();
  t_->sync(DgTransport::kDem);  // every copy and table write of the token landed before homes change
  t_->sync(DgTransport::kPf);
  const auto t_select = Clock::now();
  bt.sync_us = us(t_sync, t_select);
  if (c_.landing_blocks) {  // the blocks copied out of are free; a landing not demanded for landing_ttl boundaries (TTL
    reclaim_lands();        // 0: this one) goes back to its file, no copy (the file holds its bytes)
    for (uint32_t l = 0; l < c_.landing_blocks; ++l) {
      const uint32_t k = land_owner_[l];
      if (k == kNoKey || ++st_[k].land_age < std::max<uint32_t>(c_.landing_ttl, 1)) continue;
      unland(k);
      ++n_.landing_expired;
    }
  }
  for (uint32_t k : arriving_) {  // resident now; the block it came from is free, or kept as a clean copy
    KeyState& x = st_[k];
    if (x.where != Where::Arriving) continue;
    x.where = Where::Resident;
    x.ahead = false;
    if (x.ahead_ev) ev_.give(x.ahead_ev);
    x.ahead_ev = nullptr;
    if (x.block < 0) continue;
    if (n_clean_ < c_.inclusive) {
      x.clean = true;
      ++n_clean_;
      ++n_.inclusive_kept;
    } else {
      free_block_.push_back(x.block);
      x.block = -1;
    }
  }
  arriving_.clear();
  for (uint32_t k : in_bank_) {  // borrowed for the token: back to the block (or the file) it came from
    KeyState& x = st_[k];
    if (x.where == Where::InBank) {
      fall_back(k);
      mirror_[k] = -1;
    }
    if (x.ahead_ev) ev_.give(x.ahead_ev);
    x.ahead_ev = nullptr;
    x.ahead = false;
  }
  in_bank_.clear();
  banks_.clear();
  retire_writebacks();

  // victims until free slots + queued write-backs + victims reach the spare target, from the back of the recency
  // order or (scored) lowest rank first; the first victim with no block to go to ends the choice
  const size_t have = free_slot_.size() + queued_writebacks();
  const size_t want = c_.spare_target > have ? c_.spare_target - have : 0;
  chosen_.clear();
  bool by_score = c_.scored && (!c_.scored_auto || rows > 1);
  if (by_score) {
    for (uint32_t g = 0; g < gated() && by_score; ++g)
      by_score = !exported_[g] || hist_[g].served() == token_;  // an exported layer left unlearned: recency
    if (!by_score) ++n_.score_fallbacks;
  }
  if (by_score) {
    const auto t0 = std::chrono::steady_clock::now();
    rank_by_score(want);
    for (const Ranked& r : ranked_) {
      if (!choose(r.key)) break;
      ++n_.scored_victims;
    }
    n_.score_ns += uint64_t(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
  } else {
    size_t got = 0;
    for (uint32_t k = recent_.back(); k != KeyOrder::kEnd && got < want;) {
      const uint32_t next = recent_.toward_front(k);
      if (choosable(k)) {
        if (!choose(k)) break;
        ++got;
      }
      k = next;
    }
  }
  const auto t_upload = Clock::now();
  bt.select_us = us(t_select, t_upload);
  t_->upload_table(mirror_.data(), keys_);  // the device table equals the mirror before any write-back is enqueued
  const auto t_issue = Clock::now();
  bt.upload_us = us(t_upload, t_issue);

  // Queued write-backs older than this boundary and the one before it are submitted now (the carry); this boundary's
  // victims are queued (or, without queueing, copied whole on kD2h).
  const size_t fresh = chosen_.size(), older = queued_writebacks();
  const size_t carry = std::max(fresh, last_chosen_);
  const size_t flush = older > carry ? older - carry : 0;
  last_chosen_ = fresh;
  credit_ = 0;
  if (c_.wb_defer)
    for (uint32_t k : chosen_) {
      const KeyState& x = st_[k];
      wb_.push_back(WriteBack{k, x.slot, x.block, 0, 0, nullptr, false});
      if (wb_stream_ == DgTransport::kD2h) t_->prestage(x.slot, x.block);  // its events then follow the copies
      ++n_.wb_deferred;
      ++n_.evicted;
      ++per_layer_[gated_of(k)].evicted;
    }
  const uint64_t issued_before = n_.wb_issued_bytes;
  for (size_t i = 0; i < flush; ++i) finish_first_queued();
  n_.wb_boundary_flushed += flush;
  n_.wb_boundary_flushed_bytes += n_.wb_issued_bytes - issued_before;
  if (!c_.wb_defer) {
    if (queued_writebacks() != 0) broken("queued write-backs while queueing is off");
    for (uint32_t k : chosen_) {
      const KeyState& x = st_[k];
      t_->d2h(x.slot, x.block);
      void* ev = ev_.take();
      t_->record(ev, DgTransport::kD2h);
      wb_.push_back(WriteBack{k, x.slot, x.block, t_->parts(), unit_bytes_, ev, false});
      ++sealed_;
      in_flight_bytes_ += unit_bytes_;
      n_.wb_issued_bytes += unit_bytes_;
      ++n_.evicted;
      ++per_layer_[gated_of(k)].evicted;
    }
  }
  if (!chosen_.empty()) t_->diag_writebacks_issued();
  ev_.sweep();
  bt.issue_us = us(t_issue, Clock::now());
  bt.writebacks = uint32_t(chosen_.size());
  ++bt.boundaries;
  bt_ = bt;  // (published whole: a boundary that throws leaves the last complete one)
  ++n_.tokens;
}

bool DgCore::choose(uint32_t k) {
  KeyState& x = st_[k];
  // No copy needed: a clean copy (its block holds its bytes), or three tiers with no block to write into - when the
  // file tier's clean eviction is on and the spares are gone, or after the longest-homed pinned unit was asked for
  // its block and there was none: the unit goes to its file.
  const bool to_file_clean = !x.clean && clean_evict_now();
  const bool no_copy =
      x.clean || to_file_clean || (c_.disk_tier && free_block_.empty() && !give_up_oldest_home());
  DgLayerCounts& lc = per_layer_[gated_of(k)];
  if (no_copy) {
    if (x.clean) ++n_.inclusive_drops;
    else ++n_.disk_discards;
    if (to_file_clean) {
      ++n_.clean_drops;
      n_.clean_drop_bytes += unit_bytes_;
    }
    recent_.remove(k);
    --n_device_;
    free_slot_.push_back(x.slot);
    fall_back(k);
    mirror_[k] = -1;
    ++n_.evicted;
    ++lc.evicted;
    return true;
  }
  if (free_block_.empty()) {
    ++n_.evict_short;
    return false;
  }
  recent_.remove(k);
  --n_device_;
  x.where = Where::Draining;
  x.block = free_block_.back();
  free_block_.pop_back();
  x.wb_open = true;
  mirror_[k] = -1;
  chosen_.push_back(k);
  return true;
}

// ---- scored eviction --------------------------------------------------------------------------------------------------
// Unit u of gated layer g, with C = this token's union of g, D = the sum of the row sums over C:
//   P = ((|C| * sum_{r in C} T[r][u]) << 16) / max(1, D)      (transition pull)
//   F = (occurrences of u in the window << 16) / kWindow       (frequency)
//   R = (1 << 16) / (1 + token - token of u's last demand use)   (recency)
//   score = w_trans P + w_freq F + w_rec R, unsigned with floor division.
// With at most 65536 units and 64 ids the sum stays below 2^38 and D below 2^54, so the shifted product fits in 64
// bits; the sum is at most D, so P <= 2^22 and the score stays below 2^33. Every term is nonnegative, so when F and R
// alone already rank at or after `bar`, the full score does too and the transition rows are not read.
DgCore::Ranked DgCore::rank_of(uint32_t g, uint32_t u, uint64_t denom, const Ranked* bar) const {
  const LayerHistory& h = hist_[g];
  const uint32_t k = key(g, u);
  const KeyState& x = st_[k];
  const uint64_t F = (uint64_t(h.seen(u)) << 16) / kWindow;
  const uint64_t R = (uint64_t(1) << 16) / (1 + token_ - x.demand_token);
  Ranked r{uint64_t(c_.w_freq) * F + uint64_t(c_.w_rec) * R, x.demand_token, stamp_of_[k], k};
  if (bar && !(r < *bar)) return r;
  const uint64_t P = ((uint64_t(h.cur_size()) * h.pull(u)) << 16) / std::max<uint64_t>(1, denom);
  r.score += uint64_t(c_.w_trans) * P;
  return r;
}

// The `want` lowest-ranked choosable keys, ascending, kept as a bounded max-heap while every gated layer is scanned.
void DgCore::rank_by_score(size_t want) {
  ranked_.clear();
  if (!want) return;
  for (uint32_t g = 0; g < gated(); ++g) {
    const uint64_t denom = hist_[g].denominator();
    ++n_.score_layers;
    for (uint32_t u = 0; u < units(g); ++u) {
      if (!choosable(key(g, u))) continue;
      ++n_.score_candidates;
      if (ranked_.size() < want) {
        ranked_.push_back(rank_of(g, u, denom, nullptr));
        std::push_heap(ranked_.begin(), ranked_.end());
        continue;
      }
      const Ranked r = rank_of(g, u, denom, &ranked_.front());
      if (!(r < ranked_.front())) continue;
      std::pop_heap(ranked_.begin(), ranked_.end());
      ranked_.back() = r;
      std::push_heap(ranked_.begin(), ranked_.end());
    }
  }
  std::sort_heap(ranked_.begin(), ranked_.end());
}

void DgCore::seed_transitions(const unsigned char* cells) {
  require(c_.scored, SS_E_INVALID, "device-gated: starting transition counts need a scored policy");
  for (uint32_t g = 0; g < gated(); ++g) {
    hist_[g].set_open(cells);
    cells += 4 * size_t(units(g)) * units(g);
  }
  for (LayerHistory& h : hist_) h.restore();
  token_ = 0;
}

void DgCore::set_policy(uint32_t policy) {
  require(policy <= 2, SS_E_INVALID, "device-gated: policy " + str(policy) + " is not LRU, SCORED or SCORED_AUTO");
  require(policy == 0 || !hist_.empty(), SS_E_INVALID,
          "device-gated: scoring was not provisioned at open (the context opened under LRU)");
  quiesce();
  retire_writebacks();
  c_.scored = policy != 0;
  c_.scored_auto = policy == 2;
  for (LayerHistory& h : hist_) h.restore();
  token_ = 0;
  for (KeyState& x : st_) x.demand_token = 0;
  std::fill(stamp_of_.begin(), stamp_of_.end(), 0);
  stamp_ = 0;
  for (uint32_t k = recent_.back(); k != KeyOrder::kEnd; k = recent_.toward_front(k)) {  // the front the largest
    ++stamp_;
    if (!stamp_of_.empty()) stamp_of_[k] = stamp_;
  }
}

void DgCore::defer_writebacks(bool on) {
  if (on == c_.wb_defer) return;
  while (!on && queued_writebacks() > 0) finish_first_queued();  // sealed now, retired like any other
  c_.wb_defer = on;
  apply_wb_mode();
  credit_ = 0;
  last_chosen_ = 0;
}

void DgCore::quiesce() {
  while (queued_writebacks() > 0) finish_first_queued();
  t_->sync(DgTransport::kDem);
  t_->sync(DgTransport::kPf);
  t_->sync(DgTransport::kD2h);
  ev_.sweep();
}

void DgCore::set_spare_target(uint32_t n) {
  require(n <= c_.persistent_slots, SS_E_INVALID,
          "device-gated: spare target " + str(n) + " exceeds the " + str(c_.persistent_slots) + " persistent slots");
  c_.spare_target = n;
  if (c_.prefetch_reserve_auto) c_.prefetch_reserve = std::min<uint32_t>(24, n / 4);
}

void DgCore::set_prefetch_budget(uint32_t per_layer, uint32_t per_token) {
  c_.prefetch_per_layer = per_layer;
  c_.prefetch_per_token = per_token;
}

// ---- invariants -------------------------------------------------------------------------------------------------------
void DgCore::audit() const {
  std::vector<uint32_t> slot_owner(slots_, kNoKey), block_owner(c_.blocks, kNoKey);
  const auto own = [&](std::vector<uint32_t>& owner, int32_t i, uint32_t who, const char* what) {
    if (i < 0 || size_t(i) >= owner.size()) broken(std::string(what) + " " + str(uint64_t(int64_t(i))) + " out of range");
    if (owner[size_t(i)] != kNoKey) broken(std::string(what) + " " + str(uint64_t(i)) + " owned twice");
    owner[size_t(i)] = who;
  };
  constexpr uint32_t kFree = 0xfffffffeu;
  uint32_t n_dev = 0, n_pin = 0, n_file = 0, n_clean = 0, n_land = 0;
  for (uint32_t k = 0; k < keys_; ++k) {
    const KeyState& x = st_[k];
    const std::string who = "key " + str(k);
    const bool has_slot = x.where == Where::Resident || x.where == Where::Arriving || x.where == Where::InBank ||
                          x.where == Where::Draining;
    if (has_slot) own(slot_owner, x.slot, k, "slot");
    else if (x.slot != -1) broken(who + " holds a slot off the device");
    if (x.block >= 0) own(block_owner, x.block, k, "block");
    if (x.clean) ++n_clean;
    switch (x.where) {
      case Where::Resident:
        if (mirror_[k] != x.slot) broken(who + " resident but not published");
        if (!recent_.has(k)) broken(who + " resident but not in the recency order");
        if (x.clean != (x.block >= 0)) broken(who + " clean flag and block disagree");
        ++n_dev;
        break;
      case Where::Arriving:
        if (!recent_.has(k)) broken(who + " arriving but not in the recency order");
        ++n_dev;
        break;
      case Where::InBank:
        if (x.block < 0 && !c_.disk_tier) broken(who + " in a bank with no block to return to");
        break;
      case Where::Draining:
        if (x.block < 0 || !x.wb_open || mirror_[k] >= 0) broken(who + " draining without a block or a record");
        break;
      case Where::Pinned:
        if (x.block < 0 || mirror_[k] >= 0) broken(who + " pinned without a block, or published");
        if (c_.disk_tier && !homed_.has(k)) broken(who + " pinned but not in the homes' order");
        ++n_pin;
        break;
      case Where::File:
        if (!c_.disk_tier || x.block >= 0 || mirror_[k] >= 0) broken(who + " in its file with a block or an entry");
        ++n_file;
        break;
      case Where::Landed:
        if (x.block >= 0 || mirror_[k] >= 0 || x.land < 0 || uint32_t(x.land) >= c_.landing_blocks ||
            land_owner_[size_t(x.land)] != k)
          broken(who + " landed with a block or an entry, or not owning its landing block");
        ++n_file;
        ++n_land;
        break;
    }
    if (x.where != Where::Landed && x.land >= 0) broken(who + " holds a landing block off the landing state");
    if (x.where != Where::Pinned && homed_.has(k)) broken(who + " in the homes' order but not pinned");
    if (recent_.has(k) && x.where != Where::Resident && x.where != Where::Arriving)
      broken(who + " in the recency order off the device");
  }
  for (int32_t s : free_slot_) own(slot_owner, s, kFree, "free slot");
  for (int32_t b : free_block_) own(block_owner, b, kFree, "free block");
  if (sealed_ > wb_.size()) broken("more sealed write-backs than records");
  for (size_t i = 0; i < wb_.size(); ++i) {
    const WriteBack& w = wb_[i];
    const KeyState& x = st_[w.key];
    if (w.dropped) {  // the key came back: the record alone owns its block until the retire
      if (i >= sealed_) broken("a dropped write-back still queued");
      own(block_owner, w.block, kFree, "dropped write-back's block");
    } else if (x.where != Where::Draining || x.slot != w.slot || x.block != w.block) {
      broken("write-back of key " + str(w.key) + " does not match its key");
    }
    if ((i < sealed_) != (w.ev != nullptr)) broken("a write-back sealed without an event, or queued with one");
  }
  if (n_dev != n_device_) broken("device count");
  if (n_pin != n_pinned_) broken("pinned count");
  if (n_file != n_file_) broken("file count");
  if (n_land != n_land_) broken("landing count");
  {  // every landing block once: owned, free or copied out of since the last reclaim
    std::vector<uint8_t> seen(c_.landing_blocks, 0);
    uint32_t owned = 0;
    for (uint32_t l = 0; l < c_.landing_blocks; ++l) owned += land_owner_[l] != kNoKey;
    for (const std::vector<int32_t>* v : {&free_land_, &land_busy_})
      for (int32_t l : *v) {
        if (l < 0 || uint32_t(l) >= c_.landing_blocks || seen[size_t(l)]++ || land_owner_[size_t(l)] != kNoKey)
          broken("landing block " + str(uint64_t(int64_t(l))) + " free twice, out of range or owned");
      }
    if (owned != n_land_ || owned + free_land_.size() + land_busy_.size() != c_.landing_blocks)
      broken("landing blocks lost");
  }
  if (n_clean != n_clean_) broken("clean-copy count");
  if (recent_.size() != n_device_) broken("recency order length");
  if (c_.disk_tier && homed_.size() != n_pinned_) broken("homes' order length");
  if (c_.disk_tier && !homed_.half_consistent()) broken("the homes' order's front half");
  if (c_.scored) {  // stamps fall strictly from the front; no demand token ahead of the current one
    uint64_t above = UINT64_MAX;
    for (uint32_t k = recent_.front(); k != KeyOrder::kEnd; k = recent_.toward_back(k)) {
      if (stamp_of_[k] == 0 || stamp_of_[k] >= above || stamp_of_[k] > stamp_) broken("recency stamps out of order");
      above = stamp_of_[k];
    }
    for (const KeyState& x : st_)
      if (x.demand_token > token_) broken("a demand token ahead of the current token");
    for (const LayerHistory& h : hist_)
      if (!h.consistent()) broken("a score window's occurrence counts");
  }
}

}  // namespace tsa
