#include "host_place.hpp"

#include <algorithm>
#include <string>

#include "common.hpp"

namespace tsa {
namespace {

bool resident_tier(uint8_t t) { return t == SS_TIER_RESIDENT || t == SS_TIER_RESIDENT_BACKED; }

}  // namespace

void add_stats(ss_layer_stats& a, const ss_layer_stats& b) {
  a.routed += b.routed;
  a.hits += b.hits;
  a.admitted += b.admitted;
  a.transient += b.transient;
  a.evicted += b.evicted;
  a.prefetched += b.prefetched;
  a.spec_issued += b.spec_issued;
  a.spec_used += b.spec_used;
  a.spec_dropped += b.spec_dropped;
  a.bytes_pinned += b.bytes_pinned;
  a.bytes_disk += b.bytes_disk;
  a.wait_ns += b.wait_ns;
}

HostPlacement::HostPlacement(const Desc& d, const Plan& p, const ss_options& o) : d_(d), p_(p), o_(o) {
  require(int64_t(p_.tier.size()) == d_.total_units, SS_E_INVALID, "open: the plan is for another descriptor");
  excl_ = p_.budget.tier_mode == SS_TIER_MODE_EXCLUSIVE;
  // an exclusive-mode victim's slot is the only copy its write-back has: residents must hold their bytes from open
  require(!(excl_ && !o_.fill_residents), SS_E_INVALID, "open: the exclusive tier mode needs fill_residents = 1");
  require(!(excl_ && o_.exclusive_discard && d_.tiers == Tiers::Pinned), SS_E_INVALID,
          "open: exclusive_discard needs a descriptor whose tiers allow disk (tiers = \"pinned\" refuses it)");
  const size_t G = size_t(d_.total_units);

  // blocks: every pinned-tier home (in global unit order), then the spares of each class (lowest address first)
  const PinnedLayout pl = pinned_layout(d_, p_.tier);
  block_of_.assign(G, -1);
  for (size_t g = 0; g < G; ++g)
    if (pl.chunk_of[g] >= 0) {
      block_of_[g] = int32_t(blocks_.size());
      blocks_.push_back(BlockHome{int64_t(g), -1});
    }
  wb_batch_of_.assign(G, -1);
  L_.resize(d_.layers.size());
  if (excl_) {
    for (const SpareClass& c : p_.spares) class_bytes_.push_back(c.block_bytes);
    free_.resize(class_bytes_.size());
    for (size_t L = 0; L < d_.layers.size(); ++L) {
      const Layer& l = d_.layers[L];
      if (!l.streamable || !l.n_units) continue;
      const auto it = std::find(class_bytes_.begin(), class_bytes_.end(), host_stride(l.unit_bytes));
      require(it != class_bytes_.end(), SS_E_INVALID, "open: an exclusive plan without the layer's block class");
      L_[L].cls = int32_t(it - class_bytes_.begin());
      for (int u = 0; u < l.n_units; ++u)
        if (block_of_[size_t(d_.gidx(int(L), u))] >= 0) blocks_[size_t(block_of_[size_t(d_.gidx(int(L), u))])].cls =
            L_[L].cls;
    }
    for (size_t k = 0; k < p_.spares.size(); ++k) {
      const int32_t first = int32_t(blocks_.size());
      for (uint32_t i = 0; i < p_.spares[k].blocks; ++i) blocks_.push_back(BlockHome{-1, int32_t(k)});
      for (int32_t b = int32_t(blocks_.size()); b-- > first;) free_[k].push_back(b);  // lowest on top
      class_spares_.push_back(p_.spares[k].blocks);
      xst_.free_blocks += p_.spares[k].blocks;
    }
    xst_.min_free_blocks = xst_.free_blocks;
  }

  for (size_t L = 0; L < d_.layers.size(); ++L) {
    const Layer& l = d_.layers[L];
    LayerPlace& s = L_[L];
    if (!l.n_units) continue;
    int planned = 0;
    for (int u = 0; u < l.n_units; ++u) planned += resident_tier(p_.tier[size_t(d_.gidx(int(L), u))]) ? 1 : 0;
    const int cap = l.streamable ? std::min(l.n_units, planned + int(p_.dynamic_slots_per_layer)) : l.n_units;
    s.pool = std::make_unique<SlotPool>(l.n_units, cap, o_.policy, o_.score_window);
    s.spot.assign(size_t(l.n_units), DevSpot{});
    s.job.assign(size_t(l.n_units), -1);
    s.spec_open.assign(size_t(l.n_units), 0);
    s.uses.assign(size_t(l.n_units), 0);
    s.table.assign(size_t(l.n_units), DevSpot{});
    s.ra_asked.assign(size_t(l.n_units), 0);
  }
  // host read-ahead: buffers of the largest host stride a unit can be read from its file with (none: off)
  require(o_.readahead_units <= 64, SS_E_INVALID, "open: readahead_units must be <= 64");
  if (o_.readahead_units)
    for (size_t L = 0; L < d_.layers.size(); ++L) {
      const Layer& l = d_.layers[L];
      if (!l.streamable || !l.n_units) continue;
      for (int u = 0; u < l.n_units; ++u) {
        const uint8_t t = p_.tier[size_t(d_.gidx(int(L), u))];
        if (t == SS_TIER_PINNED || t == SS_TIER_PAIR) continue;
        ra_bytes_ = std::max(ra_bytes_, host_stride(l.unit_bytes));
        break;  // (a layer's units are one size)
      }
    }
  for (const RingClass& rc : p_.rings) {
    if (!rc.slots) continue;
    ring_cls_.push_back({rc.stride, uint32_t(ring_.size()), rc.slots});
    ring_cursor_.push_back(0);
    for (uint32_t i = 0; i < rc.slots; ++i) ring_.push_back(RingSlot{int32_t(ring_cls_.size() - 1)});
  }
  fwd_.assign(d_.layers.size(), ss_layer_stats{});
  total_.assign(d_.layers.size(), ss_layer_stats{});
}

uint64_t HostPlacement::free_blocks_now() const {
  uint64_t f = 0;
  for (const auto& v : free_) f += v.size();
  return f;
}

// ---- open and seeds -------------------------------------------------------------------------------------------------

void HostPlacement::place_residents() {
  for (size_t L = 0; L < d_.layers.size(); ++L) {
    const Layer& l = d_.layers[L];
    LayerPlace& s = L_[L];
    if (!s.pool) continue;
    for (int u = 0; u < l.n_units; ++u) {
      if (l.streamable && !resident_tier(p_.tier[size_t(d_.gidx(int(L), u))])) continue;
      const int slot = s.pool->place(u, !l.streamable || o_.pin_planned != 0);
      require(slot >= 0, SS_E_CAPACITY, "open: a planned resident found no pool slot (internal)");
      if (!o_.fill_residents) continue;
      FetchOrder f = order_for(int(L), u, false);
      f.dst = DevSpot{DevSpot::kPool, slot};
      f.after_release = int32_t(L);
      w_->fetch(f);
    }
  }
}

std::vector<int32_t> HostPlacement::seed(int layer, const int32_t* units, int n) {
  require(layer >= 0 && size_t(layer) < L_.size(), SS_E_INVALID, "seed: layer out of range");
  require(!in_fwd_ && !fwd_open_, SS_E_INVALID, "seed: only between forwards");
  LayerPlace& s = layer_with_units(layer, "seed");
  require(n >= 0 && (units || n == 0), SS_E_INVALID, "seed: bad unit list");
  const int nu = d_.layers[size_t(layer)].n_units;
  for (int i = 0; i < n; ++i) require(units[i] >= 0 && units[i] < nu, SS_E_INVALID, "seed: unit out of range");
  std::vector<int32_t> placed;
  placed.reserve(size_t(n));
  for (int i = 0; i < n; ++i) {
    const int u = units[i];
    if (s.pool->slot(u) >= 0 || p_.tier[size_t(d_.gidx(layer, u))] == SS_TIER_PAIR) continue;
    const int slot = s.pool->place(u, false);
    if (slot < 0) break;  // seeds take free slots only
    placed.push_back(u);
    FetchOrder f = order_for(layer, u, false);
    f.dst = DevSpot{DevSpot::kPool, slot};
    f.after_release = layer;  // the free slot's last reader: the layer in an earlier forward
    w_->fetch(f);
  }
  return placed;
}

void HostPlacement::seed_landed(int layer, int32_t unit, bool ok) {
  if (!ok) {
    L_[size_t(layer)].pool->drop(unit);
    return;
  }
  if (excl_) give_back_block(layer, unit);
}

// ---- orders ---------------------------------------------------------------------------------------------------------

HostPlacement::LayerPlace& HostPlacement::layer_with_units(int layer, const char* what) {
  LayerPlace& s = L_[size_t(layer)];
  require(s.pool != nullptr, SS_E_INVALID, std::string(what) + ": layer " + std::to_string(layer) + " has no units");
  return s;
}

int32_t HostPlacement::new_job(int layer, int unit, bool speculative, bool pool) {
  jobs_.push_back(Job{layer, unit, speculative, pool});
  return int32_t(jobs_.size() - 1);
}

FetchOrder HostPlacement::order_for(int layer, int unit, bool speculative) {
  FetchOrder f;
  f.layer = layer;
  f.unit = unit;
  f.speculative = speculative;
  const int64_t g = d_.gidx(layer, unit);
  f.src_block = block_of_[size_t(g)];
  if (excl_ && f.src_block >= 0) {
    f.src_writeback = wb_batch_of_[size_t(g)];
    if (f.src_writeback >= 0) ++xst_.rereads;  // its block is being written back this forward: read after it lands
  }
  return f;
}

void HostPlacement::fetch_pool(int layer, int unit, int32_t slot, bool speculative, int32_t after_writeback) {
  LayerPlace& s = L_[size_t(layer)];
  FetchOrder f = order_for(layer, unit, speculative);
  f.job = new_job(layer, unit, speculative, true);
  f.dst = DevSpot{DevSpot::kPool, slot};
  f.after_release = layer;  // the pool slot's last reader is this layer in an earlier forward
  f.after_writeback = after_writeback;
  s.spot[size_t(unit)] = f.dst;
  s.job[size_t(unit)] = f.job;
  if (!w_->fetch(f))  // (a landing from a read-ahead buffer: its file bytes count when the read-ahead ends)
    (f.src_block >= 0 ? fwd_[size_t(layer)].bytes_pinned : fwd_[size_t(layer)].bytes_disk) +=
        d_.layers[size_t(layer)].unit_bytes;
}

// The next free ring slot of the layer's stride class, round robin from the class's cursor.
bool HostPlacement::fetch_ring(int layer, int unit, bool speculative) {
  const uint64_t stride = d_.unit_stride(layer);
  size_t c = 0;
  while (c < ring_cls_.size() && ring_cls_[c].stride != stride) ++c;
  if (c == ring_cls_.size()) return false;
  const RingClassInfo& rc = ring_cls_[c];
  for (uint32_t k = 0; k < rc.count; ++k) {
    const uint32_t pos = (ring_cursor_[c] + k) % rc.count;
    RingSlot& r = ring_[rc.first + pos];
    if (r.owner >= 0) continue;
    ring_cursor_[c] = (pos + 1) % rc.count;
    LayerPlace& s = L_[size_t(layer)];
    FetchOrder f = order_for(layer, unit, speculative);
    f.job = new_job(layer, unit, speculative, false);
    f.dst = DevSpot{DevSpot::kRing, int32_t(rc.first + pos)};
    f.after_release = r.last_reader;
    r.owner = layer;
    r.job = f.job;
    s.spot[size_t(unit)] = f.dst;
    s.job[size_t(unit)] = f.job;
    if (!w_->fetch(f))
      (f.src_block >= 0 ? fwd_[size_t(layer)].bytes_pinned : fwd_[size_t(layer)].bytes_disk) +=
          d_.layers[size_t(layer)].unit_bytes;
    return true;
  }
  return false;
}

// Units waiting for a ring slot, in layer order: a later layer never takes a slot before an earlier one's waiters.
void HostPlacement::drain_waiting() {
  for (size_t L = 0; L < L_.size(); ++L) {
    std::vector<int32_t>& q = L_[L].waiting;
    size_t k = 0;
    while (k < q.size() && fetch_ring(int(L), q[k], false)) ++k;
    q.erase(q.begin(), q.begin() + std::ptrdiff_t(k));
    if (!q.empty()) return;
  }
}

uint64_t HostPlacement::free_for_writeback(int layer, bool speculative) const {
  const int32_t cls = L_[size_t(layer)].cls;
  if (cls < 0) return 0;
  uint64_t f = free_[size_t(cls)].size();
  if (speculative) {  // a guess leaves half of the class's spares to demands
    const uint64_t reserve = (class_spares_[size_t(cls)] + 1) / 2;
    f = f > reserve ? f - reserve : 0;
  }
  return f;
}

// Exclusive mode: one free block per victim; a demand admission with exclusive_discard is uncapped (victims past the
// free blocks go to their files).
int HostPlacement::eviction_cap(int layer, bool speculative) const {
  if (!excl_) return -1;
  if (L_[size_t(layer)].cls < 0) return 0;
  if (o_.exclusive_discard && !speculative) return -1;
  return int(std::min<uint64_t>(free_for_writeback(layer, speculative), uint64_t(INT32_MAX)));
}

void HostPlacement::admit(int layer, const Admission& a, bool speculative) {
  int32_t batch = -1;
  size_t written = 0;
  if (excl_ && !a.evicted.empty()) {
    const int32_t cls = L_[size_t(layer)].cls;
    const uint64_t room = free_for_writeback(layer, speculative);
    if (cls < 0 || (!o_.exclusive_discard && room < a.evicted.size()))
      fail(SS_E_BACKEND, "exclusive: more victims than free blocks (internal)");
    written = size_t(std::min<uint64_t>(room, a.evicted.size()));
    for (int32_t u : a.evicted)
      if (block_of_[size_t(d_.gidx(layer, u))] >= 0)
        fail(SS_E_BACKEND, "exclusive: a victim still owns a pinned block (internal)");
    xst_.discards += a.evicted.size() - written;  // past the free blocks: its file is its only home now
    if (written) {
      WriteBackOrder w;
      w.batch = batch = wb_batches_++;
      w.layer = layer;
      const uint64_t ub = d_.layers[size_t(layer)].unit_bytes;
      for (size_t i = 0; i < written; ++i) {
        const int64_t g = d_.gidx(layer, a.evicted[i]);
        const int32_t b = free_[size_t(cls)].back();
        free_[size_t(cls)].pop_back();
        block_of_[size_t(g)] = b;
        w.units.push_back(a.evicted[i]);
        w.slots.push_back(a.evicted_slot[i]);
        w.blocks.push_back(b);
        ++xst_.writebacks;
        xst_.writeback_bytes += ub;
      }
      w_->write_back(w);
      for (size_t i = 0; i < written; ++i) {
        const int64_t g = d_.gidx(layer, a.evicted[i]);
        wb_batch_of_[size_t(g)] = batch;
        wb_touched_.push_back(g);
      }
    }
  }
  for (size_t k = 0; k < a.admitted.size(); ++k) {
    int32_t after = -1;  // only a copy into a written-back victim's slot waits for the batch
    for (size_t i = 0; batch >= 0 && i < written && after < 0; ++i)
      if (a.evicted_slot[i] == a.admitted_slot[k]) after = batch;
    fetch_pool(layer, a.admitted[k], a.admitted_slot[k], speculative, after);
  }
}

void HostPlacement::give_back_block(int layer, int unit) {
  const int64_t g = d_.gidx(layer, unit);
  const int32_t b = block_of_[size_t(g)];
  if (b < 0) return;
  free_[size_t(L_[size_t(layer)].cls)].push_back(b);
  block_of_[size_t(g)] = -1;
  ++xst_.promoted;
}

// ---- the forward ------------------------------------------------------------------------------------------------------

void HostPlacement::open_forward() {
  if (fwd_open_) return;
  for (LayerPlace& s : L_) {
    if (!s.pool) continue;
    std::fill(s.spot.begin(), s.spot.end(), DevSpot{});
    std::fill(s.job.begin(), s.job.end(), -1);
    std::fill(s.spec_open.begin(), s.spec_open.end(), uint8_t(0));
    std::fill(s.uses.begin(), s.uses.end(), 0u);
    s.routed.clear();
    s.hits.clear();
    s.waiting.clear();
    s.groups.clear();
    std::fill(s.ra_asked.begin(), s.ra_asked.end(), uint8_t(0));
    s.routes_in = s.acquired = s.released = s.skipped = false;
  }
  std::fill(fwd_.begin(), fwd_.end(), ss_layer_stats{});
  fwd_open_ = true;
}

void HostPlacement::begin(const uint32_t* rows, int n_layers) {
  require(!in_fwd_, SS_E_INVALID, "begin: the previous forward has not ended");
  require(!rows || n_layers == int(L_.size()), SS_E_INVALID, "begin: rows_per_layer needs one entry per layer");
  open_forward();
  for (size_t L = 0; rows && L < L_.size(); ++L) L_[L].skipped = rows[L] == 0;
  if (excl_) {
    xst_.free_blocks = free_blocks_now();
    xst_.min_free_blocks = std::min(xst_.min_free_blocks, xst_.free_blocks);
  }
  in_fwd_ = true;
}

void HostPlacement::routes(int layer, const int32_t* ids, int n) {
  require(in_fwd_, SS_E_INVALID, "routes: outside a forward (call ss_begin)");
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "routes: bad ids");
  take_routes(layer, ids, n);
}

void HostPlacement::routes_all(int layer) {
  require(in_fwd_, SS_E_INVALID, "layer_all: outside a forward (call ss_begin)");
  std::vector<int32_t> all(static_cast<size_t>(d_.layers[size_t(layer)].n_units));
  for (size_t u = 0; u < all.size(); ++u) all[u] = int32_t(u);
  take_routes(layer, all.data(), int(all.size()));
}

// One layer's routes: hits stay, units fetched earlier in the forward are claimed, the other misses ask the pool
// for slots (evicting as it decides, write-backs first in exclusive mode) and the rest stream through the ring or
// wait for a ring slot.
void HostPlacement::take_routes(int layer, const int32_t* ids, int n) {
  LayerPlace& s = layer_with_units(layer, "routes");
  const Layer& l = d_.layers[size_t(layer)];
  require(!s.routes_in, SS_E_INVALID, "routes: already given for layer " + std::to_string(layer) + " in this forward");
  require(!s.skipped, SS_E_INVALID, "routes: layer " + std::to_string(layer) + " is skipped in this forward");
  for (int i = 0; i < n; ++i)
    require(ids[i] < l.n_units, SS_E_INVALID, "routes: unit id " + std::to_string(ids[i]) + " out of range");
  s.routes_in = true;
  for (int i = 0; i < n; ++i)
    if (ids[i] >= 0) ++s.uses[size_t(ids[i])];
  ss_layer_stats& st = fwd_[size_t(layer)];
  std::vector<char> busy(size_t(l.n_units), 0);
  std::vector<int32_t> misses, ask;
  for (int u = 0; u < l.n_units; ++u) {
    const bool placed = s.spot[size_t(u)].kind != DevSpot::kNone;
    busy[size_t(u)] = placed;
    if (!s.uses[size_t(u)] || p_.tier[size_t(d_.gidx(layer, u))] == SS_TIER_PAIR) continue;
    busy[size_t(u)] = 1;  // routed: never a victim of this layer's own misses
    s.routed.push_back(u);
    if (placed) {  // fetched earlier in this forward (a prefetch)
      if (s.spec_open[size_t(u)]) {
        s.spec_open[size_t(u)] = 0;
        ++st.spec_used;
        if (s.job[size_t(u)] >= 0) w_->promote(s.job[size_t(u)]);
      } else {
        ++st.prefetched;
      }
      misses.push_back(u);
    } else if (s.pool->slot(u) >= 0) {
      s.hits.push_back(u);
    } else {
      ask.push_back(u);
      misses.push_back(u);
    }
  }
  st.routed += s.routed.size();
  st.hits += s.hits.size();
  const Admission a = s.pool->admit(ask, busy, true, eviction_cap(layer, false));
  xst_.deferred += uint64_t(a.deferred);
  admit(layer, a, false);
  for (int32_t u : a.transient)
    if (!fetch_ring(layer, u, false)) {
      s.waiting.push_back(u);
      s.spot[size_t(u)] = DevSpot{DevSpot::kRing, -1};
      ra_request(layer, u, true);  // its file read need not wait for the ring slot
    }
  st.admitted += a.admitted.size();
  st.transient += a.transient.size();
  st.evicted += a.evicted.size();
  s.pool->observe(s.routed, misses);
}

// Prefetch before the layer's routes: CERTAIN admits like a demand; SPECULATIVE (at most lookahead_budget units) uses
// the ring only (unless spec_persistent) and never waits for a ring slot.
void HostPlacement::prefetch(int layer, const int32_t* ids, int n, bool speculative) {
  require(ids || n <= 0, SS_E_INVALID, "prefetch: bad ids");
  open_forward();
  LayerPlace& s = layer_with_units(layer, "prefetch");
  if (s.routes_in || s.acquired) return;  // too late to help
  const Layer& l = d_.layers[size_t(layer)];
  ss_layer_stats& st = fwd_[size_t(layer)];
  std::vector<char> busy(size_t(l.n_units), 0);
  for (int u = 0; u < l.n_units; ++u) busy[size_t(u)] = s.spot[size_t(u)].kind != DevSpot::kNone;
  uint32_t issued = 0;
  for (int i = 0; i < n; ++i) {
    if (speculative && issued >= o_.lookahead_budget) break;
    const int32_t u = ids[i];
    if (u < 0 || u >= l.n_units || busy[size_t(u)] || s.pool->slot(u) >= 0 ||
        p_.tier[size_t(d_.gidx(layer, u))] == SS_TIER_PAIR)
      continue;
    const Admission a = speculative && !o_.spec_persistent
                            ? Admission{}
                            : s.pool->admit({u}, busy, true, eviction_cap(layer, speculative));
    xst_.deferred += uint64_t(a.deferred);
    if (!a.admitted.empty()) {
      admit(layer, a, speculative);
      st.evicted += a.evicted.size();
    } else if (!fetch_ring(layer, u, speculative)) {
      if (speculative) break;
      s.waiting.push_back(u);
      s.spot[size_t(u)] = DevSpot{DevSpot::kRing, -1};
      ra_request(layer, u, true);
    }
    busy[size_t(u)] = 1;
    if (speculative) {
      s.spec_open[size_t(u)] = 1;
      ++st.spec_issued;
    }
    ++issued;
  }
}

void HostPlacement::host_prefetch(int layer, const int32_t* ids, int n) {
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "host_prefetch: bad ids");
  if (!ra_on()) return;  // read-ahead off: nothing to read
  open_forward();        // (between forwards: the requests belong to the next one)
  layer_with_units(layer, "host_prefetch");
  for (int i = 0; i < n; ++i) ra_request(layer, ids[i], false);
}

void HostPlacement::ra_request(int layer, int unit, bool pending_ok) {
  if (!ra_on()) return;
  LayerPlace& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  if (!s.pool || !l.streamable || unit < 0 || unit >= l.n_units || s.ra_asked[size_t(unit)]) return;
  if (!ra_wanted(layer, unit) || host_stride(l.unit_bytes) > ra_bytes_) return;
  const DevSpot& sp = s.spot[size_t(unit)];
  if (sp.kind != DevSpot::kNone && !(pending_ok && sp.kind == DevSpot::kRing && sp.index < 0)) return;
  s.ra_asked[size_t(unit)] = 1;
  w_->read_ahead(layer, unit);
}

bool HostPlacement::ra_wanted(int layer, int unit) const {
  const LayerPlace& s = L_[size_t(layer)];
  const int64_t g = d_.gidx(layer, unit);
  return s.pool && p_.tier[size_t(g)] != SS_TIER_PAIR && block_of_[size_t(g)] < 0 && s.pool->slot(unit) < 0 &&
         s.job[size_t(unit)] < 0;
}

HostPlacement::Acquire HostPlacement::acquire(int layer, bool wait_all) {
  LayerPlace& s = layer_with_units(layer, "acquire");
  drain_waiting();
  require(s.waiting.empty(), SS_E_CAPACITY,
          "acquire: the stream ring cannot take layer " + std::to_string(layer) + "'s " +
              std::to_string(s.waiting.size()) + " remaining transient units (release earlier layers or plan more "
              "ring slots)");
  Acquire r;
  r.wait_ready = s.ready_wait;
  s.ready_wait = false;
  // groups: 0 = resident before this forward; then the fetched units, most routed first (route order on ties),
  // group_units at a time, each group ascending
  std::vector<int32_t> fetched;
  for (int32_t u : s.routed)
    if (s.job[size_t(u)] >= 0) fetched.push_back(u);
  std::stable_sort(fetched.begin(), fetched.end(),
                   [&](int32_t a, int32_t b) { return s.uses[size_t(a)] > s.uses[size_t(b)]; });
  s.groups.assign(1, s.hits);
  const size_t per = o_.group_units ? size_t(o_.group_units) : std::max<size_t>(fetched.size(), 1);
  for (size_t k = 0; k < fetched.size(); k += per) {
    std::vector<int32_t> g(fetched.begin() + std::ptrdiff_t(k),
                           fetched.begin() + std::ptrdiff_t(std::min(fetched.size(), k + per)));
    std::sort(g.begin(), g.end());
    s.groups.push_back(std::move(g));
  }
  if (wait_all)
    for (int32_t u : fetched) r.wait_jobs.push_back(s.job[size_t(u)]);
  return r;
}

const std::vector<DevSpot>& HostPlacement::take_table(int layer) {
  LayerPlace& s = L_[size_t(layer)];
  // every routed unit, and every resident not fetched this forward
  for (size_t u = 0; u < s.table.size(); ++u) {
    DevSpot& t = s.table[u];
    const bool present = s.job[u] >= 0 ? s.uses[u] != 0 : s.pool->slot(int(u)) >= 0;
    if (!present) t = DevSpot{};
    else if (s.spot[u].kind == DevSpot::kRing) t = s.spot[u];
    else t = DevSpot{DevSpot::kPool, s.pool->slot(int(u))};
  }
  s.acquired = true;
  return s.table;
}

std::vector<int32_t> HostPlacement::group_jobs(int layer, int group) const {
  std::vector<int32_t> out;
  const LayerPlace& s = L_[size_t(layer)];
  if (group <= 0) return out;
  for (int32_t u : s.groups[size_t(group)]) out.push_back(s.job[size_t(u)]);
  return out;
}

void HostPlacement::release(int layer) {
  LayerPlace& s = L_[size_t(layer)];
  s.released = true;
  for (size_t u = 0; u < s.spec_open.size(); ++u)
    if (s.spec_open[u]) {
      s.spec_open[u] = 0;
      ++fwd_[size_t(layer)].spec_dropped;
    }
  for (RingSlot& r : ring_) {
    if (r.owner != layer) continue;
    w_->retire(r.job);
    r.last_reader = layer;
    r.owner = r.job = -1;
  }
  drain_waiting();
}

HostPlacement::Ended HostPlacement::end() {
  std::vector<uint8_t> done(jobs_.size(), 0);
  for (size_t j = 0; j < jobs_.size(); ++j) done[j] = w_->settle(int32_t(j), jobs_[j].speculative) ? 1 : 0;
  Ended e;
  for (size_t L = 0; L < L_.size(); ++L) {
    LayerPlace& s = L_[L];
    if (!s.pool) continue;
    bool landed = false;
    for (size_t u = 0; u < s.spot.size(); ++u) {
      if (s.spec_open[u]) ++fwd_[L].spec_dropped;
      if (s.spot[u].kind != DevSpot::kPool || s.job[u] < 0) continue;
      if (!done[size_t(s.job[u])]) {
        s.pool->drop(int(u));  // its copy never ran (a speculative read cancelled, or a failed one): not resident
        continue;
      }
      landed = true;
      if (excl_) give_back_block(int(L), int(u));  // promoted: its pinned block is free again
    }
    if (landed) {
      s.ready_wait = true;
      e.landed_layers.push_back(int(L));
    }
  }
  for (RingSlot& r : ring_) r.owner = r.job = -1;
  if (excl_) {
    for (int64_t g : wb_touched_) wb_batch_of_[size_t(g)] = -1;
    wb_touched_.clear();
    xst_.free_blocks = free_blocks_now();
  }
  e.writeback_batches = uint32_t(wb_batches_);
  wb_batches_ = 0;
  jobs_.clear();
  for (size_t L = 0; L < L_.size(); ++L) add_stats(total_[L], fwd_[L]);
  ++forwards_;
  in_fwd_ = fwd_open_ = false;
  return e;
}

void HostPlacement::reset_stats() { std::fill(total_.begin(), total_.end(), ss_layer_stats{}); }

}  // namespace tsa
