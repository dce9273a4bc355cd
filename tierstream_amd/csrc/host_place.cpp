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
      spare_.add_class(int32_t(blocks_.size()), p_.spares[k].blocks);
      blocks_.resize(blocks_.size() + p_.spares[k].blocks, BlockHome{-1, int32_t(k)});
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
  for (const RingClass& rc : p_.rings)
    if (rc.slots) {
      ring_cls_.push_back({rc.stride, ring_.size(), rc.slots});
      ring_.add_class(rc.stride, rc.slots);
    }
  fwd_.assign(d_.layers.size(), ss_layer_stats{});
  total_.assign(d_.layers.size(), ss_layer_stats{});
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

// Every forward copy goes out through here: the unit's spot and job for this forward, the executor's copy, and its
// bytes (a copy that lands from a read-ahead buffer has its file bytes counted when the read-ahead ends).
void HostPlacement::issue(const FetchOrder& f) {
  LayerPlace& s = L_[size_t(f.layer)];
  s.spot[size_t(f.unit)] = f.dst;
  s.job[size_t(f.unit)] = f.job;
  if (w_->fetch(f)) return;
  ss_layer_stats& st = fwd_[size_t(f.layer)];
  (f.src_block >= 0 ? st.bytes_pinned : st.bytes_disk) += d_.layers[size_t(f.layer)].unit_bytes;
}

bool HostPlacement::stream(int layer, int unit, bool speculative) {
  const int cls = ring_.class_for(d_.unit_stride(layer));
  if (!ring_.has_free(cls)) return false;
  FetchOrder f = order_for(layer, unit, speculative);
  f.job = new_job(layer, unit, speculative, false);
  const RingPool::Grant g = ring_.grant(cls, layer, f.job);
  f.dst = DevSpot{DevSpot::kRing, g.slot};
  f.after_release = g.prev_reader;
  issue(f);
  return true;
}

// No ring slot for now: the unit queues for one (kRing without a slot marks it placed), and its file read, if it has
// one to make, need not wait for the slot.
void HostPlacement::wait_for_ring(int layer, int unit) {
  L_[size_t(layer)].spot[size_t(unit)] = DevSpot{DevSpot::kRing, -1};
  line_.join(layer, unit);
  ra_request(layer, unit, true);
}

void HostPlacement::serve_wait_line() {
  line_.serve([this](int32_t layer, int32_t unit) { return stream(layer, unit, false); });
}

HostPlacement::VictimBudget HostPlacement::victim_budget(int layer, bool speculative) const {
  VictimBudget b;
  if (!excl_) return b;  // inclusive: a victim simply leaves its slot
  const int32_t cls = L_[size_t(layer)].cls;
  if (cls >= 0) {
    // a speculative admission leaves half of the class's spares (rounded up) to demand admissions
    const uint64_t keep = speculative ? (uint64_t(spare_.spares(cls)) + 1) / 2 : 0;
    const uint64_t have = spare_.free(cls);
    b.blocks = have > keep ? have - keep : 0;
  }
  // one block per victim, except that a demand admission with exclusive_discard evicts as it needs (its victims past
  // the blocks are dropped to their files); a layer without a block class evicts nothing
  b.cap = cls < 0 ? 0 : (o_.exclusive_discard && !speculative) ? -1 : int(std::min<uint64_t>(b.blocks, INT32_MAX));
  return b;
}

// Exclusive mode: the first victims (while the budget's blocks last) are written back into free blocks as one batch;
// the rest are discarded to their files. Every victim was a resident, which owns no block.
int32_t HostPlacement::write_back_victims(int layer, const Admission& a, const VictimBudget& b) {
  const int32_t cls = L_[size_t(layer)].cls;
  const size_t n = a.evicted.size();
  if (cls < 0 || (n > b.blocks && !o_.exclusive_discard))
    fail(SS_E_BACKEND, "exclusive: admission evicted past its victim budget (internal)");
  for (int32_t u : a.evicted)
    if (block_of_[size_t(d_.gidx(layer, u))] >= 0) fail(SS_E_BACKEND, "exclusive: a resident victim had a pinned block (internal)");
  const size_t kept = size_t(std::min<uint64_t>(b.blocks, n));
  xst_.discards += n - kept;
  if (!kept) return -1;
  WriteBackOrder w;
  w.batch = wb_batches_++;
  w.layer = layer;
  w.units.assign(a.evicted.begin(), a.evicted.begin() + std::ptrdiff_t(kept));
  w.slots.assign(a.evicted_slot.begin(), a.evicted_slot.begin() + std::ptrdiff_t(kept));
  for (int32_t u : w.units) {
    const size_t g = size_t(d_.gidx(layer, u));
    const int32_t blk = spare_.take(cls);
    block_of_[g] = blk;
    w.blocks.push_back(blk);
  }
  xst_.writebacks += kept;
  xst_.writeback_bytes += kept * d_.layers[size_t(layer)].unit_bytes;
  w_->write_back(w);
  // published after the order: a read of one of these blocks later in the forward waits for the batch
  for (int32_t u : w.units) {
    const int64_t g = d_.gidx(layer, u);
    wb_batch_of_[size_t(g)] = w.batch;
    wb_touched_.push_back(g);
  }
  return w.batch;
}

Admission HostPlacement::admit_units(int layer, const std::vector<int32_t>& units, const std::vector<char>& held,
                                     bool speculative) {
  const VictimBudget b = victim_budget(layer, speculative);
  Admission a = L_[size_t(layer)].pool->admit(units, held, true, b.cap);
  xst_.deferred += uint64_t(a.deferred);
  const int32_t batch = excl_ && !a.evicted.empty() ? write_back_victims(layer, a, b) : -1;
  // a copy into a slot whose victim went out in the batch waits for it; the written victims are the first ones
  std::vector<int32_t> wb_slots;
  if (batch >= 0) {
    const size_t kept = size_t(std::min<uint64_t>(b.blocks, a.evicted.size()));
    wb_slots.assign(a.evicted_slot.begin(), a.evicted_slot.begin() + std::ptrdiff_t(kept));
  }
  for (size_t k = 0; k < a.admitted.size(); ++k) {
    FetchOrder f = order_for(layer, a.admitted[k], speculative);
    f.job = new_job(layer, a.admitted[k], speculative, true);
    f.dst = DevSpot{DevSpot::kPool, a.admitted_slot[k]};
    f.after_release = layer;  // a pool slot's last reader is this layer, in an earlier forward
    if (std::find(wb_slots.begin(), wb_slots.end(), a.admitted_slot[k]) != wb_slots.end()) f.after_writeback = batch;
    issue(f);
  }
  return a;
}

void HostPlacement::give_back_block(int layer, int unit) {
  const int64_t g = d_.gidx(layer, unit);
  const int32_t b = block_of_[size_t(g)];
  if (b < 0) return;
  spare_.give(L_[size_t(layer)].cls, b);
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
    std::fill(s.ra_asked.begin(), s.ra_asked.end(), uint8_t(0));
    s.routed.clear();
    s.hits.clear();
    s.groups.clear();
    s.routes_in = s.acquired = s.released = s.skipped = false;
  }
  line_.clear();
  std::fill(fwd_.begin(), fwd_.end(), ss_layer_stats{});
  fwd_open_ = true;
}

void HostPlacement::begin(const uint32_t* rows, int n_layers) {
  require(!in_fwd_, SS_E_INVALID, "begin: the previous forward has not ended");
  require(!rows || n_layers == int(L_.size()), SS_E_INVALID, "begin: rows_per_layer needs one entry per layer");
  open_forward();
  if (rows)
    for (size_t L = 0; L < L_.size(); ++L) L_[L].skipped = rows[L] == 0;
  if (excl_) {
    xst_.free_blocks = spare_.total_free();
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

HostPlacement::RouteSort HostPlacement::sort_routes(int layer) const {
  const LayerPlace& s = L_[size_t(layer)];
  const int n = d_.layers[size_t(layer)].n_units;
  RouteSort r;
  r.held.assign(size_t(n), 0);
  for (int u = 0; u < n; ++u) {
    const bool placed = s.spot[size_t(u)].kind != DevSpot::kNone;
    const bool routed = s.uses[size_t(u)] && p_.tier[size_t(d_.gidx(layer, u))] != SS_TIER_PAIR;
    r.held[size_t(u)] = char(placed || routed);
    if (!routed) continue;
    if (placed) r.claims.push_back(u);
    else if (s.pool->slot(u) >= 0) r.hits.push_back(u);
    else r.asks.push_back(u);
  }
  return r;
}

// One layer's routes: hits stay, units placed earlier in the forward are claimed, the others ask the pool for slots
// (victims written back first in exclusive mode) and whatever the pool does not take streams through the ring or
// waits for a ring slot.
void HostPlacement::take_routes(int layer, const int32_t* ids, int n) {
  LayerPlace& s = layer_with_units(layer, "routes");
  const int nu = d_.layers[size_t(layer)].n_units;
  require(!s.routes_in, SS_E_INVALID, "routes: already given for layer " + std::to_string(layer) + " in this forward");
  require(!s.skipped, SS_E_INVALID, "routes: layer " + std::to_string(layer) + " is skipped in this forward");
  const int32_t* bad = std::find_if(ids, ids + n, [nu](int32_t id) { return id >= nu; });
  require(bad == ids + n, SS_E_INVALID, "routes: unit id " + std::to_string(bad == ids + n ? 0 : *bad) +
                                            " out of range");
  s.routes_in = true;
  for (int i = 0; i < n; ++i)
    if (ids[i] >= 0) ++s.uses[size_t(ids[i])];  // (negative ids are empty route entries)

  RouteSort r = sort_routes(layer);
  ss_layer_stats& st = fwd_[size_t(layer)];
  for (int32_t u : r.claims) {
    if (!s.spec_open[size_t(u)]) {
      ++st.prefetched;
      continue;
    }
    s.spec_open[size_t(u)] = 0;  // a guess that came true: its job turns into a demand
    ++st.spec_used;
    if (s.job[size_t(u)] >= 0) w_->promote(s.job[size_t(u)]);
  }
  std::vector<int32_t> misses(r.claims.size() + r.asks.size());
  std::merge(r.claims.begin(), r.claims.end(), r.asks.begin(), r.asks.end(), misses.begin());
  s.hits = std::move(r.hits);
  std::merge(misses.begin(), misses.end(), s.hits.begin(), s.hits.end(), std::back_inserter(s.routed));
  st.routed += s.routed.size();
  st.hits += s.hits.size();

  const Admission a = admit_units(layer, r.asks, r.held, false);
  for (int32_t u : a.transient)
    if (!stream(layer, u, false)) wait_for_ring(layer, u);
  st.admitted += a.admitted.size();
  st.transient += a.transient.size();
  st.evicted += a.evicted.size();
  s.pool->observe(s.routed, misses);
}

// Prefetch before the layer's routes, in the order asked: CERTAIN places a unit as a demand would (admission, else the
// ring, else the wait line); SPECULATIVE places at most lookahead_budget units, in the ring only unless spec_persistent
// (a guess never evicts otherwise), and stops at the first unit the ring cannot take (a guess never waits).
void HostPlacement::prefetch(int layer, const int32_t* ids, int n, bool speculative) {
  require(ids || n <= 0, SS_E_INVALID, "prefetch: bad ids");
  open_forward();
  LayerPlace& s = layer_with_units(layer, "prefetch");
  if (s.routes_in || s.acquired) return;  // too late to help
  const int nu = d_.layers[size_t(layer)].n_units;
  ss_layer_stats& st = fwd_[size_t(layer)];
  std::vector<char> held(static_cast<size_t>(nu), 0);
  for (int u = 0; u < nu; ++u) held[size_t(u)] = char(s.spot[size_t(u)].kind != DevSpot::kNone);
  const bool admits = !speculative || o_.spec_persistent;
  const uint32_t budget = speculative ? o_.lookahead_budget : UINT32_MAX;
  uint32_t placed = 0;
  for (int i = 0; i < n && placed < budget; ++i) {
    const int32_t u = ids[i];
    const bool wanted = u >= 0 && u < nu && !held[size_t(u)] && s.pool->slot(u) < 0 &&
                        p_.tier[size_t(d_.gidx(layer, u))] != SS_TIER_PAIR;
    if (!wanted) continue;
    // the admission's deferrals count even when it admitted nothing
    const Admission a = admits ? admit_units(layer, {u}, held, speculative) : Admission{};
    if (!a.admitted.empty()) {
      st.evicted += a.evicted.size();
    } else if (!stream(layer, u, speculative)) {
      if (speculative) return;
      wait_for_ring(layer, u);
    }
    held[size_t(u)] = 1;
    ++placed;
    if (speculative) {
      s.spec_open[size_t(u)] = 1;
      ++st.spec_issued;
    }
  }
}

void HostPlacement::host_prefetch(int layer, const int32_t* ids, int n) {
  require(n >= 0 && (ids || n == 0), SS_E_INVALID, "host_prefetch: bad ids");
  if (!ra_on()) return;  // read-ahead off: nothing to read
  open_forward();        // (between forwards: the requests belong to the next one)
  layer_with_units(layer, "host_prefetch");
  for (int i = 0; i < n; ++i) ra_request(layer, ids[i], false);
}

// kDevice: resident, or a copy of it already ordered this forward; kPinned: it has a pinned block; kPeer: a PAIR unit
// (never fetched); kFile: only its file holds it.
HostPlacement::Source HostPlacement::source_now(int layer, int unit) const {
  const LayerPlace& s = L_[size_t(layer)];
  const size_t g = size_t(d_.gidx(layer, unit));
  if (p_.tier[g] == SS_TIER_PAIR) return Source::kPeer;
  if (s.pool->slot(unit) >= 0 || s.job[size_t(unit)] >= 0) return Source::kDevice;
  return block_of_[g] >= 0 ? Source::kPinned : Source::kFile;
}

bool HostPlacement::ra_wanted(int layer, int unit) const {
  return L_[size_t(layer)].pool && source_now(layer, unit) == Source::kFile;
}

// Read-ahead is asked for at most once per unit and forward, for a streamable unit its file alone holds whose bytes
// fit a buffer, and which is not placed this forward (or, waiting_ok, only waits for a ring slot).
void HostPlacement::ra_request(int layer, int unit, bool waiting_ok) {
  if (!ra_on() || layer < 0 || size_t(layer) >= L_.size()) return;
  LayerPlace& s = L_[size_t(layer)];
  const Layer& l = d_.layers[size_t(layer)];
  if (!s.pool || !l.streamable || unit < 0 || unit >= l.n_units || s.ra_asked[size_t(unit)]) return;
  const DevSpot& at = s.spot[size_t(unit)];
  const bool free_to_read = at.kind == DevSpot::kNone || (waiting_ok && at.kind == DevSpot::kRing && at.index < 0);
  if (!free_to_read || host_stride(l.unit_bytes) > ra_bytes_ || source_now(layer, unit) != Source::kFile) return;
  s.ra_asked[size_t(unit)] = 1;
  w_->read_ahead(layer, unit);
}

HostPlacement::Acquire HostPlacement::acquire(int layer, bool wait_all) {
  LayerPlace& s = layer_with_units(layer, "acquire");
  serve_wait_line();
  const uint32_t left = line_.waiting(layer);
  require(left == 0, SS_E_CAPACITY,
          "acquire: the stream ring cannot take layer " + std::to_string(layer) + "'s " + std::to_string(left) +
              " remaining transient units (release earlier layers or plan more ring slots)");
  Acquire r;
  r.wait_ready = s.ready_wait;
  s.ready_wait = false;
  // group 0: the units resident before this forward; then the units fetched for it, most-routed first (lower id
  // first among equals), group_units to a group (all in one without it), each group in id order
  std::vector<int32_t> fetched;
  std::copy_if(s.routed.begin(), s.routed.end(), std::back_inserter(fetched),
               [&s](int32_t u) { return s.job[size_t(u)] >= 0; });
  std::sort(fetched.begin(), fetched.end(), [&s](int32_t a, int32_t b) {
    return s.uses[size_t(a)] != s.uses[size_t(b)] ? s.uses[size_t(a)] > s.uses[size_t(b)] : a < b;
  });
  s.groups.assign(1, s.hits);
  const size_t per = o_.group_units ? size_t(o_.group_units) : fetched.size();
  for (auto it = fetched.begin(); it != fetched.end();) {
    const auto stop = per && size_t(fetched.end() - it) > per ? it + std::ptrdiff_t(per) : fetched.end();
    s.groups.emplace_back(it, stop);
    std::sort(s.groups.back().begin(), s.groups.back().end());
    it = stop;
  }
  if (wait_all)
    for (int32_t u : fetched) r.wait_jobs.push_back(s.job[size_t(u)]);
  return r;
}

// The layer's table: a unit fetched this forward appears where its copy went, if it was routed; any other unit
// appears in its pool slot if it is resident.
const std::vector<DevSpot>& HostPlacement::take_table(int layer) {
  LayerPlace& s = L_[size_t(layer)];
  for (size_t u = 0; u < s.table.size(); ++u) {
    if (s.job[u] >= 0) {
      s.table[u] = s.uses[u] ? s.spot[u] : DevSpot{};
      continue;
    }
    const int slot = s.pool->slot(int(u));
    s.table[u] = slot >= 0 ? DevSpot{DevSpot::kPool, slot} : DevSpot{};
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
  const auto open = std::count(s.spec_open.begin(), s.spec_open.end(), uint8_t(1));
  fwd_[size_t(layer)].spec_dropped += uint64_t(open);  // guesses never routed
  std::fill(s.spec_open.begin(), s.spec_open.end(), uint8_t(0));
  ring_.release(layer, [this](int32_t job) { w_->retire(job); });
  serve_wait_line();
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
  ring_.reset_holders();
  line_.clear();
  if (excl_) {
    for (int64_t g : wb_touched_) wb_batch_of_[size_t(g)] = -1;
    wb_touched_.clear();
    xst_.free_blocks = spare_.total_free();
  }
  e.writeback_batches = uint32_t(wb_batches_);
  wb_batches_ = 0;
  jobs_.clear();
  for (size_t L = 0; L < L_.size(); ++L) add_stats(total_[L], fwd_[L]);
  ++forwards_;
  in_fwd_ = fwd_open_ = false;
  return e;
}

void HostPlacement::check_blocks() const {
  require(excl_, SS_E_INVALID, "check_exclusive: the context is not in the exclusive tier mode");
  require(!in_fwd_ && !fwd_open_, SS_E_INVALID, "check_exclusive: only between forwards");
  std::vector<uint32_t> holders(blocks_.size(), 0);
  for (size_t L = 0; L < L_.size(); ++L) {
    if (!L_[L].pool) continue;
    const Layer& l = d_.layers[L];
    for (int u = 0; u < l.n_units; ++u) {
      const size_t g = size_t(d_.gidx(int(L), u));
      if (p_.tier[g] == SS_TIER_PAIR) continue;  // another device's unit
      require(wb_batch_of_[g] < 0, SS_E_INVALID, "check_exclusive: a write-back is still pending at a boundary");
      const int32_t b = block_of_[g];
      if (b < 0) continue;
      const std::string who = "unit (" + std::to_string(L) + ", " + std::to_string(u) + ")";
      require(l.streamable, SS_E_INVALID, "check_exclusive: " + who + " is not streamable and owns a block");
      require(L_[L].pool->slot(u) < 0, SS_E_INVALID, "check_exclusive: " + who + " is in a slot and a block");
      ++holders[size_t(b)];
    }
  }
  for (size_t k = 0; k < spare_.classes(); ++k)
    for (int32_t b : spare_.free_list(int(k))) ++holders[size_t(b)];
  for (size_t b = 0; b < holders.size(); ++b)
    require(holders[b] == 1, SS_E_INVALID,
            "check_exclusive: block " + std::to_string(b) + (holders[b] ? " is held twice" : " is held by no one"));
}

void HostPlacement::reset_stats() { std::fill(total_.begin(), total_.end(), ss_layer_stats{}); }

}  // namespace tsa
