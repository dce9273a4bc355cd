#include "residency.hpp"

#include <algorithm>
#include <numeric>

#include "common.hpp"

namespace tsa {

// ---- ScoreBook ------------------------------------------------------------------------------------------------------

ScoreBook::ScoreBook(int n_units, uint32_t window)
    : n_(n_units), window_(window ? window : 16), follow_(size_t(n_units) * size_t(n_units), 0),
      led_(size_t(n_units), 0), hits_(size_t(n_units), 0), ring_(window ? window : 16) {}

void ScoreBook::record(const std::vector<int32_t>& routed) {
  for (int32_t p : last_) {
    ++led_[size_t(p)];
    uint32_t* row = follow_.data() + size_t(p) * size_t(n_);
    for (int32_t v : routed) ++row[size_t(v)];
  }
  last_ = routed;
  if (filled_ == window_) {  // the oldest forward leaves the window
    for (int32_t v : ring_[head_]) --hits_[size_t(v)];
    ring_[head_] = routed;
    head_ = (head_ + 1) % window_;
  } else {
    ring_[(head_ + filled_) % window_] = routed;
    ++filled_;
  }
  for (int32_t v : routed) ++hits_[size_t(v)];
}

// The mean over the last forward's units p of P(u follows p), each estimated as follow[p][u] / led[p] (0 for a unit
// never followed), summed in ascending p.
double ScoreBook::transition(int32_t u) const {
  if (last_.empty()) return 0.0;
  double sum = 0.0;
  for (int32_t p : last_) {
    const uint32_t led = led_[size_t(p)];
    if (led) sum += double(follow_[size_t(p) * size_t(n_) + size_t(u)]) / double(led);
  }
  return sum / double(last_.size());
}

double ScoreBook::frequency(int32_t u) const {
  return filled_ ? double(hits_[size_t(u)]) / double(filled_) : 0.0;
}

// ---- SlotPool -------------------------------------------------------------------------------------------------------

SlotPool::SlotPool(int n_units, int capacity, ss_policy policy, uint32_t window)
    : n_(n_units), policy_(policy) {
  require(capacity >= 0 && capacity <= n_units, SS_E_INVALID, "slot pool: capacity must be 0..n_units");
  slot_of_.assign(size_t(n_units), -1);
  holder_.assign(size_t(capacity), -1);
  pinned_.assign(size_t(capacity), 0);
  used_.assign(size_t(n_units), 0);
  for (int s = 0; s < capacity; ++s) free_.insert(free_.end(), s);
  if (policy == SS_POLICY_SCORED) book_.emplace_back(n_units, window);
}

void SlotPool::occupy(int32_t s, int32_t u, bool pin) {
  free_.erase(s);
  holder_[size_t(s)] = u;
  pinned_[size_t(s)] = pin ? 1 : 0;
  slot_of_[size_t(u)] = s;
  if (!pin) lru_.emplace(used_[size_t(u)], u);
}

void SlotPool::vacate(int32_t s) {
  const int32_t u = holder_[size_t(s)];
  if (!pinned_[size_t(s)]) lru_.erase({used_[size_t(u)], u});
  holder_[size_t(s)] = -1;
  pinned_[size_t(s)] = 0;
  slot_of_[size_t(u)] = -1;
  free_.insert(s);
}

void SlotPool::touch(int32_t u, uint64_t when) {
  const int32_t s = slot_of_[size_t(u)];
  const bool indexed = s >= 0 && !pinned_[size_t(s)];
  if (indexed) lru_.erase({used_[size_t(u)], u});
  used_[size_t(u)] = when;
  if (indexed) lru_.emplace(when, u);
}

int SlotPool::place(int unit, bool pin) {
  require(unit >= 0 && unit < n_, SS_E_INVALID, "slot pool: unit out of range");
  const int32_t have = slot_of_[size_t(unit)];
  if (have >= 0) {
    if (pin && !pinned_[size_t(have)]) {
      lru_.erase({used_[size_t(unit)], unit});
      pinned_[size_t(have)] = 1;
    }
    return have;
  }
  if (free_.empty()) return -1;
  const int32_t s = *free_.begin();
  occupy(s, unit, pin);
  return s;
}

void SlotPool::drop(int unit) {
  const int32_t s = slot_of_[size_t(unit)];
  if (s >= 0) vacate(s);
}

// 0.7 x transition + 0.2 x frequency + 0.1 / (1 + forwards since the last use); a unit never used scores no recency.
// (The terms and their order of evaluation are fixed: admissions must rank exactly as the reference ranks them.)
double SlotPool::score(int32_t u) const {
  const ScoreBook& b = book_.front();
  const double trans = b.transition(u);
  const double freq = b.frequency(u);
  const uint64_t last = used_[size_t(u)];
  const double recency = last ? 1.0 / (1.0 + double(clock_ - last)) : 0.0;
  return 0.7 * trans + 0.2 * freq + 0.1 * recency;
}

Admission SlotPool::admit(const std::vector<int32_t>& routed_in, const std::vector<char>& busy, bool admit_misses,
                          int max_evictions) {
  Admission a;
  std::vector<int32_t> routed(routed_in);
  std::sort(routed.begin(), routed.end());
  routed.erase(std::unique(routed.begin(), routed.end()), routed.end());
  // protected[u]: never a victim of this call (routed, in flight, admitted by it, or ranked inside the pool)
  std::vector<char> protect(size_t(n_), 0);
  std::vector<int32_t> misses;
  for (int32_t u : routed) {
    require(u >= 0 && u < n_, SS_E_INVALID, "routes: unit id out of range");
    protect[size_t(u)] = 1;
    (slot_of_[size_t(u)] >= 0 ? a.hits : misses).push_back(u);
  }
  const size_t nb = std::min(busy.size(), protect.size());
  for (size_t u = 0; u < nb; ++u) protect[u] |= busy[u];
  if (!admit_misses || holder_.empty()) {
    a.transient = std::move(misses);
    return a;
  }

  // The misses that ask for a slot, in the order they ask.
  std::vector<int32_t> askers;
  if (policy_ != SS_POLICY_SCORED) {
    askers = misses;
  } else {
    // The unpinned residents outside this forward compete with the misses for the pool's rows (its free slots plus
    // those residents): the best-ranked rows stay or come in; residents ranked below lose their protection.
    struct Ranked {
      double score;
      uint64_t last;
      int32_t unit;
      bool resident;
    };
    std::vector<Ranked> field;
    for (const auto& e : lru_)
      if (!protect[size_t(e.second)]) field.push_back({score(e.second), e.first, e.second, true});
    const size_t rows = free_.size() + field.size();
    for (int32_t u : misses) field.push_back({score(u), used_[size_t(u)], u, false});
    auto better = [](const Ranked& x, const Ranked& y) {
      if (x.score != y.score) return x.score > y.score;
      if (x.last != y.last) return x.last > y.last;
      return x.unit < y.unit;
    };
    const size_t top = std::min(rows, field.size());
    std::partial_sort(field.begin(), field.begin() + std::ptrdiff_t(top), field.end(), better);
    for (size_t i = 0; i < top; ++i) {
      if (field[i].resident) protect[size_t(field[i].unit)] = 1;
      else askers.push_back(field[i].unit);
    }
    // pinned residents are outside the index and never victims; protecting them here changes nothing
  }

  std::vector<char> got(size_t(n_), 0);
  for (int32_t u : askers) {
    int32_t s;
    if (!free_.empty()) {
      s = *free_.begin();
    } else {
      if (max_evictions >= 0 && int(a.evicted.size()) >= max_evictions) {
        ++a.deferred;
        continue;
      }
      auto v = lru_.begin();
      while (v != lru_.end() && protect[size_t(v->second)]) ++v;
      if (v == lru_.end()) break;  // every resident is pinned or protected: the rest stay transient
      const int32_t old = v->second;
      s = slot_of_[size_t(old)];
      vacate(s);
      a.evicted.push_back(old);
      a.evicted_slot.push_back(s);
    }
    occupy(s, u, false);
    protect[size_t(u)] = 1;
    got[size_t(u)] = 1;
    a.admitted.push_back(u);
    a.admitted_slot.push_back(s);
  }
  for (int32_t u : misses)
    if (!got[size_t(u)]) a.transient.push_back(u);

  auto by_unit = [](std::vector<int32_t>& units, std::vector<int32_t>& slots) {
    std::vector<size_t> order(units.size());
    std::iota(order.begin(), order.end(), size_t(0));
    std::sort(order.begin(), order.end(), [&](size_t x, size_t y) { return units[x] < units[y]; });
    std::vector<int32_t> u2(units.size()), s2(slots.size());
    for (size_t i = 0; i < order.size(); ++i) {
      u2[i] = units[order[i]];
      s2[i] = slots[order[i]];
    }
    units.swap(u2);
    slots.swap(s2);
  };
  by_unit(a.admitted, a.admitted_slot);
  by_unit(a.evicted, a.evicted_slot);
  return a;
}

void SlotPool::observe(const std::vector<int32_t>& routed_in, const std::vector<int32_t>& misses) {
  std::vector<int32_t> routed(routed_in);
  std::sort(routed.begin(), routed.end());
  routed.erase(std::unique(routed.begin(), routed.end()), routed.end());
  ++clock_;
  if (policy_ != SS_POLICY_SCORED) {
    for (int32_t u : routed) touch(u, clock_);
    return;
  }
  // SCORED: a miss (admitted or transient) and a first use refresh recency; a hit does not
  for (int32_t u : misses) touch(u, clock_);
  for (int32_t u : routed)
    if (!used_[size_t(u)]) touch(u, clock_);
  book_.front().record(routed);
}

}  // namespace tsa
