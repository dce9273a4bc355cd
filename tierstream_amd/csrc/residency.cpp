#include "residency.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>

#include "common.hpp"

namespace tsa {

Residency::Residency(int n_units, int capacity, ss_policy policy, uint32_t window)
    : n_(n_units), policy_(policy), window_(window ? window : 16) {
  require(capacity >= 0 && capacity <= n_units, SS_E_INVALID, "resident set: capacity must be 0..n_units");
  slot_of_.assign(size_t(n_units), -1);
  unit_in_.assign(size_t(capacity), -1);
  pin_.assign(size_t(capacity), 0);
  last_.assign(size_t(n_units), 0);
  if (policy_ == SS_POLICY_SCORED) {
    trans_.assign(size_t(n_units) * size_t(n_units), 0);
    trans_n_.assign(size_t(n_units), 0);
    freq_.assign(size_t(n_units), 0);
  }
}

int Residency::place(int unit, bool pin) {
  require(unit >= 0 && unit < n_, SS_E_INVALID, "resident set: unit out of range");
  if (slot_of_[size_t(unit)] >= 0) {
    if (pin) pin_[size_t(slot_of_[size_t(unit)])] = 1;
    return slot_of_[size_t(unit)];
  }
  const auto it = std::find(unit_in_.begin(), unit_in_.end(), -1);  // the lowest free slot
  if (it == unit_in_.end()) return -1;
  const int s = int(it - unit_in_.begin());
  *it = unit;
  pin_[size_t(s)] = pin;
  slot_of_[size_t(unit)] = s;
  return s;
}

void Residency::drop(int unit) {
  const int s = slot_of_[size_t(unit)];
  if (s < 0) return;
  unit_in_[size_t(s)] = -1;
  pin_[size_t(s)] = 0;
  slot_of_[size_t(unit)] = -1;
}

// 0.7 x transition from the previous route + 0.2 x window frequency + 0.1 x 1 / (1 + age).
double Residency::score(int unit) const {
  if (policy_ != SS_POLICY_SCORED) return 0.0;
  double tr = 0.0;
  if (!prev_.empty()) {
    for (int32_t p : prev_) {
      const uint32_t n = trans_n_[size_t(p)];
      if (n) tr += double(trans_[size_t(p) * size_t(n_) + size_t(unit)]) / double(n);
    }
    tr /= double(prev_.size());
  }
  const double fr = window_routes_.empty() ? 0.0 : double(freq_[size_t(unit)]) / double(window_routes_.size());
  const uint64_t lu = last_[size_t(unit)];
  const double age = lu ? double(tick_ - lu) : std::numeric_limits<double>::infinity();
  const double rec = std::isinf(age) ? 0.0 : 1.0 / (1.0 + age);
  return 0.7 * tr + 0.2 * fr + 0.1 * rec;
}

// The least recently used unpinned resident not kept this forward (ties: the lower unit id).
int Residency::lru_victim(const std::vector<char>& keep) const {
  int best = -1;
  for (size_t s = 0; s < unit_in_.size(); ++s) {
    const int32_t u = unit_in_[s];
    if (u < 0 || pin_[s] || keep[size_t(u)]) continue;
    if (best < 0) {
      best = int(s);
      continue;
    }
    const int32_t b = unit_in_[size_t(best)];
    if (last_[size_t(u)] < last_[size_t(b)] || (last_[size_t(u)] == last_[size_t(b)] && u < b)) best = int(s);
  }
  return best;
}

Admission Residency::admit(const std::vector<int32_t>& routed_in, const std::vector<char>& busy, bool admit_misses,
                           int max_evictions) {
  Admission a;
  std::vector<int32_t> routed = routed_in;
  std::sort(routed.begin(), routed.end());
  routed.erase(std::unique(routed.begin(), routed.end()), routed.end());
  std::vector<char> keep(size_t(n_), 0);
  std::vector<int32_t> misses;
  for (int32_t u : routed) {
    require(u >= 0 && u < n_, SS_E_INVALID, "routes: unit id out of range");
    keep[size_t(u)] = 1;
    (slot_of_[size_t(u)] >= 0 ? a.hits : misses).push_back(u);
  }
  for (size_t u = 0; u < busy.size() && u < keep.size(); ++u)
    if (busy[u]) keep[u] = 1;
  if (!admit_misses || unit_in_.empty()) {
    a.transient = misses;
    return a;
  }
  std::vector<int32_t> take;
  if (policy_ == SS_POLICY_LRU) {
    take = misses;
  } else {
    // scored cut: unpinned residents outside the route and the misses compete for the rows they can hold
    struct Row {
      int32_t unit;
      double s;
      uint64_t last;
      bool resident;
    };
    std::vector<Row> rows;
    size_t free_slots = 0;
    for (size_t s = 0; s < unit_in_.size(); ++s) {
      const int32_t u = unit_in_[s];
      if (u < 0) ++free_slots;
      else if (!pin_[s] && !keep[size_t(u)]) rows.push_back({u, score(u), last_[size_t(u)], true});
    }
    const size_t cut = free_slots + rows.size();
    for (int32_t u : misses) rows.push_back({u, score(u), last_[size_t(u)], false});
    std::sort(rows.begin(), rows.end(), [](const Row& x, const Row& y) {
      if (x.s != y.s) return x.s > y.s;
      if (x.last != y.last) return x.last > y.last;
      return x.unit < y.unit;
    });
    for (size_t i = 0; i < rows.size() && i < cut; ++i)
      if (!rows[i].resident) take.push_back(rows[i].unit);
    std::vector<char> below(size_t(n_), 0);
    for (size_t i = cut; i < rows.size(); ++i)
      if (rows[i].resident) below[size_t(rows[i].unit)] = 1;
    for (size_t u = 0; u < keep.size(); ++u)
      if (!below[u] && slot_of_[u] >= 0) keep[u] = 1;
  }
  std::vector<char> got(size_t(n_), 0);
  for (int32_t u : take) {
    const auto fr = std::find(unit_in_.begin(), unit_in_.end(), -1);
    int s = fr == unit_in_.end() ? -1 : int(fr - unit_in_.begin());
    if (s < 0) {
      if (max_evictions >= 0 && int(a.evicted.size()) >= max_evictions) {
        ++a.deferred;
        continue;
      }
      s = lru_victim(keep);
      if (s < 0) break;  // every resident is pinned or in use
      const int32_t old = unit_in_[size_t(s)];
      slot_of_[size_t(old)] = -1;
      a.evicted.push_back(old);
      a.evicted_slot.push_back(s);
    }
    unit_in_[size_t(s)] = u;
    pin_[size_t(s)] = 0;
    slot_of_[size_t(u)] = s;
    keep[size_t(u)] = 1;
    got[size_t(u)] = 1;
    a.admitted.push_back(u);
    a.admitted_slot.push_back(s);
  }
  for (int32_t u : misses)
    if (!got[size_t(u)]) a.transient.push_back(u);
  // ascending unit order for the admitted and evicted lists (slots move with their units)
  auto sort_pairs = [](std::vector<int32_t>& units, std::vector<int32_t>& slots) {
    std::vector<size_t> o(units.size());
    std::iota(o.begin(), o.end(), size_t(0));
    std::sort(o.begin(), o.end(), [&](size_t x, size_t y) { return units[x] < units[y]; });
    std::vector<int32_t> u2, s2;
    for (size_t i : o) {
      u2.push_back(units[i]);
      s2.push_back(slots[i]);
    }
    units.swap(u2);
    slots.swap(s2);
  };
  sort_pairs(a.admitted, a.admitted_slot);
  sort_pairs(a.evicted, a.evicted_slot);
  return a;
}

void Residency::observe(const std::vector<int32_t>& routed_in, const std::vector<int32_t>& misses) {
  std::vector<int32_t> routed = routed_in;
  std::sort(routed.begin(), routed.end());
  routed.erase(std::unique(routed.begin(), routed.end()), routed.end());
  ++tick_;
  if (policy_ == SS_POLICY_LRU) {
    for (int32_t u : routed) last_[size_t(u)] = tick_;
    return;
  }
  for (int32_t u : misses) last_[size_t(u)] = tick_;  // scored: a miss refreshes recency, a hit does not
  for (int32_t u : routed)
    if (last_[size_t(u)] == 0) last_[size_t(u)] = tick_;
  for (int32_t p : prev_) {
    ++trans_n_[size_t(p)];
    for (int32_t u : routed) ++trans_[size_t(p) * size_t(n_) + size_t(u)];
  }
  prev_ = routed;
  window_routes_.push_back(routed);
  for (int32_t u : routed) ++freq_[size_t(u)];
  if (window_routes_.size() > window_) {
    for (int32_t u : window_routes_.front()) --freq_[size_t(u)];
    window_routes_.pop_front();
  }
}

}  // namespace tsa
