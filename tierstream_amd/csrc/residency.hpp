// Per-layer residency of the host contract: which units hold a persistent device slot of the layer's pool, and the
// deterministic admission decision of a forward (every tie to the lower unit id). The rules are those of reference
// src/resident_set.cpp:86-217 (LRU and SCORED admission, observe); this is the library's own implementation.
#pragma once

#include <cstdint>
#include <deque>
#include <vector>

#include "strix_stream/ss.h"

namespace tsa {

struct Admission {
  std::vector<int32_t> hits;          // routed and resident (ascending)
  std::vector<int32_t> admitted;      // misses that take a slot (ascending)
  std::vector<int32_t> admitted_slot;
  std::vector<int32_t> evicted;       // units that lost their slot (ascending)
  std::vector<int32_t> evicted_slot;
  std::vector<int32_t> transient;     // misses served from the stream ring (ascending)
  int deferred = 0;                   // misses past the eviction cap
};

class Residency {
 public:
  Residency(int n_units, int capacity, ss_policy policy, uint32_t window);
  int capacity() const { return int(unit_in_.size()); }
  int slot(int unit) const { return slot_of_[size_t(unit)]; }
  int place(int unit, bool pin);  // a free slot at open / seed (-1 when full)
  void drop(int unit);
  Admission admit(const std::vector<int32_t>& routed, const std::vector<char>& busy, bool admit_misses,
                  int max_evictions = -1);
  void observe(const std::vector<int32_t>& routed, const std::vector<int32_t>& misses);

 private:
  int lru_victim(const std::vector<char>& keep) const;
  double score(int unit) const;

  int n_;
  ss_policy policy_;
  uint32_t window_;
  std::vector<int32_t> slot_of_, unit_in_;
  std::vector<char> pin_;
  std::vector<uint64_t> last_;
  uint64_t tick_ = 0;
  // SCORED
  std::vector<uint32_t> trans_, trans_n_, freq_;
  std::vector<int32_t> prev_;
  std::deque<std::vector<int32_t>> window_routes_;
};

}  // namespace tsa
