// One layer's pool of persistent device slots in the host contract, and the admission decision a forward's routes
// make against it. The decision rules are the reference's (src/resident_set.cpp:86-217): misses take the lowest free
// slot, else evict the least recently used unpinned resident that is neither routed nor in flight (ties: the lower
// unit id), with an optional cap on evictions; SCORED ranks residents and misses by
// 0.7 x transition + 0.2 x window frequency + 0.1 x recency and admits the misses that rank inside the pool.
//
// Data structures: the free slots are an ordered set (lowest first), and the unpinned residents are an ordered index
// keyed by (last use, unit), so a victim is the first index entry not protected this forward instead of a scan of
// every slot. The SCORED history (transition counts, the window of recent routes) lives in ScoreBook.
#pragma once

#include <cstdint>
#include <set>
#include <utility>
#include <vector>

#include "strix_stream/ss.h"

namespace tsa {

struct Admission {
  std::vector<int32_t> hits;          // routed and resident, ascending
  std::vector<int32_t> admitted;      // misses given a slot, ascending
  std::vector<int32_t> admitted_slot; // (parallel to admitted)
  std::vector<int32_t> evicted;       // residents that lost their slot, ascending
  std::vector<int32_t> evicted_slot;  // (parallel to evicted)
  std::vector<int32_t> transient;     // misses left without a slot, ascending
  int deferred = 0;                   // misses refused a slot by the eviction cap
};

// SCORED policy history of one layer: how often unit v was routed one forward after unit p, and in how many of the
// last `window` forwards each unit was routed.
class ScoreBook {
 public:
  ScoreBook(int n_units, uint32_t window);
  void record(const std::vector<int32_t>& routed);  // one forward's distinct routed units, ascending
  // The transition and frequency terms of unit u against the last recorded forward.
  double transition(int32_t u) const;
  double frequency(int32_t u) const;

 private:
  int n_;
  uint32_t window_;
  std::vector<uint32_t> follow_;  // [p * n + v]: forwards that routed v right after a forward that routed p
  std::vector<uint32_t> led_;     // [p]: forwards that followed a forward routing p
  std::vector<uint32_t> hits_;    // [v]: forwards in the window that routed v
  std::vector<std::vector<int32_t>> ring_;  // the window's routes, oldest at head_
  size_t head_ = 0, filled_ = 0;
  std::vector<int32_t> last_;               // the last recorded forward's routes
};

class SlotPool {
 public:
  SlotPool(int n_units, int capacity, ss_policy policy, uint32_t window);
  int capacity() const { return int(holder_.size()); }
  int slot(int unit) const { return slot_of_[size_t(unit)]; }
  // Open and seeds: the lowest free slot for `unit` (-1 when none); an already resident unit keeps its slot (and is
  // pinned if asked). Pinned units are never victims.
  int place(int unit, bool pin);
  void drop(int unit);
  // routed: this forward's units (any order, repeats allowed); busy[u]: u is in flight this forward (never a victim);
  // admit_misses false or no slots: every miss is transient. max_evictions < 0: uncapped.
  Admission admit(const std::vector<int32_t>& routed, const std::vector<char>& busy, bool admit_misses,
                  int max_evictions = -1);
  // The forward's routed units and its misses (admitted or not) update recency and the SCORED history.
  void observe(const std::vector<int32_t>& routed, const std::vector<int32_t>& misses);

 private:
  void occupy(int32_t slot, int32_t unit, bool pin);
  void vacate(int32_t slot);
  void touch(int32_t unit, uint64_t when);  // last use of `unit` becomes `when` (re-keys its index entry)
  double score(int32_t unit) const;

  int n_;
  ss_policy policy_;
  std::vector<int32_t> slot_of_;  // unit -> slot, -1
  std::vector<int32_t> holder_;   // slot -> unit, -1
  std::vector<uint8_t> pinned_;   // per slot
  std::vector<uint64_t> used_;    // per unit: forward of its last use (0: never)
  std::set<int32_t> free_;
  std::set<std::pair<uint64_t, int32_t>> lru_;  // unpinned residents by (last use, unit)
  uint64_t clock_ = 0;
  std::vector<ScoreBook> book_;  // one under SCORED
};

}  // namespace tsa
