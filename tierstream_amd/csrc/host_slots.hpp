// The host contract's shared slot resources, kept apart from the placement decisions that use them.
//
//  * RingPool: the stream ring's device slots, in classes of one unit stride. Each class hands its free slots out
//    round robin: the first free position at or after the class's cursor, wrapping, after which the cursor points past
//    the slot handed out. Free positions live in an ordered set per class, so a grant is one ordered lookup. A slot
//    remembers which layer released it last: a copy into it must wait for that layer's release on the device.
//  * WaitLine: transient units that found no ring slot, ordered by layer and, inside a layer, by arrival. Slots that
//    come free go to the head of the line only, so a later layer never overtakes an earlier layer's waiting unit.
//  * SpareBlocks: exclusive mode's free pinned blocks of each block class, a stack whose top at open is the class's
//    lowest block (a block given back goes on top).
#pragma once

#include <algorithm>
#include <cstdint>
#include <deque>
#include <set>
#include <utility>
#include <vector>

namespace tsa {

class RingPool {
 public:
  struct Class {
    uint64_t stride;
    uint32_t first, count;  // global slots first .. first + count - 1
  };
  struct Grant {
    int32_t slot = -1;         // global ring slot
    int32_t prev_reader = -1;  // the layer that released it last (-1: never used)
  };

  void add_class(uint64_t stride, uint32_t count) {
    const uint32_t first = uint32_t(slot_.size());
    cls_.push_back(Class{stride, first, count});
    cursor_.push_back(0);
    std::set<uint32_t> all;
    for (uint32_t i = 0; i < count; ++i) all.insert(all.end(), i);
    free_.push_back(std::move(all));
    slot_.resize(slot_.size() + count);
  }
  const std::vector<Class>& classes() const { return cls_; }
  uint32_t size() const { return uint32_t(slot_.size()); }
  int class_for(uint64_t stride) const {
    for (size_t c = 0; c < cls_.size(); ++c)
      if (cls_[c].stride == stride) return int(c);
    return -1;
  }
  bool has_free(int cls) const { return cls >= 0 && !free_[size_t(cls)].empty(); }

  // The class's next free slot in round-robin order, now held by `layer` for `job` (the class must have one free).
  Grant grant(int cls, int32_t layer, int32_t job) {
    std::set<uint32_t>& f = free_[size_t(cls)];
    auto it = f.lower_bound(cursor_[size_t(cls)]);
    if (it == f.end()) it = f.begin();
    const uint32_t pos = *it;
    f.erase(it);
    const Class& c = cls_[size_t(cls)];
    cursor_[size_t(cls)] = (pos + 1) % c.count;
    const uint32_t g = c.first + pos;
    Slot& s = slot_[g];
    s.owner = layer;
    s.job = job;
    if (size_t(layer) >= held_.size()) held_.resize(size_t(layer) + 1);
    held_[size_t(layer)].push_back(g);
    return Grant{int32_t(g), s.prev_reader};
  }

  // Every slot `layer` holds comes free, in slot order; retire(job) runs for each before it is handed out again.
  template <class F>
  void release(int32_t layer, F&& retire) {
    if (size_t(layer) >= held_.size()) return;
    std::vector<int32_t> mine;
    mine.swap(held_[size_t(layer)]);
    std::sort(mine.begin(), mine.end());
    for (int32_t g : mine) {
      Slot& s = slot_[size_t(g)];
      if (s.owner != layer) continue;
      retire(s.job);
      s.prev_reader = layer;
      vacate(g);
    }
  }

  // End of a forward: every slot still held comes free as it is (its last reader stays what it was).
  void reset_holders() {
    for (std::vector<int32_t>& h : held_) {
      for (int32_t g : h)
        if (slot_[size_t(g)].owner >= 0) vacate(g);
      h.clear();
    }
  }

 private:
  struct Slot {
    int32_t owner = -1, job = -1, prev_reader = -1;
  };
  void vacate(int32_t g) {
    Slot& s = slot_[size_t(g)];
    s.owner = s.job = -1;
    for (size_t c = 0; c < cls_.size(); ++c)
      if (uint32_t(g) >= cls_[c].first && uint32_t(g) < cls_[c].first + cls_[c].count) {
        free_[c].insert(uint32_t(g) - cls_[c].first);
        return;
      }
  }

  std::vector<Class> cls_;
  std::vector<uint32_t> cursor_;
  std::vector<std::set<uint32_t>> free_;
  std::vector<Slot> slot_;
  std::vector<std::vector<int32_t>> held_;  // by layer: the global slots it holds this forward
};

class WaitLine {
 public:
  void join(int32_t layer, int32_t unit) {
    const auto at = std::upper_bound(q_.begin(), q_.end(), layer,
                                     [](int32_t l, const std::pair<int32_t, int32_t>& w) { return l < w.first; });
    q_.insert(at, {layer, unit});
    if (size_t(layer) >= count_.size()) count_.resize(size_t(layer) + 1, 0);
    ++count_[size_t(layer)];
  }
  uint32_t waiting(int32_t layer) const { return size_t(layer) < count_.size() ? count_[size_t(layer)] : 0; }
  // place(layer, unit) -> true when the unit got its slot; the line moves until the first unit that did not.
  template <class F>
  void serve(F&& place) {
    while (!q_.empty() && place(q_.front().first, q_.front().second)) {
      --count_[size_t(q_.front().first)];
      q_.pop_front();
    }
  }
  void clear() {
    q_.clear();
    std::fill(count_.begin(), count_.end(), 0u);
  }

 private:
  std::deque<std::pair<int32_t, int32_t>> q_;
  std::vector<uint32_t> count_;
};

class SpareBlocks {
 public:
  // Blocks first .. first + n - 1 join a new class; the lowest is handed out first.
  void add_class(int32_t first, uint32_t n) {
    std::vector<int32_t> st;
    st.reserve(n);
    for (uint32_t i = n; i-- > 0;) st.push_back(first + int32_t(i));
    stack_.push_back(std::move(st));
    spares_.push_back(n);
  }
  size_t classes() const { return stack_.size(); }
  uint64_t free(int cls) const { return stack_[size_t(cls)].size(); }
  uint32_t spares(int cls) const { return spares_[size_t(cls)]; }
  uint64_t total_free() const {
    uint64_t n = 0;
    for (const auto& s : stack_) n += s.size();
    return n;
  }
  int32_t take(int cls) {
    std::vector<int32_t>& s = stack_[size_t(cls)];
    const int32_t b = s.back();
    s.pop_back();
    return b;
  }
  void give(int cls, int32_t b) { stack_[size_t(cls)].push_back(b); }
  const std::vector<int32_t>& free_list(int cls) const { return stack_[size_t(cls)]; }

 private:
  std::vector<std::vector<int32_t>> stack_;
  std::vector<uint32_t> spares_;
};

}  // namespace tsa
