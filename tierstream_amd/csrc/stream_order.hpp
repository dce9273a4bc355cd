// Cross-stream waits without the redundant ones.
//
// Work on one HIP stream completes in the order it was given, so an event recorded on stream X stands for everything X
// was given before the record, X's own earlier waits included. A stream that already waits for X's k-th record (its
// k-th "mark") follows every earlier mark of X too: a later wait for one of those is redundant and is not issued. A
// wait for an event recorded on the waiting stream itself is redundant as well.
//
// Why it matters on MI355X: each hipStreamWaitEvent on a copy stream leaves a barrier packet on the stream's queue
// that the stream's next copy starts behind, and that packet is processed late. On the host contract's Qwen3-shape
// step (2 copy streams, about 2 waits per 9 MiB copy), copies started a median 193 us (p90 700 us) after the work they
// waited for had ended; about 87 % of those waits were implied by an earlier wait of the same stream.
//
// MarkOrder is the bookkeeping alone, over any handle types; StreamOrder issues the HIP calls under one lock, so a
// wait skipped on a stream always relies on a wait that was already given to that stream.
#pragma once

#include <cstdint>
#include <mutex>
#include <unordered_map>
#include <utility>

#include "hip_rt.hpp"

namespace tsa {

template <class S, class E>
class MarkOrder {
 public:
  // e was just recorded on s: it now stands for s's next mark.
  void recorded(E e, S s) {
    const uint64_t i = id(s);
    last_[e] = {i, ++marks_[i]};
  }
  // Whether s must be given a wait for e. An event never recorded here is left to the runtime (true).
  bool needs_wait(S s, E e) const {
    const auto it = last_.find(e);
    if (it == last_.end()) return true;
    const auto own = ids_.find(s);
    if (own == ids_.end()) return true;
    if (it->second.first == own->second) return false;
    const auto w = seen_.find(own->second);
    if (w == seen_.end()) return true;
    const auto k = w->second.find(it->second.first);
    return k == w->second.end() || k->second < it->second.second;
  }
  // s was given a wait for e: it follows e's mark from now on.
  void waited(S s, E e) {
    const auto it = last_.find(e);
    const uint64_t i = id(s);
    if (it == last_.end() || it->second.first == i) return;
    uint64_t& k = seen_[i][it->second.first];
    if (k < it->second.second) k = it->second.second;
  }
  // From now on s names a stream that follows nothing and whose marks are unrelated to the earlier ones (a stream
  // handle that may name a different stream next, such as the engine's stream of a new forward).
  void forget(S s) {
    const auto it = ids_.find(s);
    if (it == ids_.end()) return;
    const uint64_t old = it->second;
    seen_.erase(old);
    for (auto& w : seen_) w.second.erase(old);  // (waits for its events are given again from now on)
    marks_.erase(old);
    ids_.erase(it);
  }

 private:
  uint64_t id(S s) {
    const auto it = ids_.find(s);
    if (it != ids_.end()) return it->second;
    return ids_[s] = next_id_++;
  }
  uint64_t next_id_ = 1;
  std::unordered_map<S, uint64_t> ids_;                                  // each handle's current stream
  std::unordered_map<uint64_t, uint64_t> marks_;                         // marks recorded per stream
  std::unordered_map<E, std::pair<uint64_t, uint64_t>> last_;            // each event's latest record: stream, mark
  std::unordered_map<uint64_t, std::unordered_map<uint64_t, uint64_t>> seen_;  // per waiting stream: per stream, the
                                                                               // mark waited for
};

class StreamOrder {
 public:
  void record(hipEvent_t e, hipStream_t s) {
    std::lock_guard<std::mutex> lk(mu_);
    ev_record(e, s);
    m_.recorded(e, s);
  }
  void wait(hipStream_t s, hipEvent_t e) {
    if (!e) return;
    std::lock_guard<std::mutex> lk(mu_);
    if (!m_.needs_wait(s, e)) {
      ++skipped_;
      return;
    }
    stream_wait(s, e);
    m_.waited(s, e);
    ++issued_;
  }
  void forget(hipStream_t s) {
    std::lock_guard<std::mutex> lk(mu_);
    m_.forget(s);
  }
  void counts(uint64_t* issued, uint64_t* skipped) {
    std::lock_guard<std::mutex> lk(mu_);
    *issued = issued_;
    *skipped = skipped_;
  }

 private:
  std::mutex mu_;
  MarkOrder<hipStream_t, hipEvent_t> m_;
  uint64_t issued_ = 0, skipped_ = 0;
};

}  // namespace tsa
