// The host contract's reader threads: which queued file read a free reader starts, and how an unaligned byte range is
// covered by aligned reads.
//
// ReadScheduler keeps the reads waiting for a reader in three classes, served in priority order:
//   kDemand  reads an engine call needs now: a routed miss, a promoted guess, a read-ahead a landing waits for;
//   kAhead   read-ahead reads into host buffers, started only while fewer than max(1, readers - 1) of them run, so
//            one reader is always left for demands (once the context stops, they drain on any reader);
//   kGuess   speculative reads, started only while at most one demand read runs.
// Inside a class, reads start in arrival order; raise() moves a queued read to the head of kDemand. The object has no
// lock of its own: it lives under the context's queue mutex (every call is made with it held; wait_next takes the
// caller's lock on it), because a read's queue position and its state change together.
//
// Covering reads: with O_DIRECT a read's offset, length and buffer must be aligned. A byte range [off, off + n) is
// covered by windows of at most `cap` bytes: window k reads the aligned span [a0, a0 + span) into a bounce buffer, in
// which its piece of the range starts at `lead`. The reference reads the same way (src/stream_ctx.cpp:584-620).
#pragma once

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <mutex>

namespace tsa {

enum class ReadClass : uint8_t { kDemand = 0, kAhead = 1, kGuess = 2 };

template <class T>
class ReadScheduler {
 public:
  void set_readers(int readers) { ahead_cap_ = readers > 2 ? readers - 1 : 1; }

  void push(ReadClass c, T item) {
    q_[int(c)].push_back(std::move(item));
    cv_.notify_all();
  }
  // A queued read leaves its class (false: it was not queued there).
  bool remove(ReadClass c, const T& item) {
    std::deque<T>& d = q_[int(c)];
    const auto it = std::find(d.begin(), d.end(), item);
    if (it == d.end()) return false;
    d.erase(it);
    return true;
  }
  // A read queued in `from` is needed now: it goes to the head of kDemand (false: it was not queued in `from`).
  bool raise(ReadClass from, const T& item) {
    if (!remove(from, item)) return false;
    q_[int(ReadClass::kDemand)].push_front(item);
    cv_.notify_all();
    return true;
  }
  // Blocks on lk (the queue mutex) until this reader may start a read, takes it and counts it running; false when the
  // scheduler is stopped and nothing is left to read.
  bool wait_next(std::unique_lock<std::mutex>& lk, T* out, ReadClass* cls) {
    cv_.wait(lk, [&] { return pick() >= 0 || (stop_ && idle()); });
    return try_next(out, cls);
  }
  // The read a reader may start now, if any (taken and counted running).
  bool try_next(T* out, ReadClass* cls) {
    const int c = pick();
    if (c < 0) return false;
    *out = std::move(q_[c].front());
    q_[c].pop_front();
    ++running_[c];
    *cls = ReadClass(c);
    return true;
  }
  void ended(ReadClass c) {  // a read that wait_next started is over (read, failed, or cancelled before it began)
    --running_[int(c)];
    cv_.notify_all();
  }
  void hold(bool h) {  // test hook: readers start nothing while held (a stop overrides it)
    hold_ = h;
    cv_.notify_all();
  }
  void stop() {
    stop_ = true;
    cv_.notify_all();
  }
  void wake() { cv_.notify_all(); }

 private:
  bool idle() const { return q_[0].empty() && q_[1].empty() && q_[2].empty(); }
  bool may_start(int c) const {
    switch (ReadClass(c)) {
      case ReadClass::kAhead: return running_[c] < ahead_cap_ || stop_;
      case ReadClass::kGuess: return running_[int(ReadClass::kDemand)] <= 1;
      default: return true;
    }
  }
  int pick() const {
    if (hold_ && !stop_) return -1;
    for (int c = 0; c < 3; ++c)
      if (!q_[c].empty() && may_start(c)) return c;
    return -1;
  }

  std::deque<T> q_[3];
  int running_[3] = {0, 0, 0};
  int ahead_cap_ = 1;
  bool hold_ = false, stop_ = false;
  std::condition_variable cv_;
};

// One aligned window of a covering read.
struct CoverWindow {
  uint64_t at;    // where the window's piece starts in the range
  uint64_t len;   // the piece's bytes
  uint64_t a0;    // the aligned file offset the window reads from
  uint64_t span;  // the aligned bytes it reads
  uint64_t lead;  // where the piece starts in the window
};

// Calls fn(window) for the windows covering [off, off + n) with reads aligned to al, each window at most cap bytes of
// the range (cap a multiple of al, and the window's span at most cap + 2 al).
template <class F>
void for_each_cover_window(uint64_t off, uint64_t n, uint64_t al, uint64_t cap, F&& fn) {
  for (uint64_t at = 0; at < n;) {
    CoverWindow w;
    w.at = at;
    w.len = std::min(cap, n - at);
    w.a0 = (off + at) / al * al;
    w.lead = off + at - w.a0;
    w.span = (off + at + w.len + al - 1) / al * al - w.a0;
    fn(w);
    at += w.len;
  }
}

}  // namespace tsa
