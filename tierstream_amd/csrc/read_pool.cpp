#include "read_pool.hpp"

#include <algorithm>
#include <string>

#include "common.hpp"

namespace tsa {

ReadPool::ReadPool(uint32_t threads, uint32_t words, std::vector<Piece> pieces, LandingRule landing,
                   PieceReader read, Finisher finish)
    : pieces_(std::move(pieces)), land_(std::move(landing)), read_(std::move(read)), finish_(std::move(finish)),
      threads_(std::max<uint32_t>(threads, 1)), limit_(std::max<uint32_t>(threads, 1)) {
  for (const Piece& p : pieces_) unit_bytes_ += p.bytes;
  land_.cap = std::max<uint32_t>(land_.cap, 1);
  at_.resize(words);
  failed_.assign(words, 0);
  for (uint32_t i = 0; i < threads_; ++i) th_.emplace_back([this] { run(); });
}

void ReadPool::adapt() {
  std::lock_guard<std::mutex> l(m_);
  ctl_ = std::make_unique<ReadDepthController>(threads_);
  limit_ = ctl_->depth();
}

void ReadPool::with_controller(const std::function<void(const ReadDepthController&)>& f) {
  std::lock_guard<std::mutex> l(m_);
  if (ctl_) f(*ctl_);
}

void ReadPool::stop() {
  {
    std::lock_guard<std::mutex> l(m_);
    for (size_t w = 0; w < at_.size(); ++w)  // (a landing read nobody claimed is never copied out)
      if (at_[w] && at_[w]->landing && !at_[w]->dropped) drop_locked(*at_[w]);
    stop_ = true;
  }
  cv_.notify_all();
  for (auto& t : th_)
    if (t.joinable()) t.join();
}

void ReadPool::enqueue(uint32_t w, uint32_t key, char* dst, uint32_t* word, uint32_t gen, bool landing) {
  {
    std::unique_lock<std::mutex> l(m_);
    require(w < at_.size(), SS_E_BACKEND, "device-gated: a read of word " + std::to_string(w) + " out of range");
    require(!landing || !land_.pieces.empty(), SS_E_BACKEND, "device-gated: a landing read with landings off");
    require(!stop_, SS_E_BACKEND, "device-gated: a read after the readers stopped");
    word_cv_.wait(l, [&] { return !at_[w]; });  // the word's previous read first
    auto u = std::make_unique<Unit>();
    u->w = w;
    u->key = key;
    u->gen = gen;
    u->dst = dst;
    u->word = word;
    u->landing = landing;
    const std::vector<Piece>& ps = landing ? land_.pieces : pieces_;
    u->left = uint32_t(ps.size());
    for (const Piece& p : ps) (landing ? lq_ : q_).push_back(Job{u.get(), &p});
    failed_[w] = 0;
    if (!landing) ++demand_inflight_;
    at_[w] = std::move(u);
  }
  cv_.notify_all();
}

bool ReadPool::landing_ready() const {
  if (!q_.empty() || lq_.empty() || running_ >= limit_) return false;
  if (!land_.reserve) return running_ < land_.cap;
  return landing_running_ < land_.cap && landing_running_ + 1 < std::max<uint32_t>(threads_, 2);
}

void ReadPool::set_partway(Unit* u, bool on) {
  const auto it = std::find(partway_.begin(), partway_.end(), u);
  if (on && it == partway_.end()) partway_.push_back(u);
  if (!on && it != partway_.end()) partway_.erase(it);
}

uint64_t ReadPool::take_landing_pieces(Unit* u, std::deque<Job>* to) {
  uint64_t bytes = 0;
  for (auto it = lq_.begin(); it != lq_.end();) {
    if (it->unit != u) {
      ++it;
      continue;
    }
    bytes += it->piece->bytes;
    if (to) to->push_back(*it);
    else --u->left;
    it = lq_.erase(it);
  }
  return bytes;
}

void ReadPool::run() {
  for (;;) {
    Job j{};
    bool from_landing = false;
    {
      std::unique_lock<std::mutex> l(m_);
      cv_.wait(l, [this] { return demand_ready() || landing_ready() || (stop_ && q_.empty() && lq_.empty()); });
      if (demand_ready()) {
        j = q_.front();
        q_.pop_front();
      } else if (landing_ready()) {
        j = lq_.front();
        lq_.pop_front();
        from_landing = true;
        ++landing_running_;
      } else {
        return;  // stopping, nothing queued
      }
      max_running_ = std::max<uint64_t>(max_running_, ++running_);
      Unit& u = *j.unit;
      ++u.running;
      u.started = true;
      if (u.landing) set_partway(&u, u.left > u.running);
      if (ctl_ && !busy_) {  // a busy period begins
        busy_ = true;
        busy_t0_ = Clock::now();
        busy_units_ = 0;
      }
    }
    Unit& u = *j.unit;
    std::exception_ptr e;
    const auto t0 = Clock::now();
    try {
      read_(u.key, j.piece->part, j.piece->off, j.piece->bytes, u.dst + j.piece->dst_off);
    } catch (...) {
      e = std::current_exception();
    }
    read_ns_.fetch_add(uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0).count()),
                       std::memory_order_relaxed);
    bool check = false;
    {
      std::lock_guard<std::mutex> l(m_);
      --running_;
      if (from_landing) --landing_running_;
      --u.running;
      if (e) {
        u.failed = true;
        if (!u.err) u.err = e;
      }
      const bool last = --u.left == 0;
      // a landing read part-way yields this reader when more demand pieces wait than the other readers idle could
      // take (reference src/dg_load.cpp:746-750, per piece here): the reader takes a demand piece next
      if (from_landing && u.landing && !u.dropped && !e && u.left > u.running && q_.size() + running_ + 1 > threads_)
        ++lc_.yields;
      if (ctl_ && busy_) {
        busy_units_ += last;
        if (running_ == 0 && q_.empty() && lq_.empty()) {  // idle again: the period's throughput picks the depth
          busy_ = false;
          const uint64_t ns =
              uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - busy_t0_).count());
          limit_ = std::min(std::max<uint32_t>(ctl_->feed(busy_units_, busy_units_ * unit_bytes_, ns), 1), threads_);
        }
      }
      cv_.notify_all();  // (a piece slot is free: a queued piece, or a landing piece under its cap)
      if (!last) continue;
      u.finishing = true;
      check = !u.failed && !u.dropped;
    }
    std::exception_ptr fe;
    if (check) {  // every piece landed: the finisher, then the word
      try {
        finish_(u.key, u.dst);
      } catch (...) {
        fe = std::current_exception();
      }
    }
    std::lock_guard<std::mutex> l(m_);
    if (fe) {
      u.failed = true;
      if (!u.err) u.err = fe;
    }
    finish_locked(u);
  }
}

void ReadPool::finish_locked(Unit& u) {
  const uint32_t w = u.w;
  if (u.failed && !u.dropped) {
    if (u.landing) {  // kept: a claim finds it failed
      ++lc_.failed;
      lc_.unread_bytes += unit_bytes_;
      failed_[w] = 1;
    } else if (!err_) {
      err_ = u.err;
    }
  }
  __atomic_store_n(u.word, u.gen, __ATOMIC_RELEASE);  // the buffer's bytes (or the failure) before the word
  if (!u.landing && --demand_inflight_ == 0) idle_.notify_all();
  set_partway(&u, false);
  at_[w].reset();
  word_cv_.notify_all();
}

ReadPool::Claim ReadPool::claim(uint32_t w) {
  std::lock_guard<std::mutex> l(m_);
  require(w < at_.size(), SS_E_BACKEND, "device-gated: a claim of word " + std::to_string(w) + " out of range");
  Unit* u = at_[w].get();
  if (!u) return failed_[w] ? Claim::Failed : Claim::Landed;
  require(u->landing && !u->dropped, SS_E_BACKEND,
          "device-gated: a claim of word " + std::to_string(w) + " that holds no landing read");
  u->landing = false;  // a demand read from now on: its queued pieces behind the demand pieces queued
  ++demand_inflight_;
  take_landing_pieces(u, &q_);
  set_partway(u, false);
  ++lc_.late;
  cv_.notify_all();
  return Claim::Late;
}

void ReadPool::drop_locked(Unit& u) {
  u.dropped = true;
  const uint64_t unread = take_landing_pieces(&u, nullptr);
  lc_.unread_bytes += unread;
  if (!u.started) ++lc_.cancelled;
  else lc_.aborted_bytes += unread;
  set_partway(&u, false);
  if (u.left == 0 && !u.finishing) finish_locked(u);  // (nothing runs: done now)
}

void ReadPool::drop(uint32_t w) {
  std::lock_guard<std::mutex> l(m_);
  require(w < at_.size(), SS_E_BACKEND, "device-gated: a drop of word " + std::to_string(w) + " out of range");
  Unit* u = at_[w].get();
  if (!u || !u->landing || u->dropped) return;
  drop_locked(*u);
  cv_.notify_all();
}

uint64_t ReadPool::wait_idle(uint32_t w) {
  std::unique_lock<std::mutex> l(m_);
  if (w >= at_.size() || !at_[w]) return 0;
  const auto t0 = Clock::now();
  word_cv_.wait(l, [&] { return !at_[w]; });
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0).count());
}

uint64_t ReadPool::drain() {
  std::unique_lock<std::mutex> l(m_);
  uint64_t ns = 0;
  if (demand_inflight_) {
    const auto t0 = Clock::now();
    idle_.wait(l, [this] { return demand_inflight_ == 0; });
    ns = uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0).count());
  }
  if (err_) {
    std::exception_ptr e = err_;
    err_ = nullptr;
    std::rethrow_exception(e);
  }
  return ns;
}

uint64_t ReadPool::max_running() {
  std::lock_guard<std::mutex> l(m_);
  return max_running_;
}

ReadPool::LandingCounts ReadPool::landing_counts() {
  std::lock_guard<std::mutex> l(m_);
  return lc_;
}

ReadPool::Load ReadPool::load() {
  std::lock_guard<std::mutex> l(m_);
  return Load{running_, landing_running_, q_.size(), lq_.size()};
}

}  // namespace tsa
