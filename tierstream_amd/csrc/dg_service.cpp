#include "dg_service.hpp"

#include <hip/hip_runtime_api.h>
#include <immintrin.h>

#include <algorithm>

#include "common.hpp"
#include "hip_rt.hpp"

namespace tsa {

// One wait on a mapped word. Between two polls the thread pauses; a wait that may be long (between tokens, before a
// step's begin kernel) turns to yielding the core once it has spun for kSpinFor. Every 64th poll the caller's slow
// checks run (stop, deadline, host abort), with the wall time the wait has taken.
class DgService::Poller {
 public:
  explicit Poller(bool may_yield) : t0_(Clock::now()), now_(t0_), may_yield_(may_yield) {}
  bool rest() {  // true: the slow checks are due
    if (yielding_) std::this_thread::yield();
    else _mm_pause();
    if ((++polls_ & 63u) != 0) return false;
    now_ = Clock::now();
    yielding_ = may_yield_ && now_ - t0_ > kSpinFor;
    return true;
  }
  Clock::duration waited() const { return now_ - t0_; }

 private:
  static constexpr std::chrono::microseconds kSpinFor{1000};
  Clock::time_point t0_, now_;
  uint32_t polls_ = 0;
  bool may_yield_, yielding_ = false;
};

namespace {
double us_between(DgService::Clock::time_point a, DgService::Clock::time_point b) {
  return double(std::chrono::duration_cast<std::chrono::nanoseconds>(b - a).count()) / 1e3;
}
std::string layer_name(uint32_t g) { return "gated layer " + std::to_string(g); }
}  // namespace

DgService::DgService(DgCore* core, const DgMappedHost& m, uint32_t max_ids, uint32_t timeout_ms, int device)
    : core_(core), m_(m), max_ids_(max_ids), timeout_(timeout_ms), device_(device), G_(core->gated()) {
  next_run_.assign(G_, 1);
  run_.assign(G_, 1);
  flag_seen_.assign(G_, 0);
  plan_.reserve(G_);
  pred_.reserve(kDgMaxIds);
}

void DgService::enable_timeline() {
  diag_ = true;
  rows_.assign(G_, Row{});
}

void DgService::start() {
  last_end_ = Clock::now();  // the first token's first seen_us counts from the start
  const uint32_t seen = opened_.load(std::memory_order_acquire);
  th_ = std::thread([this, seen] { thread_main(seen); });
}

void DgService::begin(uint32_t seq, const std::vector<uint8_t>& run) {
  std::copy(run.begin(), run.end(), next_run_.begin());
  opened_.store(seq, std::memory_order_release);  // (the run vector above is read after this is acquired)
}

DgService::Outcome DgService::wait_outcome(uint32_t seq, Clock::time_point deadline) const {
  for (uint32_t polls = 0;; ++polls) {
    if (served_.load(std::memory_order_acquire) == seq) return Outcome::kServed;
    const int h = halted_.load(std::memory_order_acquire);
    if (h) return Outcome(h);
    if ((polls & 255u) == 0 && Clock::now() > deadline) return Outcome::kPending;
    _mm_pause();
  }
}

void DgService::stop_join() {
  stop_.store(true, std::memory_order_release);
  if (m_.host_abort) store_release(m_.host_abort, 1);
  if (th_.joinable()) th_.join();
}

std::string DgService::error() const {
  std::lock_guard<std::mutex> lk(err_mu_);
  return err_;
}

// The thread ends with an outcome; a failure's message is kept (the first one) and the device's waits of the token
// end at once on host_abort.
void DgService::halt(Outcome o, const std::string& why) {
  if (o == Outcome::kFailed) {
    {
      std::lock_guard<std::mutex> lk(err_mu_);
      if (err_.empty()) err_ = why;
    }
    if (m_.host_abort) store_release(m_.host_abort, 1);
  }
  halted_.store(int(o), std::memory_order_release);
}

void DgService::thread_main(uint32_t last_seen) {
  try {
    hip_check(hipSetDevice(device_), "hipSetDevice (service)");
  } catch (const std::exception& e) {
    halt(Outcome::kFailed, e.what());
    return;
  }
  for (;;) {
    Poller idle(true);  // between tokens: the next one opens within microseconds of its ss_begin, or much later
    uint32_t seq = opened_.load(std::memory_order_acquire);
    while (seq == last_seen) {
      if (idle.rest() && stop_.load(std::memory_order_acquire)) return halt(Outcome::kStopped, "");
      seq = opened_.load(std::memory_order_acquire);
    }
    last_seen = seq;
    try {
      serve(seq);
    } catch (const Stop&) {
      return halt(Outcome::kStopped, "");
    } catch (const std::exception& e) {
      return halt(Outcome::kFailed, e.what());
    } catch (...) {
      return halt(Outcome::kFailed, "device-gated: the service thread failed");
    }
    served_.store(seq, std::memory_order_release);
  }
}

// A word of the mapped area reaches this token's sequence. With `last` (the export flags), any value but the one it
// held after its previous export is a step outside ss_begin / ss_end; without (the prediction flags), older values
// are simply not there yet.
void DgService::await_flag(const uint32_t* w, uint32_t seq, uint32_t g, const char* what, const uint32_t* last) {
  Poller p(false);
  for (;;) {
    const uint32_t v = load_acquire(w);
    if (v == seq) return;
    if (hooks_.while_waiting) hooks_.while_waiting();
    if (last && v != *last)
      fail(SS_E_BACKEND, "device-gated: sequence desync: the " + std::string(what) + " of " + layer_name(g) +
                             " reads " + std::to_string(v) + ", neither token " + std::to_string(seq) +
                             " nor the one it last exported (" + std::to_string(*last) + ")");
    if (!p.rest()) continue;
    if (stop_.load(std::memory_order_acquire)) throw Stop{};
    if (p.waited() > timeout_)
      fail(SS_E_BACKEND, "device-gated: the " + std::string(what) + " of " + layer_name(g) + " did not come within " +
                             std::to_string(timeout_.count()) + " ms (token " + std::to_string(seq) + ")");
  }
}

// The step's begin kernel. No deadline here: a legal step may capture and instantiate its graph between ss_begin and
// its launch, and a step that never launches is caught by ss_end's own deadline. A began word past this sequence is
// a step outside ss_begin / ss_end; stop and the host's abort end the wait.
void DgService::await_began(uint32_t seq) {
  Poller p(true);
  for (;;) {
    const uint32_t v = load_acquire(m_.began);
    if (v == seq) return;
    if (int32_t(v - seq) > 0)
      fail(SS_E_BACKEND, "device-gated: sequence desync: a step began as token " + std::to_string(v) +
                             " while token " + std::to_string(seq) + " is served (a step ran outside ss_begin / ss_end)");
    if (p.rest() && (stop_.load(std::memory_order_acquire) || load_acquire(m_.host_abort))) throw Stop{};
  }
}

DgService::Record DgService::read_record(uint32_t seq, uint32_t g) const {
  const DgRecord& r = m_.rec[g];
  require(r.seq == seq, SS_E_BACKEND,
          "device-gated: sequence desync: the export record of " + layer_name(g) + " carries token " +
              std::to_string(r.seq) + " while token " + std::to_string(seq) + " is served");
  require(r.n_ids >= 1 && r.n_ids <= max_ids_, SS_E_BACKEND,
          "device-gated: " + layer_name(g) + " exported " + std::to_string(r.n_ids) + " ids (1 to " +
              std::to_string(max_ids_) + " allowed)");
  require(r.n_pred_promised <= kDgMaxIds && (r.n_pred_promised == 0 || g + 1 < G_), SS_E_BACKEND,
          "device-gated: " + layer_name(g) + " promised " + std::to_string(r.n_pred_promised) +
              " predicted ids" + (g + 1 < G_ ? "" : " as the last gated layer"));
  Record rec;
  rec.ids.assign(r.ids, r.ids + r.n_ids);
  rec.dev_mask = uint64_t(r.mask_lo) | uint64_t(r.mask_hi) << 32;
  rec.n_pred = r.n_pred_promised;
  return rec;
}

void DgService::serve(uint32_t seq) {
  run_ = next_run_;
  plan_.clear();
  for (uint32_t g = 0; g < G_; ++g)
    if (run_[g]) plan_.push_back(g);
  if (diag_) std::fill(rows_.begin(), rows_.end(), Row{});  // a failed token leaves the rows of the layers it reached
  core_->open_token(seq, &run_);
  await_began(seq);  // every flag's deadline starts once the step has begun
  for (size_t i = 0; i < plan_.size(); ++i) serve_layer(seq, plan_[i], i + 1 < plan_.size() ? plan_[i + 1] : G_);
  if (hooks_.before_served) hooks_.before_served();
  last_end_ = Clock::now();
}

// One exported gated layer; `next` is the next exported one (G_: none).
void DgService::serve_layer(uint32_t seq, uint32_t g, uint32_t next) {
  await_flag(&m_.flag[g], seq, g, "export flag", &flag_seen_[g]);
  flag_seen_[g] = seq;
  const Clock::time_point t_seen = Clock::now();
  const DgCounts before = diag_ ? core_->counts() : DgCounts{};
  const Record r = read_record(seq, g);
  const uint32_t n = uint32_t(r.ids.size());
  // the canonical schedule's mask: the host mirror's absent entries now, after the previous layer's prediction was
  // served (a prefetch that had not landed when the layer exported is a hit there, as in an eager schedule); the
  // device mask may only add such bits
  const uint64_t mask = core_->absent_mask(g, r.ids.data(), n);
  require((mask & ~r.dev_mask) == 0, SS_E_BACKEND,
          "device-gated: " + layer_name(g) + " exported a hit for a unit absent from the table");
  core_->serve_misses(g, r.ids.data(), n, mask, r.dev_mask);
  const Clock::time_point t_demand = Clock::now();
  core_->note_uses(g, r.ids.data(), n, mask);
  Row row;
  row.seen_us = us_between(last_end_, t_seen);
  row.demand_us = us_between(t_seen, t_demand);
  if (r.n_pred > 0 && next == g + 1) {  // a prediction for a layer the token does not export is ignored
    await_flag(&m_.pflag[g], seq, g, "prediction flag", nullptr);
    const Clock::time_point t_pred = Clock::now();
    const DgPredRecord& pr = m_.prec[g];
    require(pr.n_pred == r.n_pred, SS_E_BACKEND,
            "device-gated: the prediction record of " + layer_name(g) + " holds " + std::to_string(pr.n_pred) +
                " ids, its export promised " + std::to_string(r.n_pred));
    pred_.assign(pr.pred, pr.pred + r.n_pred);
    core_->prefetch_next(g + 1, pred_.data(), r.n_pred);
    row.pred_wait_us = us_between(t_demand, t_pred);
    row.prefetch_us = us_between(t_pred, Clock::now());
  }
  if (next < G_ && core_->queued_writebacks()) core_->spend_wb_credit(g);
  const Clock::time_point t_end = Clock::now();
  row.serve_us = us_between(t_seen, t_end);
  last_end_ = t_end;
  if (!diag_) return;
  const DgCounts& a = core_->counts();
  row.ids = uint32_t(a.lookups - before.lookups);  // one lookup per distinct id
  row.misses = uint32_t(a.misses - before.misses);
  row.covered = uint32_t(a.covered - before.covered);
  row.fetched = uint32_t(a.fetched - before.fetched);
  row.prefetched = uint32_t(a.prefetched - before.prefetched);
  row.predicted_true = uint32_t(a.predicted_true - before.predicted_true);
  row.covered_waits = uint32_t(a.covered_waits - before.covered_waits);
  rows_[g] = row;
}

}  // namespace tsa
