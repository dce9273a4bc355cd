#include "depth_ctl.hpp"

#include <algorithm>

namespace tsa {

ReadDepthController::ReadDepthController(uint32_t bound, const Tuning& t) : t_(t), u_(std::max<uint32_t>(bound, 1)) {
  t_.window_reads = std::max<uint64_t>(t_.window_reads, 1);
  depth_ = u_;
  next_backoff_ = t_.first_backoff;
  calibrate(Why::Start);
}

void ReadDepthController::go(uint32_t d) {
  changes += d != depth_;
  depth_ = d;
}

void ReadDepthController::calibrate(Why) {
  stage_ = Stage::U0;
  ++calibrations;
  go(u_);
  win_ = Window{};
}

void ReadDepthController::remember(const Verdict& v) {
  if (recent_.size() == kRecent) recent_.pop_front();
  recent_.push_back(v);
}

// The four windows are in: U before / 1, U after / 1 (each bracket compares neighbours in time).
void ReadDepthController::conclude() {
  const double bar = 1.0 + t_.margin;
  const bool before = rate_[0] >= bar * rate_[1], after = rate_[3] >= bar * rate_[2];
  Verdict v;
  v.seq = ++verdicts_;
  v.reads = all_reads_;
  v.from = depth_;
  v.gbps_u = (rate_[0] + rate_[3]) / 2;
  v.gbps_1 = (rate_[1] + rate_[2]) / 2;
  if (before != after && !repeating_) {  // the rate moved inside the calibration: measure once more
    repeating_ = true;
    v.to = u_;
    v.why = Why::Split;
    remember(v);
    calibrate(Why::Split);
    --calibrations;  // (the same calibration)
    return;
  }
  repeating_ = false;
  const bool keep_u = before && after;
  v.to = keep_u ? u_ : 1;
  v.why = keep_u ? Why::KeepU : Why::Keep1;
  remember(v);
  stage_ = Stage::Held;
  far_in_a_row_ = 0;
  held_reads_ = 0;
  held_rate_ = keep_u ? v.gbps_u : v.gbps_1;
  if (keep_u) {  // U won: the back-off starts over
    hold_for_ = t_.recheck_at_u;
    next_backoff_ = t_.first_backoff;
  } else {
    hold_for_ = next_backoff_;
    next_backoff_ = t_.later_backoff;
  }
  go(keep_u ? u_ : 1);
}

uint32_t ReadDepthController::feed(uint64_t reads, uint64_t bytes, uint64_t ns) {
  if (u_ == 1 || reads == 0) return depth_;
  all_reads_ += reads;
  (depth_ == 1 ? reads_1 : reads_u) += reads;
  (depth_ == 1 ? bytes_1 : bytes_u) += bytes;
  (depth_ == 1 ? ns_1 : ns_u) += ns;
  win_.reads += reads;
  win_.bytes += bytes;
  win_.ns += ns;
  if (stage_ == Stage::Held) held_reads_ += reads;
  if (win_.reads < t_.window_reads) return depth_;
  const double rate = win_.ns ? double(win_.bytes) / double(win_.ns) : 0.0;
  win_ = Window{};
  ++windows;
  if (stage_ != Stage::Held) {
    const int w = int(stage_);
    rate_[w] = rate;
    if (stage_ == Stage::U1) {
      conclude();
    } else {
      stage_ = Stage(w + 1);
      go(stage_ == Stage::One0 || stage_ == Stage::One1 ? 1 : u_);
    }
    return depth_;
  }
  const bool far = held_rate_ > 0 && (rate > held_rate_ * (1 + t_.drift) || rate < held_rate_ * (1 - t_.drift));
  far_in_a_row_ = far ? far_in_a_row_ + 1 : 0;
  if (far_in_a_row_ >= 2) calibrate(Why::Drift);
  else if (held_reads_ >= hold_for_) calibrate(Why::Recheck);
  return depth_;
}

}  // namespace tsa
