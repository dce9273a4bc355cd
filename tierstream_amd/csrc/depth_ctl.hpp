// dg_disk_queue_adapt: the depth a three-tier read pool dispatches at - 1, or its bound U (every reader stays
// allocated) - chosen from the pool's own measured read throughput. Pure: no clock, no thread; the pool feeds it one
// busy period at a time (from idle to idle: in decode, one layer's file reads), and only how many reads run at once
// depends on it, never which bytes land where.
//
// The rules are the reference's (docs/design.md 3.17, src/dg_load.hpp DgDepthCtl), kept as they are because the
// controller's choices show in the stats: busy periods add up into windows of at least 32 reads, a window's rate is
// its bytes over its busy ns. A calibration measures four windows at U, 1, 1, U; U stays only when both brackets show
// it at least 3 % faster, a split verdict is measured once more and then gives depth 1. Held at U it recalibrates
// after 512 reads; held at 1 after 4096, then every 8192 while U keeps losing; two windows in a row more than 25 %
// away from the held depth's calibrated rate recalibrate at once.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>

namespace tsa {

class ReadDepthController {
 public:
  struct Tuning {
    uint64_t window_reads = 32, recheck_at_u = 512, first_backoff = 4096, later_backoff = 8192;
    double margin = 0.03, drift = 0.25;
  };
  enum class Why : uint8_t { Start, KeepU, Keep1, Split, Recheck, Drift };
  struct Verdict {
    uint64_t seq = 0, reads = 0;          // its number; reads completed before it
    uint32_t from = 0, to = 0;            // depth before and after
    double gbps_u = 0, gbps_1 = 0;        // the calibration's mean window rates (bytes / ns)
    Why why = Why::Start;
  };
  static constexpr size_t kRecent = 16;

  explicit ReadDepthController(uint32_t bound) : ReadDepthController(bound, Tuning{}) {}
  ReadDepthController(uint32_t bound, const Tuning& t);

  uint32_t depth() const { return depth_; }
  uint32_t bound() const { return u_; }
  bool calibrating() const { return stage_ != Stage::Held; }
  // A busy period at depth() ended with `reads` reads of `bytes` over `ns`; returns the depth of the next one.
  uint32_t feed(uint64_t reads, uint64_t bytes, uint64_t ns);
  const std::deque<Verdict>& recent() const { return recent_; }  // the last kRecent verdicts, oldest first
  uint64_t verdicts() const { return verdicts_; }

  // depth changes, calibrations begun, windows closed; reads / bytes / busy ns at depth 1 and at U
  uint64_t changes = 0, calibrations = 0, windows = 0;
  uint64_t reads_1 = 0, bytes_1 = 0, ns_1 = 0, reads_u = 0, bytes_u = 0, ns_u = 0;

 private:
  enum class Stage : uint8_t { U0, One0, One1, U1, Held };  // the calibration's four windows, then held
  struct Window {
    uint64_t reads = 0, bytes = 0, ns = 0;
  };
  void go(uint32_t d);
  void calibrate(Why why);
  void conclude();
  void remember(const Verdict& v);

  Tuning t_;
  uint32_t u_, depth_;
  Stage stage_ = Stage::U0;
  Window win_;
  double rate_[4] = {0, 0, 0, 0};  // the calibration's window rates, in window order
  bool repeating_ = false;         // this calibration repeats a split one
  double held_rate_ = 0;
  uint32_t far_in_a_row_ = 0;
  uint64_t held_reads_ = 0, hold_for_ = 0, next_backoff_ = 0, all_reads_ = 0, verdicts_ = 0;
  std::deque<Verdict> recent_;
};

}  // namespace tsa
