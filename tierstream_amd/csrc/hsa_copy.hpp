// Unit copies issued to the HSA runtime's copy engines directly, each with a completion signal that the host polls and
// that later copies name as dependencies (the copy engine waits for those itself).
//
// Why not a HIP stream: a copy on a HIP stream followed by anything on the same stream (an event record, a value
// write) leaves a barrier packet on the stream's compute queue that waits for the copy engine. On MI355X such a
// barrier parked on one CU-masked queue slows every kernel dispatched from the other CU-masked queues - the device
// check of landed units among them. Measured on one MI355X, one 336 MiB check (3 parts of 112 MiB, 2 KiB segments):
// 57 us alone; 85 us beside H2D copies on a CU-masked stream with an event after each; 58 us beside the same copies
// issued here; both copy at 57.3 GB/s. D2H copies with an event after them did not slow it.
//
// The runtime's entry points are taken from the HSA runtime the HIP runtime has already loaded (no link-time
// dependency for engines that link this library statically).
#pragma once

#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <cstdint>
#include <deque>
#include <mutex>
#include <vector>

namespace tsa {

class HsaCopier {
 public:
  // The GPU agent of HIP device `hip_device` (matched by PCI location) and a CPU agent for host memory.
  explicit HsaCopier(int hip_device);
  ~HsaCopier();  // waits for every copy issued here
  HsaCopier(const HsaCopier&) = delete;
  HsaCopier& operator=(const HsaCopier&) = delete;

  // Signals are indices; 0 is "nothing" (always complete). copy() returns the copy's signal holding one reference
  // (the caller's); a signal goes back to the pool once it has no reference left and its copy has ended.
  // to_host: device memory -> pinned host memory, else the other way. The copy starts once every dep has ended.
  uint32_t copy(void* dst, const void* src, uint64_t bytes, bool to_host, const uint32_t* deps, uint32_t n_deps);
  bool done(uint32_t sig) const;
  void ref(uint32_t sig);
  void unref(uint32_t sig);
  // Copy-engine timestamps for the copies issued while on (process-wide in the runtime); copy_ns: the engine's
  // start-to-end time of an ended copy issued while on (false: none recorded).
  void profiling(bool on);
  bool copy_ns(uint32_t sig, uint64_t* ns) const;
  void wait_all() const;

 private:
  struct Api;
  struct Entry {
    hsa_signal_t s{};
    uint32_t refs = 0;
    // the signals this copy's engine polls before it starts: held until the copy has ended (a signal recycled for a
    // later copy while a poll of it is still queued would make the poll wait for that later copy)
    std::vector<uint32_t> deps;
  };
  void release_locked(uint32_t sig);
  uint32_t take_locked();
  bool done_locked(uint32_t sig) const;

  const Api* api_;
  hsa_agent_t gpu_{}, cpu_{};
  double ticks_per_ns_ = 1.0;
  mutable std::mutex mu_;
  std::deque<Entry> e_;                // e_[0] unused (index 0 is "nothing")
  std::vector<uint32_t> free_, retiring_;  // free: ended and unreferenced; retiring: unreferenced, maybe running
  std::vector<hsa_signal_t> dep_buf_;
};

}  // namespace tsa
