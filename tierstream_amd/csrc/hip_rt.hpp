// The discrete-GPU device layer: HBM allocations, pinned host memory, streams, events and copies on one MI355X.
// Every HIP error becomes Error(SS_E_BACKEND) (SS_E_NOMEM for allocations). Streams are created non-blocking at the
// default priority; copy streams are served by the SDMA engines.
//
// Hardware queues. The runtime multiplexes a process's streams over a few hardware queues (GPU_MAX_HW_QUEUES, 4 by
// default). Work behind a kernel that occupies a queue waits for that kernel, whatever stream it came from, and that
// includes SDMA copies and value-writes (their ordering packets go through the same queue). A device-gated engine
// spins in its wait kernel until the library publishes a ready word, so a publishing stream that shared the engine's
// queue would deadlock until the wait timed out. Streams the library publishes or copies on are therefore created with
// a CU mask that names every CU: the runtime gives such a stream a hardware queue of its own.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

#include "common.hpp"

namespace tsa {

void hip_check(hipError_t e, const char* what);

class HipDevice {
 public:
  explicit HipDevice(int device);
  int device() const { return dev_; }
  void bind() const;  // hipSetDevice on the calling thread

  void* alloc_device(uint64_t bytes, const char* what);
  void free_device(void* p) noexcept;
  // Coarse-grained pinned host memory: DMA sources and destinations (the pinned tier, staging, tables).
  void* alloc_pinned(uint64_t bytes, const char* what);
  // Fine-grained, coherent, device-mapped host memory: words the device writes and the host polls (and back).
  void* alloc_mapped(uint64_t bytes, void** dev_ptr, const char* what);
  void free_pinned(void* p) noexcept;

  hipStream_t stream_create();            // pooled hardware queue (open-time work)
  hipStream_t stream_create_dedicated();  // a hardware queue of its own (serve-time copies and publications)
  void stream_destroy(hipStream_t s) noexcept;
  hipEvent_t event_create();  // timing disabled
  hipEvent_t event_create_timed();
  void event_destroy(hipEvent_t e) noexcept;

 private:
  int dev_;
  int cus_ = 0;
};

inline void ev_record(hipEvent_t e, hipStream_t s) { hip_check(hipEventRecord(e, s), "hipEventRecord"); }
inline void ev_sync(hipEvent_t e) {
  if (e) hip_check(hipEventSynchronize(e), "hipEventSynchronize");
}
inline bool ev_done(hipEvent_t e) {
  const hipError_t r = hipEventQuery(e);
  if (r == hipSuccess) return true;
  if (r == hipErrorNotReady) return false;
  hip_check(r, "hipEventQuery");
  return false;
}
inline void stream_wait(hipStream_t s, hipEvent_t e) {
  if (e) hip_check(hipStreamWaitEvent(s, e, 0), "hipStreamWaitEvent");
}
inline void stream_sync(hipStream_t s) { hip_check(hipStreamSynchronize(s), "hipStreamSynchronize"); }
inline void copy_h2d(void* dst, const void* src, uint64_t n, hipStream_t s) {
  hip_check(hipMemcpyAsync(dst, src, size_t(n), hipMemcpyHostToDevice, s), "hipMemcpyAsync (host to device)");
}
inline void copy_d2h(void* dst, const void* src, uint64_t n, hipStream_t s) {
  hip_check(hipMemcpyAsync(dst, src, size_t(n), hipMemcpyDeviceToHost, s), "hipMemcpyAsync (device to host)");
}
inline void copy_d2d(void* dst, const void* src, uint64_t n, hipStream_t s) {
  hip_check(hipMemcpyAsync(dst, src, size_t(n), hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (device to device)");
}

}  // namespace tsa
