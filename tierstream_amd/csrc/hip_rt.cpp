#include "hip_rt.hpp"

#include <vector>

namespace tsa {

void hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  fail(e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation ? SS_E_NOMEM : SS_E_BACKEND,
       std::string(what) + ": " + hipGetErrorString(e));
}

HipDevice::HipDevice(int device) : dev_(device) {
  int n = 0;
  hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
  require(device >= 0 && device < n, SS_E_INVALID,
          "open: HIP device " + std::to_string(device) + " does not exist (" + std::to_string(n) + " visible)");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  require(prop.integrated == 0, SS_E_UNSUPPORTED,
          "open: SS_BACKEND_HIP in this library is the discrete-GPU backend; device " + std::to_string(device) +
              " is an integrated (unified-memory) GPU");
  cus_ = prop.multiProcessorCount;
  bind();
}

void HipDevice::bind() const { hip_check(hipSetDevice(dev_), "hipSetDevice"); }

void* HipDevice::alloc_device(uint64_t bytes, const char* what) {
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, size_t(bytes ? bytes : 1));
  if (e != hipSuccess)
    fail(SS_E_NOMEM, std::string("device allocation of ") + std::to_string(bytes) + " bytes (" + what +
                         ") failed: " + hipGetErrorString(e));
  return p;
}

void HipDevice::free_device(void* p) noexcept {
  if (p) (void)hipFree(p);
}

void* HipDevice::alloc_pinned(uint64_t bytes, const char* what) {
  void* p = nullptr;
  const hipError_t e = hipHostMalloc(&p, size_t(bytes ? bytes : 1), hipHostMallocDefault | hipHostMallocNonCoherent);
  if (e != hipSuccess)
    fail(SS_E_NOMEM, std::string("pinned allocation of ") + std::to_string(bytes) + " bytes (" + what +
                         ") failed: " + hipGetErrorString(e));
  return p;
}

void* HipDevice::alloc_mapped(uint64_t bytes, void** dev_ptr, const char* what) {
  void* p = nullptr;
  const hipError_t e =
      hipHostMalloc(&p, size_t(bytes ? bytes : 1), hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable);
  if (e != hipSuccess)
    fail(SS_E_NOMEM, std::string("mapped allocation of ") + std::to_string(bytes) + " bytes (" + what +
                         ") failed: " + hipGetErrorString(e));
  std::memset(p, 0, size_t(bytes ? bytes : 1));
  if (dev_ptr) hip_check(hipHostGetDevicePointer(dev_ptr, p, 0), "hipHostGetDevicePointer");
  return p;
}

void HipDevice::free_pinned(void* p) noexcept {
  if (p) (void)hipHostFree(p);
}

hipStream_t HipDevice::stream_create() {
  hipStream_t s = nullptr;
  hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  return s;
}

hipStream_t HipDevice::stream_create_dedicated() {
  std::vector<uint32_t> mask(size_t((cus_ + 31) / 32), 0u);
  for (int c = 0; c < cus_; ++c) mask[size_t(c / 32)] |= 1u << (c % 32);
  hipStream_t s = nullptr;
  hip_check(hipExtStreamCreateWithCUMask(&s, uint32_t(mask.size()), mask.data()), "hipExtStreamCreateWithCUMask");
  return s;
}

void HipDevice::stream_destroy(hipStream_t s) noexcept {
  if (s) (void)hipStreamDestroy(s);
}

hipEvent_t HipDevice::event_create() {
  hipEvent_t e = nullptr;
  hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags");
  return e;
}

// Timing brackets carry only timestamps: recorded without a system-scope fence (no L2 write-back and invalidate at a
// bracket, which would also touch the work it measures).
hipEvent_t HipDevice::event_create_timed() {
  hipEvent_t e = nullptr;
  hip_check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreateWithFlags (timing)");
  return e;
}

void HipDevice::event_destroy(hipEvent_t e) noexcept {
  if (e) (void)hipEventDestroy(e);
}

}  // namespace tsa
