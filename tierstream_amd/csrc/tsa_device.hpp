// Device-side types shared by the HIP kernels and the host code that launches them. The POD layouts are also the
// C ABI's (include/tierstream_amd/tsa.h declares the same structs for callers).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

extern "C" {
#include "tierstream_amd/tsa.h"
}

namespace tsa {

using TsaUnit = tsa_unit;
using TsaVerifyUnit = tsa_verify_unit;
using TsaScatterJob = tsa_scatter_job;

// The synthetic generator's stream key (tsa_synth): a splitmix64 finalizer of the seed mixed with the stream id.
inline uint64_t host_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline uint64_t dev_key(uint64_t seed, uint64_t stream_id) {
  return host_mix64(seed ^ (stream_id * 0xD1B54A32D192ED03ull));
}

// Each returns a hipError_t as an int (0 = launched); none synchronizes or allocates.
int launch_digest(const TsaUnit* units_dev, uint32_t n, uint64_t* out_dev, hipStream_t stream);
int launch_verify(const TsaVerifyUnit* units_dev, uint32_t n_units, uint64_t n_segments, uint64_t seg_bytes,
                  uint32_t* fail_dev, hipStream_t stream);
int launch_scatter(const TsaScatterJob* jobs_dev, uint32_t n_jobs, uint64_t n_blocks, hipStream_t stream);
int launch_synth(void* dst, uint64_t bytes, uint64_t seed, uint64_t stream_id, uint64_t offset, uint32_t kind,
                 float sigma, hipStream_t stream);

}  // namespace tsa
