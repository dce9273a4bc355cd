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

// One device-gated verify launch: up to kDgVerifyMax landed units of the arena's shape, passed by value (a launch
// needs no table upload). Unit i is key keys[i] in slot slots[i]: part p at arena[p] + slot x part_bytes[p]; its
// checkpoints at ckpt + key x unit_segs x 4 and its digest at digests[key]. A mismatch sets fail[i] |= 1 and, when
// abort is set (the gate), the token's first error (err, aux) and its sticky abort word, before the kernel ends.
constexpr uint32_t kDgVerifyMax = 64;
struct DgVerifyLaunch {
  const unsigned char* arena[4] = {};
  uint64_t part_bytes[4] = {};
  uint64_t part_segs[4] = {};  // segments of each part: ceil(span / seg_bytes), the last part's span rounded down to 32
  uint32_t n_parts = 0;
  uint32_t n = 0;
  uint64_t seg_bytes = 0;
  uint64_t unit_segs = 0;  // the sum of part_segs: checkpoints per unit
  uint64_t unit_bytes = 0;
  const uint64_t* ckpt = nullptr;
  const uint64_t* digests = nullptr;
  uint32_t* fail = nullptr;
  uint32_t* abort = nullptr;
  uint32_t* err_code = nullptr;
  uint32_t* err_aux = nullptr;
  uint32_t err = 0, aux = 0;
  // Publication (publish 0: none): once the check has ended, a one-wave kernel on the same stream writes every unit's
  // entry slot_of[key] = slot (when slot_of is set), then ready[ready_g] = seq (when ready is set).
  uint32_t publish = 0;
  int32_t* slot_of = nullptr;
  uint32_t* ready = nullptr;
  uint32_t ready_g = 0, seq = 0;
  uint32_t keys[kDgVerifyMax] = {};
  int32_t slots[kDgVerifyMax] = {};
};

// The arena shape of a launch: parts, their segments at seg_bytes (the checkpoint layout of tsa_checkpoint_count with
// the parts as the extents) and the unit's bytes. Returns false when a part but the last is not a multiple of 32.
inline bool set_dg_verify_shape(DgVerifyLaunch& l, const void* const* arena, const uint64_t* part_bytes, uint32_t n_parts,
                                uint64_t seg_bytes) {
  uint64_t segs = 0;
  l.unit_bytes = 0;
  for (uint32_t p = 0; p < n_parts; ++p) {
    const bool last = p + 1 == n_parts;
    const uint64_t span = last ? part_bytes[p] / 32 * 32 : part_bytes[p];
    if (!last && span % 32 != 0) return false;
    l.arena[p] = static_cast<const unsigned char*>(arena[p]);
    l.part_bytes[p] = part_bytes[p];
    l.part_segs[p] = (span + seg_bytes - 1) / seg_bytes;
    if (last && l.part_segs[p] == 0) l.part_segs[p] = 1;
    segs += l.part_segs[p];
    l.unit_bytes += part_bytes[p];
  }
  l.n_parts = n_parts;
  l.seg_bytes = seg_bytes;
  l.unit_segs = segs;
  return true;
}

// Each returns a hipError_t as an int (0 = launched); none synchronizes or allocates.
int launch_digest(const TsaUnit* units_dev, uint32_t n, uint64_t* out_dev, hipStream_t stream);
// start / stop (timing events, or null): recorded with the kernel's own begin and end (hipExtLaunchKernelGGL).
int launch_verify(const TsaVerifyUnit* units_dev, uint32_t n_units, uint64_t n_segments, uint64_t seg_bytes,
                  uint32_t* fail_dev, hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// start / stop (timing events, or null): recorded with the kernel's own begin and end (hipExtLaunchKernelGGL).
int launch_dg_verify(const DgVerifyLaunch& a, hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// The staged units' fused scatter and check: unit i's parts lie back to back at src + i x unit_bytes (HBM staging);
// each is written to its arena slot while it is hashed, with the same checks and publication as launch_dg_verify.
int launch_dg_scatter_verify(const DgVerifyLaunch& a, const void* src, hipStream_t stream, hipEvent_t start = nullptr,
                             hipEvent_t stop = nullptr);
int launch_scatter(const TsaScatterJob* jobs_dev, uint32_t n_jobs, uint64_t n_blocks, hipStream_t stream);
int launch_synth(void* dst, uint64_t bytes, uint64_t seed, uint64_t stream_id, uint64_t offset, uint32_t kind,
                 float sigma, hipStream_t stream);

}  // namespace tsa
