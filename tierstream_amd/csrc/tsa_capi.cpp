// C ABI of the MI355X extensions (include/tierstream_amd/tsa.h) and the library-wide error state.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <string>

#include "common.hpp"
#include "tsa_device.hpp"

namespace tsa {
namespace {
thread_local std::string g_last_error;
}

void set_last_error(const char* msg) noexcept {
  try {
    g_last_error = msg ? msg : "";
  } catch (...) {
  }
}
void clear_last_error() noexcept {}

namespace {

void hip_ck(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  fail(e == hipErrorOutOfMemory ? SS_E_NOMEM : SS_E_BACKEND, std::string(what) + ": " + hipGetErrorString(e));
}
void launch_ck(int e, const char* what) { hip_ck(hipError_t(e), what); }

void check_extents(const tsa_extent* ext, uint32_t n, const char* what) {
  require(n >= 1 && n <= TSA_MAX_EXTENTS, SS_E_INVALID, std::string(what) + ": 1..4 extents per unit");
  for (uint32_t e = 0; e < n; ++e) {
    require(ext[e].ptr != nullptr || ext[e].bytes == 0, SS_E_INVALID, std::string(what) + ": null extent");
    require(reinterpret_cast<uintptr_t>(ext[e].ptr) % 8 == 0, SS_E_INVALID,
            std::string(what) + ": extents must start 8-byte aligned");
    if (e + 1 < n)
      require(ext[e].bytes % 32 == 0, SS_E_INVALID,
              std::string(what) + ": every extent but the last must be a multiple of 32 bytes");
  }
}

uint64_t count_checkpoints(const uint64_t* bytes, uint32_t n, uint64_t seg) {
  uint64_t c = 0;
  for (uint32_t e = 0; e < n; ++e) {
    const bool last = e + 1 == n;
    const uint64_t span = last ? bytes[e] / 32 * 32 : bytes[e];
    uint64_t k = (span + seg - 1) / seg;
    if (last && k == 0) k = 1;
    c += k;
  }
  return c;
}

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" {

const char* ss_last_error(void) { return g_last_error.c_str(); }
int ss_abi_version(void) { return SS_ABI_VERSION; }
void ss_free(void* p) { std::free(p); }

ss_status tsa_xxh64_digest(const tsa_unit* units_dev, uint32_t n, uint64_t* digests_dev, void* stream) {
  return guard([&] {
    require(n == 0 || (units_dev && digests_dev), SS_E_INVALID, "tsa_xxh64_digest: null table");
    launch_ck(launch_digest(units_dev, n, digests_dev, static_cast<hipStream_t>(stream)), "tsa_xxh64_digest");
  });
}

uint64_t tsa_xxh64_host(const void* data, uint64_t bytes) {
  if (!data && bytes) return 0;
  return xxh64(data, size_t(bytes));
}

uint64_t tsa_checkpoint_count(const uint64_t* extent_bytes, uint32_t n_ext, uint64_t seg_bytes) {
  if (!extent_bytes || n_ext == 0 || n_ext > TSA_MAX_EXTENTS || seg_bytes == 0 || seg_bytes % 32) return 0;
  return count_checkpoints(extent_bytes, n_ext, seg_bytes);
}

ss_status tsa_xxh64_checkpoints(const tsa_unit* u, uint64_t seg, uint64_t* states, uint64_t n_states,
                                uint64_t* digest) {
  return guard([&] {
    require(u != nullptr, SS_E_INVALID, "tsa_xxh64_checkpoints: null unit");
    require(seg > 0 && seg % 32 == 0, SS_E_INVALID, "tsa_xxh64_checkpoints: seg_bytes must be a multiple of 32");
    check_extents(u->ext, u->n_ext, "tsa_xxh64_checkpoints");
    uint64_t bytes[TSA_MAX_EXTENTS];
    for (uint32_t e = 0; e < u->n_ext; ++e) bytes[e] = u->ext[e].bytes;
    const uint64_t need = count_checkpoints(bytes, u->n_ext, seg);
    require(states != nullptr && n_states >= need, SS_E_INVALID,
            "tsa_xxh64_checkpoints: the states array holds " + std::to_string(n_states) + " of " +
                std::to_string(need) + " checkpoints");
    Xxh64 h;
    uint64_t k = 0;
    for (uint32_t e = 0; e < u->n_ext; ++e) {
      const bool last = e + 1 == u->n_ext;
      const char* p = static_cast<const char*>(u->ext[e].ptr);
      const uint64_t span = last ? bytes[e] / 32 * 32 : bytes[e];
      uint64_t nseg = (span + seg - 1) / seg;
      if (last && nseg == 0) nseg = 1;
      for (uint64_t s = 0; s < nseg; ++s) {
        std::memcpy(states + 4 * k, h.acc(), 32);
        ++k;
        const uint64_t off = s * seg, end = std::min(off + seg, span);
        if (end > off) h.update(p + off, size_t(end - off));
      }
      if (last && bytes[e] > span) h.update(p + span, size_t(bytes[e] - span));
    }
    if (digest) *digest = h.digest();
  });
}

ss_status tsa_xxh64_verify(const tsa_verify_unit* units_dev, uint32_t n_units, uint64_t n_segments,
                           uint64_t seg_bytes, uint32_t* fail_dev, void* stream) {
  return guard([&] {
    require(n_units == 0 || (units_dev && fail_dev), SS_E_INVALID, "tsa_xxh64_verify: null table");
    require(seg_bytes > 0 && seg_bytes % 32 == 0, SS_E_INVALID, "tsa_xxh64_verify: seg_bytes must be a multiple of 32");
    launch_ck(launch_verify(units_dev, n_units, n_segments, seg_bytes, fail_dev, static_cast<hipStream_t>(stream)),
              "tsa_xxh64_verify");
  });
}

// The checks of n arena units in launches of up to kDgVerifyMax; src_dev (the fused scatter): the units' bytes back
// to back, unit i at src_dev + i x unit_bytes, written to their slots while they are hashed.
static void arena_checks(const char* what, const tsa_arena_verify* a, const uint32_t* keys, const int32_t* slots,
                         uint32_t n, const void* src_dev, uint32_t* fail_dev, void* stream) {
  const std::string w(what);
  require(a != nullptr, SS_E_INVALID, w + ": null arena");
  require(n == 0 || (keys && slots && fail_dev), SS_E_INVALID, w + ": null argument");
  require(a->n_parts >= 1 && a->n_parts <= TSA_MAX_EXTENTS, SS_E_INVALID, w + ": 1..4 parts");
  require(a->seg_bytes > 0 && a->seg_bytes % 32 == 0, SS_E_INVALID, w + ": seg_bytes must be a multiple of 32");
  require(n == 0 || (a->states_dev && a->digests_dev), SS_E_INVALID, w + ": null states or digests");
  for (uint32_t p = 0; p < a->n_parts; ++p)
    require(a->arena[p] != nullptr && reinterpret_cast<uintptr_t>(a->arena[p]) % 8 == 0 && a->part_bytes[p] % 8 == 0,
            SS_E_INVALID, w + ": every arena part 8-byte aligned with a multiple of 8 bytes");
  DgVerifyLaunch l;
  require(set_dg_verify_shape(l, a->arena, a->part_bytes, a->n_parts, a->seg_bytes), SS_E_INVALID,
          w + ": a part but the last is not a multiple of 32");
  require(n == 0 || !src_dev || reinterpret_cast<uintptr_t>(src_dev) % 8 == 0, SS_E_INVALID,
          w + ": the staged bytes must be 8-byte aligned");
  l.ckpt = a->states_dev;
  l.digests = a->digests_dev;
  for (uint32_t i0 = 0; i0 < n; i0 += kDgVerifyMax) {
    l.n = std::min(kDgVerifyMax, n - i0);
    l.fail = fail_dev + i0;
    for (uint32_t i = 0; i < l.n; ++i) {
      require(slots[i0 + i] >= 0, SS_E_INVALID, w + ": negative slot");
      l.keys[i] = keys[i0 + i];
      l.slots[i] = slots[i0 + i];
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (src_dev)
      launch_ck(launch_dg_scatter_verify(l, static_cast<const char*>(src_dev) + uint64_t(i0) * l.unit_bytes, s), what);
    else
      launch_ck(launch_dg_verify(l, s), what);
  }
}

ss_status tsa_xxh64_verify_slots(const tsa_arena_verify* a, const uint32_t* keys, const int32_t* slots, uint32_t n,
                                 uint32_t* fail_dev, void* stream) {
  return guard([&] { arena_checks("tsa_xxh64_verify_slots", a, keys, slots, n, nullptr, fail_dev, stream); });
}

ss_status tsa_xxh64_scatter_verify_slots(const tsa_arena_verify* a, const uint32_t* keys, const int32_t* slots,
                                         uint32_t n, const void* src_dev, uint32_t* fail_dev, void* stream) {
  return guard([&] {
    require(n == 0 || src_dev, SS_E_INVALID, "tsa_xxh64_scatter_verify_slots: null staged bytes");
    arena_checks("tsa_xxh64_scatter_verify_slots", a, keys, slots, n, src_dev, fail_dev, stream);
  });
}

uint64_t tsa_scatter_blocks(const uint64_t* part_bytes, uint32_t n_parts) {
  uint64_t b = 0;
  for (uint32_t p = 0; part_bytes && p < n_parts && p < TSA_MAX_EXTENTS; ++p)
    b += (part_bytes[p] + TSA_SCATTER_BLOCK_BYTES - 1) / TSA_SCATTER_BLOCK_BYTES;
  return b;
}

ss_status tsa_scatter(const tsa_scatter_job* jobs_dev, uint32_t n_jobs, uint64_t n_blocks, void* stream) {
  return guard([&] {
    require(n_jobs == 0 || jobs_dev, SS_E_INVALID, "tsa_scatter: null job table");
    launch_ck(launch_scatter(jobs_dev, n_jobs, n_blocks, static_cast<hipStream_t>(stream)), "tsa_scatter");
  });
}

ss_status tsa_synth(void* dst_dev, uint64_t bytes, uint64_t seed, uint64_t stream_id, uint64_t offset, uint32_t kind,
                    float sigma, void* stream) {
  return guard([&] {
    require(bytes % 8 == 0 && offset % 8 == 0, SS_E_INVALID, "tsa_synth: bytes and offset must be multiples of 8");
    require(kind <= 2, SS_E_INVALID, "tsa_synth: kind 0 (uniform bytes), 1 (bf16 normal) or 2 (Q4 blocks)");
    require(bytes == 0 || dst_dev, SS_E_INVALID, "tsa_synth: null destination");
    launch_ck(launch_synth(dst_dev, bytes, seed, stream_id, offset, kind, sigma, static_cast<hipStream_t>(stream)),
              "tsa_synth");
  });
}

ss_status tsa_device_count(int* n) {
  return guard([&] {
    require(n != nullptr, SS_E_INVALID, "tsa_device_count: null");
    hip_ck(hipGetDeviceCount(n), "hipGetDeviceCount");
  });
}
ss_status tsa_set_device(int device) { return guard([&] { hip_ck(hipSetDevice(device), "hipSetDevice"); }); }
ss_status tsa_malloc(void** p, uint64_t bytes) {
  return guard([&] {
    require(p != nullptr, SS_E_INVALID, "tsa_malloc: null");
    *p = nullptr;
    hip_ck(hipMalloc(p, size_t(bytes ? bytes : 1)), "hipMalloc");
  });
}
ss_status tsa_free(void* p) { return guard([&] { hip_ck(hipFree(p), "hipFree"); }); }
ss_status tsa_host_alloc(void** p, uint64_t bytes) {
  return guard([&] {
    require(p != nullptr, SS_E_INVALID, "tsa_host_alloc: null");
    *p = nullptr;
    hip_ck(hipHostMalloc(p, size_t(bytes ? bytes : 1), hipHostMallocDefault), "hipHostMalloc");
  });
}
ss_status tsa_host_free(void* p) { return guard([&] { hip_ck(hipHostFree(p), "hipHostFree"); }); }
ss_status tsa_memcpy(void* dst, const void* src, uint64_t bytes, int kind, void* stream) {
  return guard([&] {
    static const hipMemcpyKind kinds[4] = {hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice,
                                           hipMemcpyDefault};
    require(kind >= 0 && kind <= 3, SS_E_INVALID, "tsa_memcpy: kind 0..3");
    hip_ck(hipMemcpyAsync(dst, src, size_t(bytes), kinds[kind], static_cast<hipStream_t>(stream)), "hipMemcpyAsync");
  });
}
ss_status tsa_memset(void* dst, int value, uint64_t bytes, void* stream) {
  return guard([&] {
    hip_ck(hipMemsetAsync(dst, value, size_t(bytes), static_cast<hipStream_t>(stream)), "hipMemsetAsync");
  });
}
ss_status tsa_stream_create(void** stream) {
  return guard([&] {
    require(stream != nullptr, SS_E_INVALID, "tsa_stream_create: null");
    hipStream_t s = nullptr;
    hip_ck(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *stream = s;
  });
}
ss_status tsa_stream_destroy(void* stream) {
  return guard([&] { hip_ck(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy"); });
}
ss_status tsa_stream_sync(void* stream) {
  return guard([&] { hip_ck(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize"); });
}
ss_status tsa_device_sync(void) { return guard([&] { hip_ck(hipDeviceSynchronize(), "hipDeviceSynchronize"); }); }
ss_status tsa_event_create(void** ev) {
  return guard([&] {
    require(ev != nullptr, SS_E_INVALID, "tsa_event_create: null");
    hipEvent_t e = nullptr;
    hip_ck(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreateWithFlags");
    *ev = e;
  });
}
ss_status tsa_event_destroy(void* ev) {
  return guard([&] { hip_ck(hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy"); });
}
ss_status tsa_event_record(void* ev, void* stream) {
  return guard([&] {
    hip_ck(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream)), "hipEventRecord");
  });
}
ss_status tsa_event_sync(void* ev) {
  return guard([&] { hip_ck(hipEventSynchronize(static_cast<hipEvent_t>(ev)), "hipEventSynchronize"); });
}
ss_status tsa_event_elapsed_ms(void* a, void* b, float* ms) {
  return guard([&] {
    require(ms != nullptr, SS_E_INVALID, "tsa_event_elapsed_ms: null");
    hip_ck(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)), "hipEventElapsedTime");
  });
}

}  // extern "C"
