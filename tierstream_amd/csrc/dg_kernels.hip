// Device-gated control kernels for CDNA4 (gfx950): begin, export, predict, wait, end, and the await of a file read.
// Each is one wavefront or one lane; none touches weight bytes. The protocol (sequence authorization, sticky abort,
// first error wins, the export record then its flag, the ready wait with a deadline, the completion word) is the
// reference's (src/dg_kernels.cu:31-135); the implementation is wave64-native: the export's miss mask is one ballot,
// the wait is one wavefront that polls a system-scope acquire load and sleeps between polls, and time is the
// constant-rate wall clock.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dg_proto.hpp"

namespace tsa {
namespace dgk {

__device__ __forceinline__ uint32_t ld_acq_sys(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ int32_t ld_acq_sys(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// First error of the token wins the code; abort is sticky; err_count counts wait timeouts.
__device__ void set_error(const DgDevWords& d, uint32_t code, uint32_t aux) {
  if (atomicCAS(d.err_code, 0u, code) == 0u) atomicExch(d.err_aux, aux);
  if (code == kDgTimeout) atomicAdd(d.err_count, 1u);
  atomicExch(d.abort, 1u);
}

// The step is authorized only when its sequence is the one the host published at ss_begin.
__global__ __launch_bounds__(64) void begin_kernel(DgDevWords d) {
  if (threadIdx.x != 0) return;
  const uint32_t seq = __hip_atomic_load(d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  __hip_atomic_store(d.seq, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ld_acq_sys(d.host_seq) != seq) set_error(d, kDgDesync, seq);
  __threadfence_system();
  st_sys(d.began, seq);
}

// One wavefront: lane t exports id t; the lanes whose id is absent from the device form the miss mask (one ballot).
__global__ __launch_bounds__(64) void export_kernel(DgDevWords d, uint32_t g, const int32_t* ids, uint32_t n,
                                                    uint32_t n_pred) {
  const uint32_t t = threadIdx.x;
  const uint32_t seq = __hip_atomic_load(d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t base = d.unit_base[g], units = d.unit_base[g + 1] - base;
  bool bad = false, miss = false;
  if (t < n) {
    const uint32_t id = uint32_t(ids[t]);
    d.rec[g].ids[t] = id;
    if (id >= units) bad = true;  // never looked up; the service fails the token too
    else miss = ld_acq_sys(d.slot_of + base + id) < 0;
  }
  const uint64_t mask = __ballot(miss);
  const uint64_t badm = __ballot(bad);
  if (t == 0) {
    if (badm) set_error(d, kDgBadId, g);
    DgRecord& r = d.rec[g];
    r.n_ids = n;
    r.n_pred_promised = n_pred;
    r.mask_lo = uint32_t(mask);
    r.mask_hi = uint32_t(mask >> 32);
    r.seq = seq;
    d.any_miss[g] = mask != 0ull ? 1u : 0u;
    if (d.stamps) {
      d.stamps[4u * g + 1u] = 0ull;
      d.stamps[4u * g + 2u] = 0ull;
      d.stamps[4u * g + 3u] = 0ull;
      d.stamps[4u * g] = wall_clock64();
    }
  }
  __threadfence_system();  // every lane's record stores are visible before the flag
  if (t == 0) st_sys(d.flag + g, seq);
}

__global__ __launch_bounds__(64) void predict_kernel(DgDevWords d, uint32_t g, const int32_t* ids, uint32_t n) {
  const uint32_t t = threadIdx.x;
  if (t < n) d.prec[g].pred[t] = uint32_t(ids[t]);
  if (t == 0) d.prec[g].n_pred = n;
  __threadfence_system();
  if (t == 0) st_sys(d.pflag + g, __hip_atomic_load(d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// One wavefront; lane 0 polls. Zero-miss layers return at once on the HBM any_miss word. A miss waits for ready[g] to
// reach the token's sequence (a system-scope acquire that pairs with the service's value-write behind the copies),
// polling with an s_sleep backoff; the host's abort word and the wall-clock deadline end it with an error.
// Stamps (wall clock): [1] entry and [3] exit on every path, [2] the poll that saw ready (left 0 by the export when
// the layer had no miss).
__device__ __forceinline__ void wait_poll(const DgDevWords& d, uint32_t g, uint64_t t0) {
  if (__hip_atomic_load(d.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
  if (!__hip_atomic_load(d.any_miss + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
  const uint32_t seq = __hip_atomic_load(d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (uint32_t polls = 0;; ++polls) {
    if (int32_t(ld_acq_sys(d.ready + g) - seq) >= 0) {
      if (d.stamps) d.stamps[4u * g + 2u] = wall_clock64();
      return;
    }
    if ((polls & 15u) == 15u) {  // the host's abort lives across PCIe: looked at every 16th poll
      if (ld_acq_sys(d.host_abort)) {
        set_error(d, kDgHostAbort, g);
        return;
      }
      if (wall_clock64() - t0 > d.timeout_ticks) {
        set_error(d, kDgTimeout, g);
        return;
      }
    }
    __builtin_amdgcn_s_sleep(2);
  }
}
__global__ __launch_bounds__(64) void wait_kernel(DgDevWords d, uint32_t g) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  wait_poll(d, g, t0);
  if (d.stamps) {
    d.stamps[4u * g + 1u] = t0;
    d.stamps[4u * g + 3u] = wall_clock64();
  }
}

__global__ __launch_bounds__(64) void end_kernel(DgDevWords d) {
  if (threadIdx.x != 0) return;
  if (__hip_atomic_load(d.absent_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &&
      !__hip_atomic_load(d.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
    set_error(d, kDgAbsent, 0);
  st_sys(d.m_err_count, __hip_atomic_load(d.err_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  st_sys(d.m_err_code, __hip_atomic_load(d.err_code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  st_sys(d.m_err_aux, __hip_atomic_load(d.err_aux, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  __threadfence_system();
  st_sys(d.done, __hip_atomic_load(d.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// A staging buffer's file read, awaited on the stream that copies out of it: lane 0 polls the reader's word (a
// system-scope acquire: the reader stores the read's generation after the read returned) with the wait kernel's
// exits: the token's device abort (it fails already), the host's abort, and the deadline.
__global__ __launch_bounds__(64) void await_kernel(DgDevWords d, const uint32_t* word, uint32_t gen, uint32_t aux) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  for (uint32_t polls = 0;; ++polls) {
    if (ld_acq_sys(word) == gen) return;
    if (__hip_atomic_load(d.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
    if ((polls & 15u) == 15u) {
      if (ld_acq_sys(d.host_abort)) {
        set_error(d, kDgHostAbort, aux);
        return;
      }
      if (wall_clock64() - t0 > d.timeout_ticks) {
        set_error(d, kDgTimeout, aux);
        return;
      }
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

__global__ __launch_bounds__(64) void store_kernel(uint32_t* word, uint32_t v) {
  if (threadIdx.x != 0) return;
  __threadfence_system();
  __hip_atomic_store(word, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace dgk

int dg_launch_begin(const DgDevWords& d, void* s) {
  hipLaunchKernelGGL(dgk::begin_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d);
  return int(hipGetLastError());
}
int dg_launch_export(const DgDevWords& d, uint32_t g, const int32_t* ids, uint32_t n, uint32_t n_pred, void* s) {
  hipLaunchKernelGGL(dgk::export_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d, g, ids, n, n_pred);
  return int(hipGetLastError());
}
int dg_launch_predict(const DgDevWords& d, uint32_t g, const int32_t* ids, uint32_t n, void* s) {
  hipLaunchKernelGGL(dgk::predict_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d, g, ids, n);
  return int(hipGetLastError());
}
int dg_launch_wait(const DgDevWords& d, uint32_t g, void* s) {
  hipLaunchKernelGGL(dgk::wait_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d, g);
  return int(hipGetLastError());
}
int dg_launch_end(const DgDevWords& d, void* s) {
  hipLaunchKernelGGL(dgk::end_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d);
  return int(hipGetLastError());
}
int dg_launch_await(const DgDevWords& d, const uint32_t* word, uint32_t gen, uint32_t aux, void* s) {
  hipLaunchKernelGGL(dgk::await_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), d, word, gen, aux);
  return int(hipGetLastError());
}
int dg_launch_store(uint32_t* word, uint32_t v, void* s) {
  hipLaunchKernelGGL(dgk::store_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s), word, v);
  return int(hipGetLastError());
}

}  // namespace tsa
