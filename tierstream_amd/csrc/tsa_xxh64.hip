// Device XXH64 (seed 0) for units already resident in HBM, two kernels:
//
//  * digest: one lane-quad per unit, lane q owns accumulator q and streams the unit's 32-byte stripes in order. XXH64
//    keeps four dependent 64-bit chains per input, each chain a sequence of rotl(v + w*P2, 31)*P1 steps: there is no
//    associative combine, so a unit's digest is chain-latency bound (one quad) and the kernel reaches HBM speed only
//    with thousands of units in one launch.
//  * verify: checkpoint-parallel. The host hashes every unit once while it fills the pinned tier / the arena and keeps
//    the four accumulators at the start of every segment (a fixed byte count inside each extent). On the device each
//    (unit, segment) pair is an independent quad: start from the segment's checkpoint, run the segment's stripes over
//    the device bytes, and require the next checkpoint (or, for the unit's last segment, the finalized digest equal to
//    the descriptor's hash). All segments of all units run in parallel, so one launch is HBM-bound even for one unit.
//    If every segment agrees, the device bytes' XXH64 equals the descriptor hash exactly (the transitions compose).
//
// Byte order and the algorithm follow the published XXH64 description (reference src/xxh64.cpp:39-112 restates it).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tsa_device.hpp"

namespace tsa {
namespace dev {

constexpr uint64_t P1 = 0x9E3779B185EBCA87ull;
constexpr uint64_t P2 = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t P3 = 0x165667B19E3779F9ull;
constexpr uint64_t P4 = 0x85EBCA77C2B2AE63ull;
constexpr uint64_t P5 = 0x27D4EB2F165667C5ull;

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
// rotl by 31 as two funnel shifts (v_alignbit_b32) on the 32-bit halves: hi' = (hi:lo) >> 1, lo' = (lo:hi) >> 1
__device__ __forceinline__ uint64_t rotl31(uint64_t x) {
  const uint32_t hi = uint32_t(x >> 32), lo = uint32_t(x);
  return uint64_t(__builtin_amdgcn_alignbit(hi, lo, 1u)) << 32 | __builtin_amdgcn_alignbit(lo, hi, 1u);
}
__device__ __forceinline__ uint64_t xround(uint64_t acc, uint64_t w) { return rotl31(acc + w * P2) * P1; }
__device__ __forceinline__ uint64_t xmerge(uint64_t h, uint64_t v) { return (h ^ xround(0, v)) * P1 + P4; }

// Digest of the four accumulators, the total length and the (< 32 byte) tail. Runs on one lane.
__device__ uint64_t xfinal(const uint64_t v[4], uint64_t total, const unsigned char* tail, uint32_t tail_len) {
  uint64_t h;
  if (total >= 32) {
    h = rotl64(v[0], 1) + rotl64(v[1], 7) + rotl64(v[2], 12) + rotl64(v[3], 18);
    for (int k = 0; k < 4; ++k) h = xmerge(h, v[k]);
  } else {
    h = P5;  // seed 0
  }
  h += total;
  uint32_t i = 0;
  for (; i + 8 <= tail_len; i += 8) {
    uint64_t w = 0;
    for (int b = 7; b >= 0; --b) w = (w << 8) | tail[i + b];
    h ^= xround(0, w);
    h = rotl64(h, 27) * P1 + P4;
  }
  if (i + 4 <= tail_len) {
    const uint32_t w = uint32_t(tail[i]) | uint32_t(tail[i + 1]) << 8 | uint32_t(tail[i + 2]) << 16 |
                       uint32_t(tail[i + 3]) << 24;
    h ^= uint64_t(w) * P1;
    h = rotl64(h, 23) * P2 + P3;
    i += 4;
  }
  for (; i < tail_len; ++i) {
    h ^= uint64_t(tail[i]) * P5;
    h = rotl64(h, 11) * P1;
  }
  h ^= h >> 33;
  h *= P2;
  h ^= h >> 29;
  h *= P3;
  h ^= h >> 32;
  return h;
}

// One chain (lane q of the quad) over n stripes starting at p (p is 8-byte aligned: extents start 256-byte aligned
// in every caller, and every extent but the last is a multiple of 32 bytes). Each block of kBlock stripes is loaded
// (kBlock independent 8-byte loads per lane in flight), then run. The loads go through the global address space (the
// pointer is cast to it): a generic pointer makes flat loads, which also count on the LDS counter and cost 4 % here.
// They are ordinary cached loads: the quad reads 32 bytes of a 128-byte line per stripe and the next three stripes
// read the rest of it, so the line must stay in the CU's cache (a streaming hint that skips it cost 40 % on gfx950).
//
// Measured on one 336 MiB unit (8 KiB segments): this loop reads at 5.8 TB/s, 95 % of what a fully coalesced 16-byte
// streaming read of the same bytes reaches in one launch (6.1 TB/s); the rounds alone (no loads) run at 17 TB/s. So
// the kernel is bound by the read, not the multiplies, and neither a software-pipelined nor an LDS-staged variant
// (coalesced 16-byte loads into LDS, chains run from LDS) beat it.
constexpr int kBlock = 16;
typedef __attribute__((address_space(1))) const uint64_t gword_t;
typedef __attribute__((address_space(1))) uint64_t gout_t;

// kCopy: each word read is also stored at the same offset from d (the staged unit's bytes into their arena slot while
// they are hashed: the bytes cross HBM once each way).
template <bool kCopy>
__device__ __forceinline__ uint64_t chain_t(uint64_t v, const unsigned char* p, unsigned char* d, uint64_t n,
                                            uint32_t q) {
  gword_t* w = reinterpret_cast<gword_t*>(reinterpret_cast<uintptr_t>(p)) + q;
  gout_t* o = reinterpret_cast<gout_t*>(reinterpret_cast<uintptr_t>(d)) + q;
  uint64_t s = 0;
  for (; s + kBlock <= n; s += kBlock) {
    uint64_t buf[kBlock];
#pragma unroll
    for (int k = 0; k < kBlock; ++k) buf[k] = w[4 * (s + k)];
    if (kCopy) {
#pragma unroll
      for (int k = 0; k < kBlock; ++k) o[4 * (s + k)] = buf[k];
    }
#pragma unroll
    for (int k = 0; k < kBlock; ++k) v = xround(v, buf[k]);
  }
  for (; s < n; ++s) {
    const uint64_t x = w[4 * s];
    if (kCopy) o[4 * s] = x;
    v = xround(v, x);
  }
  return v;
}
__device__ __forceinline__ uint64_t chain(uint64_t v, const unsigned char* p, uint64_t n, uint32_t q) {
  return chain_t<false>(v, p, nullptr, n, q);
}

__device__ __forceinline__ void init_acc(uint64_t v[4]) {
  v[0] = P1 + P2;
  v[1] = P2;
  v[2] = 0;
  v[3] = 0 - P1;
}

__global__ __launch_bounds__(256) void digest_kernel(const TsaUnit* __restrict__ units, uint32_t n,
                                                     uint64_t* __restrict__ out) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t u = gid >> 2, q = gid & 3u;
  const bool live = u < n;
  uint64_t acc[4];
  init_acc(acc);
  uint64_t v = acc[q];
  uint64_t total = 0;
  const unsigned char* tail = nullptr;
  uint32_t tail_len = 0;
  if (live) {
    const TsaUnit un = units[u];
    for (uint32_t e = 0; e < un.n_ext; ++e) {
      const unsigned char* p = static_cast<const unsigned char*>(un.ext[e].ptr);
      const uint64_t b = un.ext[e].bytes;
      const uint64_t stripes = b / 32;
      v = chain(v, p, stripes, q);
      total += b;
      if (e + 1 == un.n_ext) {
        tail = p + stripes * 32;
        tail_len = uint32_t(b - stripes * 32);
      }
    }
  }
  // the quad's accumulators to its lane 0 (all lanes of the wave take part in the shuffles)
  uint64_t all[4];
  const uint32_t base = threadIdx.x & ~3u;
#pragma unroll
  for (int k = 0; k < 4; ++k) all[k] = __shfl(v, int(base + k), 64);
  if (live && q == 0) out[u] = xfinal(all, total, tail, tail_len);
}

// Both verify kernels are held to 8 waves per SIMD (at most 64 VGPRs): unbounded, the compiler spends registers on
// scheduling (83-86 VGPRs, 5 waves per SIMD) and the kernel has 5/8 of the loads in flight it could; bounded it needs
// 52-58 with no spill, and one 336 MiB unit's check (3 parts, 2 KiB segments, timed alone in a fresh process) ran
// 67 -> 62 us.
#define TSA_VERIFY_BOUNDS __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))

// One (unit, segment) per quad. seg_first is the prefix sum of segments over the launch's units (ascending).
__global__ TSA_VERIFY_BOUNDS void verify_kernel(const TsaVerifyUnit* __restrict__ units, uint32_t n_units,
                                                     uint64_t n_segments, uint64_t seg_bytes,
                                                     uint32_t* __restrict__ fail) {
  const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t s = gid >> 2;
  const uint32_t q = uint32_t(gid & 3u);
  const bool live = s < n_segments;
  uint32_t ui = 0;
  if (live) {  // the unit holding global segment s (units sorted by seg_first)
    uint32_t lo = 0, hi = n_units;
    while (hi - lo > 1) {
      const uint32_t mid = (lo + hi) / 2;
      if (units[mid].seg_first <= s) lo = mid;
      else hi = mid;
    }
    ui = lo;
  }
  uint64_t v = 0;
  bool last = false, check_state = false;
  uint64_t local = 0, total = 0;
  const unsigned char* tail = nullptr;
  uint32_t tail_len = 0;
  const TsaVerifyUnit* un = units + ui;
  if (live) {
    local = s - un->seg_first;  // the unit's segment index (its checkpoint index)
    // the extent and the segment inside it
    uint64_t k = local;
    uint32_t e = 0;
    uint64_t off = 0, stripes = 0;
    for (; e < un->n_ext; ++e) {
      const uint64_t b = un->ext[e].bytes;
      const bool last_ext = e + 1 == un->n_ext;
      const uint64_t span = last_ext ? b / 32 * 32 : b;
      uint64_t nseg = (span + seg_bytes - 1) / seg_bytes;
      if (last_ext && nseg == 0) nseg = 1;
      if (k < nseg) {
        off = k * seg_bytes;
        const uint64_t end = off + seg_bytes < span ? off + seg_bytes : span;
        stripes = (end - off) / 32;
        last = last_ext && k + 1 == nseg;
        if (last) {
          tail = static_cast<const unsigned char*>(un->ext[e].ptr) + span;
          tail_len = uint32_t(b - span);
        }
        break;
      }
      k -= nseg;
    }
    if (e == un->n_ext) {  // the launch's prefix sums disagree with the extents: reported, nothing read
      if (q == 0) atomicOr(fail + ui, 2u);
      return;  // (the whole quad: its lanes share s)
    }
    v = un->states[4 * local + q];
    v = chain(v, static_cast<const unsigned char*>(un->ext[e].ptr) + off, stripes, q);
    total = un->total;
    check_state = !last;
  }
  uint64_t all[4];
  const uint32_t base = threadIdx.x & ~3u;
#pragma unroll
  for (int k = 0; k < 4; ++k) all[k] = __shfl(v, int(base + k), 64);
  if (!live) return;
  if (check_state) {
    if (v != un->states[4 * (local + 1) + q]) atomicOr(fail + ui, 1u);
  } else if (q == 0) {
    if (xfinal(all, total, tail, tail_len) != un->digest) atomicOr(fail + ui, 1u);
  }
}

// Device-gated verify: one quad per (unit, segment) of the launch's units, all of the arena's part shape. kCopy (the
// staged units' fused scatter): unit u's bytes are read from src + u x unit_bytes, where its parts lie back to back,
// and written to their arena slot as they are hashed; the last segment's lane 0 also moves the unit's tail.
template <bool kCopy>
__device__ __forceinline__ void dg_verify_body(const DgVerifyLaunch& a, const unsigned char* src) {
  const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t s = gid >> 2;
  const uint32_t q = uint32_t(gid & 3u);
  const bool live = s < uint64_t(a.n) * a.unit_segs;
  uint64_t v = 0, local = 0, key = 0;
  uint32_t u = 0;
  bool last = false;
  const unsigned char* tail = nullptr;
  uint32_t tail_len = 0;
  if (live) {
    u = uint32_t(s / a.unit_segs);
    local = s - uint64_t(u) * a.unit_segs;
    uint64_t k = local;
    uint32_t p = 0;
    uint64_t src_off = uint64_t(u) * a.unit_bytes;  // (kCopy) the part's first byte in src
    while (p + 1 < a.n_parts && k >= a.part_segs[p]) {
      k -= a.part_segs[p];
      src_off += a.part_bytes[p++];
    }
    const bool last_part = p + 1 == a.n_parts;
    const uint64_t span = last_part ? a.part_bytes[p] / 32 * 32 : a.part_bytes[p];
    const uint64_t off = k * a.seg_bytes;
    const uint64_t end = off + a.seg_bytes < span ? off + a.seg_bytes : span;
    const unsigned char* base = a.arena[p] + uint64_t(a.slots[u]) * a.part_bytes[p];
    const unsigned char* from = kCopy ? src + src_off : base;
    last = last_part && k + 1 == a.part_segs[p];
    if (last) {
      tail = from + span;
      tail_len = uint32_t(a.part_bytes[p] - span);
      if (kCopy && q == 0)
        for (uint32_t i = 0; i < tail_len; ++i) const_cast<unsigned char*>(base)[span + i] = tail[i];
    }
    key = a.keys[u];
    v = a.ckpt[(key * a.unit_segs + local) * 4 + q];
    v = chain_t<kCopy>(v, from + off, const_cast<unsigned char*>(base) + off, end > off ? (end - off) / 32 : 0, q);
  }
  uint64_t all[4];
  const uint32_t base4 = threadIdx.x & ~3u;
#pragma unroll
  for (int k = 0; k < 4; ++k) all[k] = __shfl(v, int(base4 + k), 64);
  bool bad = false;
  if (live) {
    if (!last) bad = v != a.ckpt[(key * a.unit_segs + local + 1) * 4 + q];
    else if (q == 0) bad = xfinal(all, a.unit_bytes, tail, tail_len) != a.digests[key];
  }
  if (bad) {
    atomicOr(a.fail + u, 1u);
    if (a.abort) {  // the gate: the token fails before the layer's ready word is written
      if (atomicCAS(a.err_code, 0u, a.err) == 0u) atomicExch(a.err_aux, a.aux);
      atomicExch(a.abort, 1u);
    }
    __threadfence();  // performed before this thread reaches the barrier below (and so before its group counts)
  }
  if (!a.done_count) return;
  // publication by the last workgroup to finish. Only a failing thread has words to release, and it did so above;
  // the count itself is relaxed (a release fence per workgroup is an L2 write-back each on this chip).
  __syncthreads();
  if (threadIdx.x != 0) return;
  if (__hip_atomic_fetch_add(a.done_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != gridDim.x - 1u) return;
  if (a.slot_of)
    for (uint32_t i = 0; i < a.n; ++i)
      __hip_atomic_store(a.slot_of + a.keys[i], a.slots[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(a.done_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a.ready) {
    __threadfence_system();
    __hip_atomic_store(a.ready + a.ready_g, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

__global__ TSA_VERIFY_BOUNDS void dg_verify_kernel(const DgVerifyLaunch a) { dg_verify_body<false>(a, nullptr); }
__global__ TSA_VERIFY_BOUNDS void dg_scatter_verify_kernel(const DgVerifyLaunch a, const unsigned char* src) {
  dg_verify_body<true>(a, src);
}

}  // namespace dev

int launch_digest(const TsaUnit* units_dev, uint32_t n, uint64_t* out_dev, hipStream_t stream) {
  if (n == 0) return 0;
  const uint32_t threads = 256;
  const uint64_t lanes = uint64_t(n) * 4;
  const uint32_t blocks = uint32_t((lanes + threads - 1) / threads);
  hipLaunchKernelGGL(dev::digest_kernel, dim3(blocks), dim3(threads), 0, stream, units_dev, n, out_dev);
  return int(hipGetLastError());
}

int launch_dg_verify(const DgVerifyLaunch& a, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (a.n == 0 || a.unit_segs == 0) return 0;
  if (a.n > kDgVerifyMax || a.n_parts == 0 || a.n_parts > 4) return int(hipErrorInvalidValue);
  const uint32_t threads = 256;
  const uint64_t blocks = (uint64_t(a.n) * a.unit_segs * 4 + threads - 1) / threads;
  if (blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  if (start && stop)  // the events take the dispatch's own begin and end timestamps
    hipExtLaunchKernelGGL(dev::dg_verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, start, stop, 0, a);
  else
    hipLaunchKernelGGL(dev::dg_verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, a);
  return int(hipGetLastError());
}

int launch_dg_scatter_verify(const DgVerifyLaunch& a, const void* src, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop) {
  if (a.n == 0 || a.unit_segs == 0) return 0;
  if (a.n > kDgVerifyMax || a.n_parts == 0 || a.n_parts > 4 || !src) return int(hipErrorInvalidValue);
  const uint32_t threads = 256;
  const uint64_t blocks = (uint64_t(a.n) * a.unit_segs * 4 + threads - 1) / threads;
  if (blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  const unsigned char* s = static_cast<const unsigned char*>(src);
  if (start && stop)
    hipExtLaunchKernelGGL(dev::dg_scatter_verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, start, stop,
                          0, a, s);
  else
    hipLaunchKernelGGL(dev::dg_scatter_verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, a, s);
  return int(hipGetLastError());
}

int launch_verify(const TsaVerifyUnit* units_dev, uint32_t n_units, uint64_t n_segments, uint64_t seg_bytes,
                  uint32_t* fail_dev, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (n_units == 0 || n_segments == 0) return 0;
  const uint32_t threads = 256;
  const uint64_t blocks = (n_segments * 4 + threads - 1) / threads;
  if (blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  if (start && stop)  // the events take the dispatch's own begin and end timestamps
    hipExtLaunchKernelGGL(dev::verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, start, stop, 0,
                          units_dev, n_units, n_segments, seg_bytes, fail_dev);
  else
    hipLaunchKernelGGL(dev::verify_kernel, dim3(uint32_t(blocks)), dim3(threads), 0, stream, units_dev, n_units,
                       n_segments, seg_bytes, fail_dev);
  return int(hipGetLastError());
}

}  // namespace tsa
