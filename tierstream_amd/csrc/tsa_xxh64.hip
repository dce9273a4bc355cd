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

// ---- The LDS-streamed check (2 KiB segments in 16-byte aligned memory) ----
//
// The chain loop above reads 8 bytes per lane at a 32-byte stride: every load instruction of a wave touches 16 lines
// (one per quad) and relies on the CU cache to keep each line for the next three. Here every wave streams its 16
// segments through LDS instead, with direct-to-LDS 16-byte loads (global_load_lds_dwordx4): 64 lanes fill 1 KiB of
// LDS per instruction, eight whole 128-byte lines, with the non-temporal hint (the bytes are read once). The quads
// then run their chains from LDS. Measured on one 336 MiB unit: 52-53 us against 58 us for the chain loop, the same
// as a plain coalesced 16-byte streaming read of the unit.
//
// Per wave: a chunk is 256 bytes (8 stripes) of each of its 16 segments, 4 KiB, four loads: load k carries segments
// 4k..4k+3, lanes 16i..16i+15 the 16 pieces of segment 4k+i. A segment's stripes are rotated by (its quad index mod 8)
// inside its 256 bytes, so that the wave's ds_read_b64 of one stripe of all 16 segments spreads over the LDS banks.
// Two chunk buffers per wave: the loads of chunk c+2 are issued when chunk c has been hashed. The loads are inline
// assembly, so the compiler neither waits for them nor knows them; each chunk waits for its own loads with an explicit
// vmcnt (loads complete in order) and the buffer is reused only after its LDS reads have completed (lgkmcnt 0).
// Lanes whose piece lies past their segment's stripes load the segment's first bytes instead (never out of bounds),
// and every wave issues the same number of loads, which the vmcnt counts rely on.
constexpr uint32_t kLdsSegBytes = 2048;  // 8 chunks of 256 bytes per segment
constexpr uint32_t kLdsChunks = kLdsSegBytes / 256;
constexpr uint32_t kLdsWaveBytes = 2 * 4096;  // two chunk buffers

__device__ __forceinline__ void lds_load16(const unsigned char* g, uint32_t lds_addr) {
  uint32_t save;  // M0 (the LDS destination) is restored for the compiler; s_nop: an M0 write before an LDS load
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0"
      : "=&s"(save)
      : "v"(g), "s"(lds_addr)
      : "memory");
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 gu32x4_t;

template <int N>
__device__ __forceinline__ void wait_loads() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The wave's 16 quads (lane = 4 j + q) each hash `stripes` (<= 64) stripes from `from` (16-byte aligned) starting at
// state v; all 64 lanes must call it. lds: the wave's kLdsWaveBytes of LDS (its address and its 32-bit LDS offset).
// kCopy: every stripe is also written to the same offset from `to` (16-byte aligned), each lane storing the 16-byte
// pieces it loaded, from LDS, once they have landed.
template <bool kCopy>
__device__ __forceinline__ uint64_t lds_chain_t(uint64_t v, const unsigned char* from, unsigned char* to,
                                                uint32_t stripes, const unsigned char* lds, uint32_t lds_off) {
  const uint32_t lane = threadIdx.x & 63u, q = lane & 3u, j = lane >> 2;
  const uint32_t i = lane >> 4, m = lane & 15u;
  const unsigned char* src[4];
  unsigned char* dst[4];
  uint32_t n[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // the lane loads for segment 4k + i (quad 4k + i's lane 0 holds its source)
    const int owner = int((4 * k + i) * 4);
    src[k] = reinterpret_cast<const unsigned char*>(
        __shfl(static_cast<unsigned long long>(reinterpret_cast<uintptr_t>(from)), owner, 64));
    if (kCopy)
      dst[k] = reinterpret_cast<unsigned char*>(
          __shfl(static_cast<unsigned long long>(reinterpret_cast<uintptr_t>(to)), owner, 64));
    n[k] = uint32_t(__shfl(int(stripes), owner, 64));
  }
  auto piece = [&](uint32_t c, uint32_t k) {  // the global stripe this lane's piece of load k of chunk c holds
    return (((m >> 1) - ((4 * k + i) & 7u)) & 7u) + 8 * c;
  };
  auto issue = [&](uint32_t c) {
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
      const uint32_t g = piece(c, k);
      const unsigned char* at = g < n[k] ? src[k] + g * 32 + (m & 1u) * 16 : src[k];
      lds_load16(at, lds_off + (c & 1u) * 4096 + k * 1024);
    }
  };
  issue(0);
  issue(1);
  // v (the segment's checkpoint) arrives here: the compiler's wait for it (a vmcnt(0), which also covers the two
  // chunks just issued) then sits before the loop, not inside it at every use of the loop-carried state
  asm volatile("" : "+v"(v));
  const uint32_t rot = j & 7u;
  const unsigned char* rd = lds + (j >> 2) * 1024 + (j & 3u) * 256 + q * 8;
  auto hash = [&](uint32_t c) {
    if (kCopy) {  // the lane's own four pieces, as they landed in LDS
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t g = piece(c, k);
        const u32x4 x = *reinterpret_cast<const u32x4*>(lds + (c & 1u) * 4096 + k * 1024 + lane * 16);
        if (g < n[k])  // (a global store: a generic one would also count on the LDS counter waited on below)
          *reinterpret_cast<gu32x4_t*>(reinterpret_cast<uintptr_t>(dst[k] + g * 32 + (m & 1u) * 16)) = x;
      }
    }
    const unsigned char* b = rd + (c & 1u) * 4096;
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t) {
      const uint64_t x = *reinterpret_cast<const uint64_t*>(b + ((t + rot) & 7u) * 32);
      const uint64_t r = xround(v, x);
      v = 8 * c + t < stripes ? r : v;
    }
  };
  // chunks 0 .. kLdsChunks - 3: the next chunk's four loads may still be in flight (vmcnt 4 also holds with the copy's
  // stores among them: loads complete in order among themselves); then this buffer is refilled
#pragma unroll 2
  for (uint32_t c = 0; c + 2 < kLdsChunks; ++c) {
    wait_loads<4>();
    hash(c);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this buffer's LDS reads are done before it is refilled
    issue(c + 2);
  }
  wait_loads<4>();
  hash(kLdsChunks - 2);
  wait_loads<0>();
  hash(kLdsChunks - 1);
  return v;
}
__device__ __forceinline__ uint64_t lds_chain(uint64_t v, const unsigned char* from, uint32_t stripes,
                                              const unsigned char* lds, uint32_t lds_off) {
  return lds_chain_t<false>(v, from, nullptr, stripes, lds, lds_off);
}

// The chain-loop kernels (dg_verify_kernel, dg_scatter_verify_kernel) are held to 8 waves per SIMD (at most 64
// VGPRs): unbounded, the compiler spends registers on scheduling (83-86 VGPRs, 5 waves per SIMD) and the kernel has
// 5/8 of the loads in flight it could; bounded it needs 52-58 with no spill, and one 336 MiB unit's check (3 parts,
// 2 KiB segments, timed alone in a fresh process) ran 67 -> 62 us. The LDS-streamed kernels keep their loads in LDS,
// not in registers, and run 5 waves per SIMD (their 32 KiB of LDS per workgroup).
#define TSA_VERIFY_BOUNDS __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))

// One (unit, segment) per quad. seg_first is the prefix sum of segments over the launch's units (ascending). A wave
// whose segments are all 2 KiB pieces of 16-byte aligned extents, each of at least one stripe, streams them through
// LDS (lds_chain); any other wave (other segment sizes, unaligned extents, a last extent under 32 bytes) runs the
// chain loop. The choice is the wave's: all its lanes take one path.
__global__ __launch_bounds__(256) void verify_kernel(const TsaVerifyUnit* __restrict__ units, uint32_t n_units,
                                                     uint64_t n_segments, uint64_t seg_bytes,
                                                     uint32_t* __restrict__ fail) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[4 * kLdsWaveBytes];
  const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t s = gid >> 2;
  const uint32_t q = uint32_t(gid & 3u);
  bool live = s < n_segments;
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
  bool last = false;
  uint64_t local = 0, total = 0, stripes = 0;
  const unsigned char* from = nullptr;
  const unsigned char* tail = nullptr;
  uint32_t tail_len = 0;
  const TsaVerifyUnit* un = units + ui;
  if (live) {
    local = s - un->seg_first;  // the unit's segment index (its checkpoint index)
    // the extent and the segment inside it
    uint64_t k = local;
    uint32_t e = 0;
    for (; e < un->n_ext; ++e) {
      const uint64_t b = un->ext[e].bytes;
      const bool last_ext = e + 1 == un->n_ext;
      const uint64_t span = last_ext ? b / 32 * 32 : b;
      uint64_t nseg = (span + seg_bytes - 1) / seg_bytes;
      if (last_ext && nseg == 0) nseg = 1;
      if (k < nseg) {
        const uint64_t off = k * seg_bytes;
        const uint64_t end = off + seg_bytes < span ? off + seg_bytes : span;
        stripes = (end - off) / 32;
        from = static_cast<const unsigned char*>(un->ext[e].ptr) + off;
        last = last_ext && k + 1 == nseg;
        if (last) {
          tail = static_cast<const unsigned char*>(un->ext[e].ptr) + span;
          tail_len = uint32_t(b - span);
        }
        break;
      }
      k -= nseg;
    }
    if (e == un->n_ext) {  // the launch's prefix sums disagree with the extents: reported, nothing read or checked
      if (q == 0) atomicOr(fail + ui, 2u);
      live = false;
    } else {
      v = un->states[4 * local + q];
      total = un->total;
    }
  }
  const uint64_t lanes_live = __ballot(live);
  if (lanes_live == 0) return;  // (the whole wave)
  const bool lds_path = seg_bytes == kLdsSegBytes &&
                        __all(!live || ((reinterpret_cast<uintptr_t>(from) & 15u) == 0 && stripes >= 1));
  if (lds_path) {
    // a dead lane streams a live lane's segment (in bounds) and hashes none of it
    const unsigned char* any = reinterpret_cast<const unsigned char*>(__shfl(
        static_cast<unsigned long long>(reinterpret_cast<uintptr_t>(from)), __ffsll((long long)lanes_live) - 1, 64));
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    unsigned char* mine = lds + wave * kLdsWaveBytes;
    const uint32_t mine_off =
        uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)(mine)));
    v = lds_chain(v, live ? from : any, live ? uint32_t(stripes) : 0u, mine, mine_off);
  } else if (live) {
    v = chain(v, from, stripes, q);
  }
  uint64_t all[4];
  const uint32_t base = threadIdx.x & ~3u;
#pragma unroll
  for (int k = 0; k < 4; ++k) all[k] = __shfl(v, int(base + k), 64);
  if (!live) return;
  if (!last) {
    if (v != un->states[4 * (local + 1) + q]) atomicOr(fail + ui, 1u);
  } else if (q == 0) {
    if (xfinal(all, total, tail, tail_len) != un->digest) atomicOr(fail + ui, 1u);
  }
}

// Device-gated verify: one quad per (unit, segment) of the launch's units, all of the arena's part shape. kCopy (the
// staged units' fused scatter): unit u's bytes are read from src + u x unit_bytes, where its parts lie back to back,
// and written to their arena slot as they are hashed; the last segment's lane 0 also moves the unit's tail.
struct DgSeg {
  uint64_t v = 0, local = 0, key = 0;
  uint32_t u = 0, stripes = 0, tail_len = 0;
  bool live = false, last = false;
  const unsigned char* from = nullptr;  // the segment's first byte (where it is read)
  unsigned char* to = nullptr;          // (kCopy) where it is written
  const unsigned char* tail = nullptr;
};

// The launch's tables (keys, slots, the parts' arrays) are kernel arguments. Indexed by a per-lane value they become
// per-lane loads from the argument segment; so the wave reads its first lane's unit with scalar loads (per-lane
// loads only run in a wave that straddles two units) and the part's fields are carried along the walk over the parts
// with constant indices, which keeps every other read of the arguments a scalar load.

template <bool kCopy>
__device__ __forceinline__ DgSeg dg_segment(const DgVerifyLaunch& a, const unsigned char* src, uint64_t s, uint32_t q) {
  DgSeg g;
  g.live = s < uint64_t(a.n) * a.unit_segs;
  const uint32_t u_lane = g.live ? uint32_t(s / a.unit_segs) : a.n - 1;  // (a dead lane sides with the last unit)
  const uint32_t u0 = __builtin_amdgcn_readfirstlane(u_lane);
  uint32_t key = a.keys[u0];  // scalar loads, here (the empty asm takes them as scalars before any branch)
  int32_t slot = a.slots[u0];
  asm volatile("" ::"s"(key), "s"(slot));
  if (!__all(u_lane == u0)) {  // only in a wave that straddles two units
    key = a.keys[u_lane];
    slot = a.slots[u_lane];
  }
  if (!g.live) return g;
  g.u = u_lane;
  g.local = s - uint64_t(g.u) * a.unit_segs;
  uint64_t k = g.local;
  uint32_t p = 0;
  uint64_t src_off = uint64_t(g.u) * a.unit_bytes;  // (kCopy) the part's first byte in src
  uint64_t pbytes = a.part_bytes[0], psegs = a.part_segs[0];
  const unsigned char* parena = a.arena[0];
#pragma unroll
  for (uint32_t i = 0; i + 1 < 4; ++i) {
    if (p == i && i + 1 < a.n_parts && k >= a.part_segs[i]) {
      k -= a.part_segs[i];
      src_off += a.part_bytes[i];
      p = i + 1;
      pbytes = a.part_bytes[i + 1];
      psegs = a.part_segs[i + 1];
      parena = a.arena[i + 1];
    }
  }
  const bool last_part = p + 1 == a.n_parts;
  const uint64_t span = last_part ? pbytes / 32 * 32 : pbytes;
  const uint64_t off = k * a.seg_bytes;
  const uint64_t end = off + a.seg_bytes < span ? off + a.seg_bytes : span;
  unsigned char* base = const_cast<unsigned char*>(parena) + uint64_t(slot) * pbytes;
  const unsigned char* from = kCopy ? src + src_off : base;
  g.last = last_part && k + 1 == psegs;
  if (g.last) {
    g.tail = from + span;
    g.tail_len = uint32_t(pbytes - span);
    if (kCopy && q == 0)
      for (uint32_t i = 0; i < g.tail_len; ++i) base[span + i] = g.tail[i];
  }
  g.key = key;
  g.v = a.ckpt[(g.key * a.unit_segs + g.local) * 4 + q];
  g.from = from + off;
  g.to = base + off;
  g.stripes = end > off ? uint32_t((end - off) / 32) : 0;
  return g;
}

// The segment's check (the next checkpoint, or for the unit's last segment the digest) and the gate.
__device__ __forceinline__ void dg_finish(const DgVerifyLaunch& a, const DgSeg& g, uint64_t v, uint32_t q) {
  uint64_t all[4];
  const uint32_t base4 = threadIdx.x & ~3u;
#pragma unroll
  for (int k = 0; k < 4; ++k) all[k] = __shfl(v, int(base4 + k), 64);
  bool bad = false;
  if (g.live) {
    if (!g.last) bad = v != a.ckpt[(g.key * a.unit_segs + g.local + 1) * 4 + q];
    else if (q == 0) bad = xfinal(all, a.unit_bytes, g.tail, g.tail_len) != a.digests[g.key];
  }
  if (bad) {
    atomicOr(a.fail + g.u, 1u);
    if (a.abort) {  // the gate: the token fails before the layer's ready word is written
      if (atomicCAS(a.err_code, 0u, a.err) == 0u) atomicExch(a.err_aux, a.aux);
      atomicExch(a.abort, 1u);
    }
  }
}

// Publication after a check, launched behind it on its stream (so it starts once every workgroup of the check has
// ended and its writes, a failing one's abort among them, are visible): the landed units' slot entries, then the
// layer's ready word. Counting the check's workgroups in the check itself instead (an agent-scope atomic per
// workgroup, the last one publishing) cost 8 us per 336 MiB check on this chip: each atomic waits in the memory
// queues behind the check's own reads and holds its workgroup's slot.
__global__ __launch_bounds__(64) void dg_publish_kernel(const DgVerifyLaunch a) {
  if (threadIdx.x != 0) return;
  if (a.slot_of)
    for (uint32_t i = 0; i < a.n; ++i)
      __hip_atomic_store(a.slot_of + a.keys[i], a.slots[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a.ready) {
    __threadfence_system();
    __hip_atomic_store(a.ready + a.ready_g, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

template <bool kCopy>
__device__ __forceinline__ void dg_verify_body(const DgVerifyLaunch& a, const unsigned char* src) {
  const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint32_t q = uint32_t(gid & 3u);
  const DgSeg g = dg_segment<kCopy>(a, src, gid >> 2, q);
  uint64_t v = 0;
  if (g.live) v = chain_t<kCopy>(g.v, g.from, g.to, g.stripes, q);
  dg_finish(a, g, v, q);
}

__global__ TSA_VERIFY_BOUNDS void dg_verify_kernel(const DgVerifyLaunch a) { dg_verify_body<false>(a, nullptr); }
__global__ TSA_VERIFY_BOUNDS void dg_scatter_verify_kernel(const DgVerifyLaunch a, const unsigned char* src) {
  dg_verify_body<true>(a, src);
}

template <bool kCopy>
__device__ __forceinline__ void dg_verify_lds_body(const DgVerifyLaunch& a, const unsigned char* src) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[4 * kLdsWaveBytes];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char* mine = lds + wave * kLdsWaveBytes;
  const uint32_t mine_off = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)(mine)));
  const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint32_t q = uint32_t(gid & 3u);
  const DgSeg g = dg_segment<kCopy>(a, src, gid >> 2, q);
  // a dead quad (past the launch's segments) streams unit 0's first bytes and hashes (and writes) none of them
  const unsigned char* from = g.live ? g.from : kCopy ? src : a.arena[0] + uint64_t(a.slots[0]) * a.part_bytes[0];
  const uint64_t v = lds_chain_t<kCopy>(g.v, from, g.to, g.live ? g.stripes : 0u, mine, mine_off);
  dg_finish(a, g, v, q);
}
__global__ __launch_bounds__(256) void dg_verify_lds_kernel(const DgVerifyLaunch a) { dg_verify_lds_body<false>(a, nullptr); }
__global__ __launch_bounds__(256) void dg_scatter_verify_lds_kernel(const DgVerifyLaunch a, const unsigned char* src) {
  dg_verify_lds_body<true>(a, src);
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

// The LDS-streamed kernel needs 2 KiB segments and every part of every unit of the launch 16-byte aligned and at
// least 16 bytes long (a lane with nothing to load reads its segment's first 16 bytes).
static bool dg_lds_shape(const DgVerifyLaunch& a) {
  if (a.seg_bytes != dev::kLdsSegBytes) return false;
  for (uint32_t p = 0; p < a.n_parts; ++p) {
    if (reinterpret_cast<uintptr_t>(a.arena[p]) % 16 != 0 || a.part_bytes[p] < 16) return false;
    if (a.part_bytes[p] % 16 == 0) continue;
    for (uint32_t u = 0; u < a.n; ++u)
      if (uint64_t(a.slots[u]) * a.part_bytes[p] % 16 != 0) return false;
  }
  return true;
}

static int launch_publish(const DgVerifyLaunch& a, hipStream_t stream) {
  if (!a.publish || (!a.slot_of && !a.ready)) return 0;
  hipLaunchKernelGGL(dev::dg_publish_kernel, dim3(1), dim3(64), 0, stream, a);
  return int(hipGetLastError());
}

int launch_dg_verify(const DgVerifyLaunch& a, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (a.n == 0 || a.unit_segs == 0) return 0;
  if (a.n > kDgVerifyMax || a.n_parts == 0 || a.n_parts > 4) return int(hipErrorInvalidValue);
  const uint32_t threads = 256;
  const uint64_t blocks = (uint64_t(a.n) * a.unit_segs * 4 + threads - 1) / threads;
  if (blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  auto* k = dg_lds_shape(a) ? dev::dg_verify_lds_kernel : dev::dg_verify_kernel;
  if (start && stop)  // the events take the dispatch's own begin and end timestamps
    hipExtLaunchKernelGGL(k, dim3(uint32_t(blocks)), dim3(threads), 0, stream, start, stop, 0, a);
  else
    hipLaunchKernelGGL(k, dim3(uint32_t(blocks)), dim3(threads), 0, stream, a);
  const int e = int(hipGetLastError());
  return e ? e : launch_publish(a, stream);
}

// The fused kernel's LDS form also needs the staged bytes 16-byte aligned: src and every part of every staged unit.
static bool dg_scatter_lds_shape(const DgVerifyLaunch& a, const void* src) {
  if (!dg_lds_shape(a) || reinterpret_cast<uintptr_t>(src) % 16 != 0) return false;
  for (uint32_t p = 0; p < a.n_parts; ++p)
    if (a.part_bytes[p] % 16 != 0) return false;
  return true;
}

int launch_dg_scatter_verify(const DgVerifyLaunch& a, const void* src, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop) {
  if (a.n == 0 || a.unit_segs == 0) return 0;
  if (a.n > kDgVerifyMax || a.n_parts == 0 || a.n_parts > 4 || !src) return int(hipErrorInvalidValue);
  const uint32_t threads = 256;
  const uint64_t blocks = (uint64_t(a.n) * a.unit_segs * 4 + threads - 1) / threads;
  if (blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  const unsigned char* s = static_cast<const unsigned char*>(src);
  auto* k = dg_scatter_lds_shape(a, src) ? dev::dg_scatter_verify_lds_kernel : dev::dg_scatter_verify_kernel;
  if (start && stop)
    hipExtLaunchKernelGGL(k, dim3(uint32_t(blocks)), dim3(threads), 0, stream, start, stop, 0, a, s);
  else
    hipLaunchKernelGGL(k, dim3(uint32_t(blocks)), dim3(threads), 0, stream, a, s);
  const int e = int(hipGetLastError());
  return e ? e : launch_publish(a, stream);
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
