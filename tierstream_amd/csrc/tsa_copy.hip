// Byte-moving kernels over HBM: the unit scatter (a staged unit's parts into their arena slots) and the synthetic
// byte generator the benchmarks and tests fill sources with.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tsa_device.hpp"

namespace tsa {
namespace dev {

// ---- scatter ------------------------------------------------------------------------------------------------------
// The launch is a flat list of 16 KiB blocks: job j owns blocks [block_first_j, block_first_j + blocks_j), part by
// part. A workgroup of 256 lanes moves one block: 4 x 16 bytes per lane, each load and store a 128-bit access, lanes
// adjacent in memory (a wavefront covers 1 KiB per instruction). Consecutive workgroups take consecutive blocks, so a
// part streams through HBM in order. Reads are non-temporal (each byte is read once); stores are plain (the engine reads
// the slot next).
constexpr uint32_t kBlock = TSA_SCATTER_BLOCK_BYTES;
constexpr uint32_t kThreads = 256;
constexpr uint32_t kPerLane = kBlock / (16 * kThreads);  // 4

__global__ __launch_bounds__(kThreads) void scatter_kernel(const TsaScatterJob* __restrict__ jobs, uint32_t n_jobs,
                                                           uint64_t n_blocks) {
  const uint64_t blk = blockIdx.x;
  if (blk >= n_blocks) return;
  uint32_t lo = 0, hi = n_jobs;  // the job holding this block
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (jobs[mid].block_first <= blk) lo = mid;
    else hi = mid;
  }
  const TsaScatterJob& j = jobs[lo];
  uint64_t b = blk - j.block_first;
  uint64_t src_off = 0;
  uint32_t p = 0;
  for (; p < j.n_parts; ++p) {
    const uint64_t nb = (j.bytes[p] + kBlock - 1) / kBlock;
    if (b < nb) break;
    b -= nb;
    src_off += j.bytes[p];
  }
  if (p == j.n_parts) return;  // (the host computed block_first from the same bytes: never reached)
  const uint64_t part_bytes = j.bytes[p];
  const uint64_t off = b * kBlock;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* __restrict__ s = reinterpret_cast<const u32x4*>(static_cast<const char*>(j.src) + src_off + off);
  u32x4* __restrict__ d = reinterpret_cast<u32x4*>(static_cast<char*>(j.dst[p]) + off);
  const uint64_t n16 = (part_bytes - off < kBlock ? part_bytes - off : kBlock) / 16;
  u32x4 v[kPerLane];
#pragma unroll
  for (uint32_t k = 0; k < kPerLane; ++k) {
    const uint64_t i = threadIdx.x + uint64_t(k) * kThreads;
    if (i < n16) v[k] = __builtin_nontemporal_load(s + i);
  }
#pragma unroll
  for (uint32_t k = 0; k < kPerLane; ++k) {
    const uint64_t i = threadIdx.x + uint64_t(k) * kThreads;
    if (i < n16) d[i] = v[k];
  }
}

// ---- synthetic bytes ----------------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// Word i of stream `sid` under `seed`: mix64(key + (i + 1) * golden), key = mix64(seed ^ sid * odd).
__device__ __forceinline__ uint64_t word_at(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x007fffffu)) return uint16_t((x >> 16) | 0x40u);  // NaN stays NaN
  x += 0x7fffu + ((x >> 16) & 1u);
  return uint16_t(x >> 16);
}

// Q4 blocks of 18 bytes (kind 2): block b is a little-endian fp16 scale, then 16 bytes of packed 4-bit values. The
// scale is 0x2000 | (low 10 bits of word 3b): exponent field 8, so 2^-7 x (1 + m / 1024), a positive scale in
// [0.0078, 0.0156); the 16 value bytes are words 3b + 1 and 3b + 2, little-endian. Byte j of the stream is byte j % 18
// of block j / 18 (the blocks start at the stream's byte 0).
__device__ __forceinline__ uint32_t q4_byte(uint64_t key, uint64_t j) {
  const uint64_t b = j / 18u;
  const uint32_t o = uint32_t(j - b * 18u);
  if (o < 2u) {
    const uint32_t scale = 0x2000u | uint32_t(word_at(key, 3u * b) & 0x3FFu);
    return (scale >> (8u * o)) & 0xFFu;
  }
  const uint32_t q = o - 2u;
  return uint32_t(word_at(key, 3u * b + 1u + (q >> 3)) >> (8u * (q & 7u))) & 0xFFu;
}

// kind 0: every 8-byte word is word_at(i). kind 1: word i gives two bf16 values (elements 2i, 2i + 1) by Box-Muller:
// u1 = (hi32 + 0.5) / 2^32, u2 = (lo32 + 0.5) / 2^32, r = sigma sqrt(-2 ln u1), (r cos 2 pi u2, r sin 2 pi u2); a
// 64-bit output word then holds elements 4w .. 4w + 3, i.e. source words 2w and 2w + 1. kind 2: Q4 blocks (above).
__global__ __launch_bounds__(256) void synth_kernel(uint64_t* __restrict__ dst, uint64_t n_words, uint64_t key,
                                                    uint64_t first_word, uint32_t kind, float sigma) {
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  for (uint64_t w = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; w < n_words; w += stride) {
    const uint64_t gw = first_word + w;
    uint64_t out;
    if (kind == 0) {
      out = word_at(key, gw);
    } else if (kind == 2) {
      out = 0;
      for (uint32_t k = 0; k < 8u; ++k) out |= uint64_t(q4_byte(key, 8u * gw + k)) << (8u * k);
    } else {
      out = 0;
      for (int h = 0; h < 2; ++h) {
        const uint64_t r = word_at(key, 2 * gw + uint64_t(h));
        const float u1 = (float(uint32_t(r >> 32)) + 0.5f) * 2.3283064365386963e-10f;
        const float u2 = (float(uint32_t(r)) + 0.5f) * 2.3283064365386963e-10f;
        const float rad = sigma * sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.283185307179586f * u2, &sn, &cs);
        const uint64_t pair = uint64_t(bf16_rne(rad * cs)) | uint64_t(bf16_rne(rad * sn)) << 16;
        out |= pair << (32 * h);
      }
    }
    dst[w] = out;
  }
}

}  // namespace dev

int launch_scatter(const TsaScatterJob* jobs_dev, uint32_t n_jobs, uint64_t n_blocks, hipStream_t stream) {
  if (n_jobs == 0 || n_blocks == 0) return 0;
  if (n_blocks > 0x7fffffffull) return int(hipErrorInvalidValue);
  hipLaunchKernelGGL(dev::scatter_kernel, dim3(uint32_t(n_blocks)), dim3(dev::kThreads), 0, stream, jobs_dev, n_jobs,
                     n_blocks);
  return int(hipGetLastError());
}

int launch_synth(void* dst, uint64_t bytes, uint64_t seed, uint64_t stream_id, uint64_t offset, uint32_t kind,
                 float sigma, hipStream_t stream) {
  const uint64_t n_words = bytes / 8;
  if (n_words == 0) return 0;
  const uint64_t key = dev_key(seed, stream_id);
  const uint64_t want = (n_words + 255) / 256;
  const uint32_t blocks = uint32_t(want < 256 * 64 ? want : 256 * 64);  // grid-stride beyond 64 waves per CU
  hipLaunchKernelGGL(dev::synth_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<uint64_t*>(dst), n_words, key,
                     offset / 8, kind, sigma);
  return int(hipGetLastError());
}

}  // namespace tsa
