// SHA-256 as FIPS 180-4 §6.2 states it. The constants are derived at first use, exactly, from their definition
// (§4.2.2, §5.3.3): K[t] = the first 32 fractional bits of the cube root of the t-th prime, H0[i] = those of the square
// root of the i-th prime, each an integer root of p << 96 (resp. p << 64) taken mod 2^32.
#include "sha256.hpp"

#include <cstdint>
#include <cstring>

namespace tsa {
namespace {

using u128 = unsigned __int128;

uint64_t iroot(u128 v, int k) {  // floor(v^(1/k)), k = 2 or 3, v < 2^120
  uint64_t lo = 0, hi = uint64_t(1) << 41;
  while (lo < hi) {
    const uint64_t mid = lo + (hi - lo + 1) / 2;
    u128 p = mid;
    for (int i = 1; i < k; ++i) p *= mid;
    if (p <= v) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

struct Consts {
  uint32_t K[64], H0[8];
  Consts() {
    int n = 0;
    for (uint32_t p = 2; n < 64; ++p) {
      bool prime = true;
      for (uint32_t d = 2; d * d <= p; ++d)
        if (p % d == 0) prime = false;
      if (!prime) continue;
      K[n] = uint32_t(iroot(u128(p) << 96, 3));
      if (n < 8) H0[n] = uint32_t(iroot(u128(p) << 64, 2));
      ++n;
    }
  }
};

const Consts& consts() {
  static const Consts c;
  return c;
}

inline uint32_t rotr(uint32_t x, int n) { return x >> n | x << (32 - n); }

void block(uint32_t h[8], const unsigned char* b, const uint32_t* K) {
  uint32_t w[64];
  for (int t = 0; t < 16; ++t)
    w[t] = uint32_t(b[4 * t]) << 24 | uint32_t(b[4 * t + 1]) << 16 | uint32_t(b[4 * t + 2]) << 8 | b[4 * t + 3];
  for (int t = 16; t < 64; ++t) {
    const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
    const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
    w[t] = w[t - 16] + s0 + w[t - 7] + s1;
  }
  uint32_t a = h[0], bb = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
  for (int t = 0; t < 64; ++t) {
    const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[t] + w[t];
    const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
    hh = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = bb;
    bb = a;
    a = t1 + t2;
  }
  h[0] += a, h[1] += bb, h[2] += c, h[3] += d, h[4] += e, h[5] += f, h[6] += g, h[7] += hh;
}

}  // namespace

std::string sha256(const void* data, size_t n) {
  const Consts& k = consts();
  uint32_t h[8];
  std::memcpy(h, k.H0, sizeof h);
  const auto* p = static_cast<const unsigned char*>(data);
  size_t i = 0;
  for (; i + 64 <= n; i += 64) block(h, p + i, k.K);
  // the tail, a 1 bit, zeros, then the message length in bits (big endian) closing the last block
  unsigned char tail[128] = {};
  const size_t rest = n - i;
  if (rest) std::memcpy(tail, p + i, rest);
  tail[rest] = 0x80;
  const size_t len = rest + 1 + 8 <= 64 ? 64 : 128;
  const uint64_t bits = uint64_t(n) * 8;
  for (int b = 0; b < 8; ++b) tail[len - 1 - b] = (unsigned char)(bits >> (8 * b));
  for (size_t off = 0; off < len; off += 64) block(h, tail + off, k.K);
  std::string out(32, '\0');
  for (int j = 0; j < 8; ++j)
    for (int b = 0; b < 4; ++b) out[size_t(4 * j + b)] = char(h[j] >> (24 - 8 * b));
  return out;
}

}  // namespace tsa
