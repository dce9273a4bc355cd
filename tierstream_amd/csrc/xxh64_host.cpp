// Host XXH64 (seed 0), from the published algorithm: 32-byte stripes into four accumulators, then a merge, the tail and
// an avalanche. Reads words little-endian independent of the host byte order. Restates reference src/xxh64.cpp:39-112.
#include "common.hpp"

namespace tsa {
namespace {

constexpr uint64_t P1 = 0x9E3779B185EBCA87ull;
constexpr uint64_t P2 = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t P3 = 0x165667B19E3779F9ull;
constexpr uint64_t P4 = 0x85EBCA77C2B2AE63ull;
constexpr uint64_t P5 = 0x27D4EB2F165667C5ull;

inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t le64(const unsigned char* p) {
  uint64_t v;
  std::memcpy(&v, p, 8);
#if __BYTE_ORDER__ == __ORDER_BIG_ENDIAN__
  v = __builtin_bswap64(v);
#endif
  return v;
}
inline uint32_t le32(const unsigned char* p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
#if __BYTE_ORDER__ == __ORDER_BIG_ENDIAN__
  v = __builtin_bswap32(v);
#endif
  return v;
}
inline uint64_t rnd(uint64_t a, uint64_t w) { return rotl(a + w * P2, 31) * P1; }

}  // namespace

Xxh64::Xxh64() {
  v_[0] = P1 + P2;
  v_[1] = P2;
  v_[2] = 0;
  v_[3] = 0 - P1;
}

void Xxh64::update(const void* data, size_t len) {
  const unsigned char* p = static_cast<const unsigned char*>(data);
  total_ += len;
  if (buf_len_ + len < 32) {
    std::memcpy(buf_ + buf_len_, p, len);
    buf_len_ += len;
    return;
  }
  if (buf_len_) {
    const size_t take = 32 - buf_len_;
    std::memcpy(buf_ + buf_len_, p, take);
    for (int k = 0; k < 4; ++k) v_[k] = rnd(v_[k], le64(buf_ + 8 * k));
    p += take;
    len -= take;
    buf_len_ = 0;
  }
  uint64_t a = v_[0], b = v_[1], c = v_[2], d = v_[3];
  for (; len >= 32; p += 32, len -= 32) {
    a = rnd(a, le64(p));
    b = rnd(b, le64(p + 8));
    c = rnd(c, le64(p + 16));
    d = rnd(d, le64(p + 24));
  }
  v_[0] = a;
  v_[1] = b;
  v_[2] = c;
  v_[3] = d;
  std::memcpy(buf_, p, len);
  buf_len_ = len;
}

uint64_t Xxh64::digest() const {
  uint64_t h;
  if (total_ >= 32) {
    h = rotl(v_[0], 1) + rotl(v_[1], 7) + rotl(v_[2], 12) + rotl(v_[3], 18);
    for (int k = 0; k < 4; ++k) h = (h ^ rnd(0, v_[k])) * P1 + P4;
  } else {
    h = P5;
  }
  h += total_;
  const unsigned char* p = buf_;
  size_t len = buf_len_;
  for (; len >= 8; p += 8, len -= 8) {
    h ^= rnd(0, le64(p));
    h = rotl(h, 27) * P1 + P4;
  }
  if (len >= 4) {
    h ^= uint64_t(le32(p)) * P1;
    h = rotl(h, 23) * P2 + P3;
    p += 4;
    len -= 4;
  }
  for (; len; ++p, --len) {
    h ^= uint64_t(*p) * P5;
    h = rotl(h, 11) * P1;
  }
  h ^= h >> 33;
  h *= P2;
  h ^= h >> 29;
  h *= P3;
  h ^= h >> 32;
  return h;
}

uint64_t xxh64(const void* data, size_t len) {
  Xxh64 x;
  x.update(data, len);
  return x.digest();
}

}  // namespace tsa
