/*
 * ORACLE (test infrastructure only): a CPU restatement of the reference's XXH64 and of the checkpoint layout the device
 * verifier uses. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only to compare
 * against; the product never links or calls it.
 *
 * xxh64: reference src/xxh64.cpp:39-112 (XXH64, seed 0, little-endian 64-bit lanes, 32-byte stripes into four
 * accumulators v = rotl(v + lane * P2, 31) * P1, merge of the four, length, tail by 8 / 4 / 1 bytes, avalanche).
 * Pinned by: the reference's known answers (tests/test_core.cpp:64-82), the independent python-xxhash library on
 * random inputs of every length class, and streaming == one-shot.
 *
 * checkpoints: the accumulators before each segment of a unit's extents (include/tierstream_amd/tsa.h layout); pinned
 * by construction against the oracle's own one-shot digest (the chain run from the checkpoints reproduces it) and by
 * the product/oracle comparison in the tests.
 *
 * Written plainly and byte by byte on purpose: a second, independent formulation of what the product computes.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define O_P1 0x9E3779B185EBCA87ull
#define O_P2 0xC2B2AE3D27D4EB4Full
#define O_P3 0x165667B19E3779F9ull
#define O_P4 0x85EBCA77C2B2AE63ull
#define O_P5 0x27D4EB2F165667C5ull

static uint64_t o_rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }

static uint64_t o_rd64(const unsigned char* p) {
  uint64_t v = 0;
  for (int k = 7; k >= 0; --k) v = (v << 8) | p[k];
  return v;
}

static uint32_t o_rd32(const unsigned char* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static uint64_t o_round(uint64_t acc, uint64_t lane) {
  acc += lane * O_P2;
  acc = o_rotl(acc, 31);
  return acc * O_P1;
}

typedef struct {
  uint64_t v[4];
  uint64_t total;
  unsigned char buf[32];
  size_t buf_len;
} oracle_xxh64_state;

void oracle_xxh64_init(oracle_xxh64_state* s) {
  s->v[0] = O_P1 + O_P2;
  s->v[1] = O_P2;
  s->v[2] = 0;
  s->v[3] = (uint64_t)0 - O_P1;
  s->total = 0;
  s->buf_len = 0;
}

void oracle_xxh64_update(oracle_xxh64_state* s, const void* data, size_t len) {
  const unsigned char* p = (const unsigned char*)data;
  s->total += len;
  while (len) {
    size_t take = 32 - s->buf_len;
    if (take > len) take = len;
    memcpy(s->buf + s->buf_len, p, take);
    s->buf_len += take;
    p += take;
    len -= take;
    if (s->buf_len == 32) {
      for (int k = 0; k < 4; ++k) s->v[k] = o_round(s->v[k], o_rd64(s->buf + 8 * k));
      s->buf_len = 0;
    }
  }
}

uint64_t oracle_xxh64_digest(const oracle_xxh64_state* s) {
  uint64_t h;
  if (s->total >= 32) {
    h = o_rotl(s->v[0], 1) + o_rotl(s->v[1], 7) + o_rotl(s->v[2], 12) + o_rotl(s->v[3], 18);
    for (int k = 0; k < 4; ++k) {
      h ^= o_round(0, s->v[k]);
      h = h * O_P1 + O_P4;
    }
  } else {
    h = O_P5;
  }
  h += s->total;
  const unsigned char* p = s->buf;
  size_t len = s->buf_len;
  while (len >= 8) {
    h ^= o_round(0, o_rd64(p));
    h = o_rotl(h, 27) * O_P1 + O_P4;
    p += 8;
    len -= 8;
  }
  if (len >= 4) {
    h ^= (uint64_t)o_rd32(p) * O_P1;
    h = o_rotl(h, 23) * O_P2 + O_P3;
    p += 4;
    len -= 4;
  }
  while (len) {
    h ^= (uint64_t)(*p) * O_P5;
    h = o_rotl(h, 11) * O_P1;
    ++p;
    --len;
  }
  h ^= h >> 33;
  h *= O_P2;
  h ^= h >> 29;
  h *= O_P3;
  h ^= h >> 32;
  return h;
}

uint64_t oracle_xxh64(const void* data, size_t len) {
  oracle_xxh64_state s;
  oracle_xxh64_init(&s);
  oracle_xxh64_update(&s, data, len);
  return oracle_xxh64_digest(&s);
}

/* Digest of n extents back to back (the unit byte stream). */
uint64_t oracle_xxh64_extents(const void* const* ptrs, const uint64_t* bytes, uint32_t n) {
  oracle_xxh64_state s;
  oracle_xxh64_init(&s);
  for (uint32_t e = 0; e < n; ++e) oracle_xxh64_update(&s, ptrs[e], (size_t)bytes[e]);
  return oracle_xxh64_digest(&s);
}

/* Checkpoints: per extent e, span = bytes (last: rounded down to 32, at least one segment), segments of seg bytes; the
 * accumulators before each segment. Returns the count written (0 if `cap` is too small or the layout is invalid). */
uint64_t oracle_checkpoints(const void* const* ptrs, const uint64_t* bytes, uint32_t n, uint64_t seg,
                            uint64_t* states, uint64_t cap, uint64_t* digest) {
  if (n == 0 || seg == 0 || seg % 32) return 0;
  oracle_xxh64_state s;
  oracle_xxh64_init(&s);
  uint64_t k = 0;
  for (uint32_t e = 0; e < n; ++e) {
    const int last = e + 1 == n;
    if (!last && bytes[e] % 32) return 0;
    const uint64_t span = last ? bytes[e] - bytes[e] % 32 : bytes[e];
    uint64_t nseg = (span + seg - 1) / seg;
    if (last && nseg == 0) nseg = 1;
    const unsigned char* p = (const unsigned char*)ptrs[e];
    for (uint64_t i = 0; i < nseg; ++i) {
      if (k >= cap) return 0;
      memcpy(states + 4 * k, s.v, 32);
      ++k;
      const uint64_t off = i * seg;
      const uint64_t end = off + seg < span ? off + seg : span;
      if (end > off) oracle_xxh64_update(&s, p + off, (size_t)(end - off));
    }
    if (last && bytes[e] > span) oracle_xxh64_update(&s, p + span, (size_t)(bytes[e] - span));
  }
  if (digest) *digest = oracle_xxh64_digest(&s);
  return k;
}
