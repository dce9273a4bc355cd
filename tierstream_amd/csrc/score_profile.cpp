// TSSCPRF1 score profiles: the model identity they are bound to, and the checks a profile passes before its counts
// seed scored eviction. The byte layout and the identity's definition are the format's (reference src/dg_score.cpp,
// include/strix_stream/ss.h:730-746); the refusals match the reference's profile check profile by profile.
#include "score_profile.hpp"

#include <cstring>

#include "common.hpp"
#include "sha256.hpp"

namespace tsa {
namespace {

constexpr char kMagic[8] = {'T', 'S', 'S', 'C', 'P', 'R', 'F', '1'};
constexpr uint32_t kVersion = 1;
constexpr uint32_t kProvenanceLimit = 4096;
constexpr uint32_t kScoredUnitLimit = 65536;

[[noreturn]] void refuse(const std::string& why) { fail(SS_E_INVALID, "score profile (TSSCPRF1): " + why); }

// Sizes from a header nobody vouches for: an overflow is a refusal, not a wrap.
uint64_t add(uint64_t a, uint64_t b) {
  uint64_t r = 0;
  if (__builtin_add_overflow(a, b, &r)) refuse("a size in the header overflows 64 bits");
  return r;
}
uint64_t mul(uint64_t a, uint64_t b) {
  uint64_t r = 0;
  if (__builtin_mul_overflow(a, b, &r)) refuse("a size in the header overflows 64 bits");
  return r;
}

void put_le(std::string& out, uint64_t v, int bytes) {
  for (int i = 0; i < bytes; ++i, v >>= 8) out.push_back(char(v & 0xff));
}

uint32_t le32_at(const unsigned char* p, uint64_t at) {
  uint32_t v = 0;
  for (int i = 3; i >= 0; --i) v = v << 8 | p[at + uint64_t(i)];
  return v;
}

}  // namespace

std::string score_identity(const Desc& d, const std::vector<int>& gated) {
  std::string msg;
  put_le(msg, gated.size(), 4);
  for (size_t g = 0; g < gated.size(); ++g) {
    const Layer& l = d.layers[size_t(gated[g])];
    require(l.hash.size() == size_t(l.n_units), SS_E_INVALID,
            "score profile: gated layer " + std::to_string(g) +
                " has no per-unit xxh64 list in the descriptor, and a profile is bound to it");
    put_le(msg, uint32_t(l.index), 4);
    put_le(msg, uint32_t(l.n_units), 4);
    put_le(msg, l.unit_bytes, 8);
    for (uint64_t h : l.hash) put_le(msg, h, 8);
  }
  return sha256(msg.data(), msg.size());
}

uint64_t score_cells(const std::vector<uint32_t>& units) {
  uint64_t cells = 0;
  for (size_t g = 0; g < units.size(); ++g) {
    require(units[g] <= kScoredUnitLimit, SS_E_INVALID,
            "scored eviction: gated layer " + std::to_string(g) + " has " + std::to_string(units[g]) +
                " units, above 65536");
    cells = add(cells, mul(units[g], units[g]));
  }
  return cells;
}

ScoreProfile check_score_profile(const void* data, uint64_t len, const std::vector<uint32_t>& units,
                                 const std::string& identity) {
  if (!data) refuse("no bytes");
  const auto* p = static_cast<const unsigned char*>(data);
  const uint64_t n_gated = units.size();
  // magic, version, layer count, per-layer units | identity | provenance length
  const uint64_t units_at = 16, identity_at = add(units_at, mul(4, n_gated)), prov_len_at = add(identity_at, 32);
  const uint64_t prov_at = add(prov_len_at, 4);
  if (len < prov_at) refuse(std::to_string(len) + " bytes is shorter than the fixed header");
  if (std::memcmp(p, kMagic, sizeof kMagic) != 0) refuse("not a TSSCPRF1 profile (magic)");
  if (le32_at(p, 8) != kVersion) refuse("version " + std::to_string(le32_at(p, 8)) + " (only 1 is read)");
  if (le32_at(p, 12) != n_gated)
    refuse("written for " + std::to_string(le32_at(p, 12)) + " gated layers, the context has " +
           std::to_string(n_gated));
  for (uint64_t g = 0; g < n_gated; ++g) {
    const uint32_t written = le32_at(p, units_at + 4 * g);
    if (written != units[size_t(g)])
      refuse("gated layer " + std::to_string(g) + " has " + std::to_string(written) + " units in the profile and " +
             std::to_string(units[size_t(g)]) + " in the context");
  }
  const uint32_t prov_len = le32_at(p, prov_len_at);
  if (prov_len > kProvenanceLimit) refuse("provenance of " + std::to_string(prov_len) + " bytes (at most 4096)");
  const uint64_t cells_at = add(prov_at, prov_len);
  const uint64_t expect = add(add(cells_at, mul(4, score_cells(units))), 32);
  if (len != expect) refuse(std::to_string(len) + " bytes where the header implies " + std::to_string(expect));
  if (identity.size() != 32 || std::memcmp(p + identity_at, identity.data(), 32) != 0)
    refuse("bound to another model identity (descriptor, gated layers or hashes differ)");
  if (sha256(p, size_t(len - 32)).compare(0, 32, reinterpret_cast<const char*>(p + len - 32), 32) != 0)
    refuse("the SHA-256 at its end does not match its bytes");
  ScoreProfile v;
  v.provenance.assign(reinterpret_cast<const char*>(p + prov_at), prov_len);
  v.cells = p + cells_at;
  return v;
}

}  // namespace tsa
