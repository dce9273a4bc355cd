// TSSCPRF1 profiles: checks and the model identity (reference src/dg_score.cpp:45-120).
#include "score_profile.hpp"

#include <cstring>

#include "common.hpp"
#include "sha256.hpp"

namespace tsa {
namespace {

void le32(std::string& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back(char(v >> (8 * i)));
}
void le64(std::string& b, uint64_t v) {
  for (int i = 0; i < 8; ++i) b.push_back(char(v >> (8 * i)));
}
uint32_t rd32(const unsigned char* p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }

[[noreturn]] void bad(const std::string& why) { fail(SS_E_INVALID, "dg_score_profile (TSSCPRF1): " + why); }

// a + b and a * b on sizes a hostile header could overflow
uint64_t sum(uint64_t a, uint64_t b) {
  if (a > UINT64_MAX - b) bad("size overflows");
  return a + b;
}
uint64_t prod(uint64_t a, uint64_t b) {
  if (b && a > UINT64_MAX / b) bad("size overflows");
  return a * b;
}

}  // namespace

std::string score_identity(const Desc& d, const std::vector<int>& gated) {
  std::string b;
  le32(b, uint32_t(gated.size()));
  for (size_t g = 0; g < gated.size(); ++g) {
    const Layer& l = d.layers[size_t(gated[g])];
    require(l.hash.size() == size_t(l.n_units), SS_E_INVALID,
            "dg_score_profile: gated layer " + std::to_string(g) +
                " has no per-unit hashes in the descriptor (a profile is bound to them)");
    le32(b, uint32_t(l.index));
    le32(b, uint32_t(l.n_units));
    le64(b, l.unit_bytes);
    for (uint64_t h : l.hash) le64(b, h);
  }
  return sha256(b.data(), b.size());
}

uint64_t score_cells(const std::vector<uint32_t>& units) {
  uint64_t n = 0;
  for (size_t g = 0; g < units.size(); ++g) {
    require(units[g] <= 65536, SS_E_INVALID,
            "device-gated: scored eviction needs at most 65536 units per gated layer (gated layer " +
                std::to_string(g) + " has " + std::to_string(units[g]) + ")");
    n = sum(n, prod(units[g], units[g]));
  }
  return n;
}

ScoreProfile check_score_profile(const void* data, uint64_t len, const std::vector<uint32_t>& units,
                                 const std::string& identity) {
  if (!data) bad("null data");
  const auto* p = static_cast<const unsigned char*>(data);
  const uint64_t G = units.size();
  const uint64_t at_id = sum(16, prod(4, G));  // magic, version, n_gated, units
  const uint64_t fixed = sum(at_id, 36);       // identity, prov_len
  if (len < fixed) bad("truncated header (" + std::to_string(len) + " bytes)");
  if (std::memcmp(p, "TSSCPRF1", 8) != 0) bad("bad magic");
  if (rd32(p + 8) != 1) bad("unsupported version " + std::to_string(rd32(p + 8)));
  if (rd32(p + 12) != G) bad("n_gated " + std::to_string(rd32(p + 12)) + " != the context's " + std::to_string(G));
  for (uint64_t g = 0; g < G; ++g)
    if (rd32(p + 16 + 4 * g) != units[size_t(g)])
      bad("units of gated layer " + std::to_string(g) + " are " + std::to_string(rd32(p + 16 + 4 * g)) +
          ", the context has " + std::to_string(units[size_t(g)]));
  const uint32_t prov = rd32(p + at_id + 32);
  if (prov > 4096) bad("provenance longer than 4096 bytes");
  const uint64_t header = fixed + prov;
  const uint64_t want = sum(sum(header, prod(4, score_cells(units))), 32);
  if (len != want) bad("size " + std::to_string(len) + " != " + std::to_string(want) + " (header + cells + checksum)");
  if (identity.size() != 32 || std::memcmp(p + at_id, identity.data(), 32) != 0)
    bad("identity mismatch (another model, layer set or descriptor)");
  if (sha256(p, size_t(len - 32)) != std::string(reinterpret_cast<const char*>(p + len - 32), 32))
    bad("checksum mismatch");
  ScoreProfile v;
  v.provenance.assign(reinterpret_cast<const char*>(p + fixed), prov);
  v.cells = p + header;
  return v;
}

}  // namespace tsa
