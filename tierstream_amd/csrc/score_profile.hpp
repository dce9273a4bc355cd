// Scored eviction's starting counts: the TSSCPRF1 profile format and the model identity it is bound to (reference
// src/dg_score.hpp:4-8, include/strix_stream/ss.h:730-746; the format is frozen, so it is kept byte for byte).
//
// Profile, little endian: "TSSCPRF1", u32 version 1, u32 n_gated, u32 units[n_gated], identity[32], u32 prov_len
// (<= 4096), prov[prov_len], then per gated layer units^2 u32 counts row-major [previous unit][unit], then the SHA-256
// of every byte before it. identity = SHA-256 of u32 n_gated, then per gated layer: u32 model layer index, u32 units,
// u64 unit_bytes, the descriptor's per-unit xxh64 list.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "model.hpp"

namespace tsa {

// The 32 raw identity bytes of the gated layers (descriptor layer indices). SS_E_INVALID when a gated layer has no
// per-unit hashes.
std::string score_identity(const Desc& d, const std::vector<int>& gated);

// sum_g units(g)^2; SS_E_INVALID for a layer above 65536 units.
uint64_t score_cells(const std::vector<uint32_t>& units);

struct ScoreProfile {
  const unsigned char* cells = nullptr;  // into the checked bytes: the first gated layer's first count
  std::string provenance;
};
// Every rule of the format, in order: size of the fixed header, magic, version, n_gated, units, provenance length,
// exact total size, identity, checksum. SS_E_INVALID naming the first broken one.
ScoreProfile check_score_profile(const void* data, uint64_t len, const std::vector<uint32_t>& units,
                                 const std::string& identity);

}  // namespace tsa
