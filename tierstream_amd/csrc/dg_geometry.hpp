// Device-gated decode: what an open derives from the descriptor, the plan and the options before it allocates
// anything - the refused configurations, the gated layers and their one part shape, the units' homes (resident,
// pinned, file), the arena's slots (persistent R + D, two banks of dg_max_ids, the guard), the pinned blocks
// (homes + spares), the file tier's staging and reads in flight, and scored eviction's weights and profile.
//
// The rules are the reference's (src/dg_layout.cpp:159-180 and :182-393): the geometry is part of what an engine sees
// (slot counts, the guard slot) and the refusals are part of the ABI. This library serves a subset of the reference's
// options (no-admit, prefetch revert, strict admission and priors are refused with SS_E_UNSUPPORTED), and it does not
// re-check the host budget for its own control memory (an allocation that does not fit fails the open with
// SS_E_NOMEM).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "model.hpp"
#include "strix_stream/ss.h"

namespace tsa {

struct DgGeometry {
  std::vector<int> gated;            // descriptor layer of each gated ordinal
  std::vector<int> ordinal;          // per descriptor layer: its gated ordinal, -1
  std::vector<uint32_t> unit_base;   // gated ordinal -> first key (G + 1 entries)
  std::vector<uint64_t> part_bytes, part_offset;
  uint64_t unit_bytes = 0, host_stride = 0;
  uint32_t keys = 0;
  uint32_t R = 0;  // planned residents (the first slots at open)
  uint32_t D = 0;  // spare slots (the boundary keeps that many free)
  uint32_t B = 0;  // ids per export (dg_max_ids): one bank of slots
  uint32_t P = 0;  // pinned homes
  uint32_t F = 0;  // file homes (three tiers)
  uint32_t Q = 0;  // spare pinned blocks
  uint32_t I = 0;  // clean copies kept in spare blocks (dg_inclusive_blocks)
  uint32_t S = 0;  // file-tier staging buffers
  uint32_t disk_queue = 0;       // file reads in flight (1: inside the fetch)
  uint32_t persistent_slots = 0; // R + D
  uint32_t slots = 0;            // R + D + 2B + 1
  uint32_t guard_slot = 0;       // the last slot, zeroed
  uint32_t blocks = 0;           // P + Q
  std::vector<uint32_t> residents;  // keys of the planned residents, in key order
  bool disk_tier = false, disk_prefetch = false;
  uint32_t bank_keep = 0;     // dg_bank_keep with the file tier (0 without it)
  // landings (dg_landing_blocks, only with file homes in the plan): L landing blocks (block indices blocks + S ..);
  // landing pieces running at most; the TTL in boundaries (0: expiry after the target layer); a landing read's piece
  // bytes (0: one piece per part, dg_landing_chunk 0xFFFFFFFF)
  uint32_t L = 0, landing_queued = 1, landing_ttl = 0;
  uint64_t landing_chunk = 4ull << 20;
  std::vector<uint8_t> disk;  // per key: a file home (three tiers only)
  bool scored = false;
  uint32_t w_trans = 700, w_freq = 200, w_rec = 100;
  std::string score_identity;  // the profile's model identity (a profile given)
  uint64_t arena_need = 0;     // device bytes the open admits in place of the plan's billed slots
};

// Throws Error(status, "device-gated: <rule>") for the first rule the configuration breaks.
DgGeometry dg_geometry(const Desc& d, const Plan& p, const ss_options& o);

}  // namespace tsa
