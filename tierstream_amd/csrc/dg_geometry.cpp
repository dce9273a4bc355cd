#include "dg_geometry.hpp"

#include <algorithm>

#include "common.hpp"
#include "score_profile.hpp"

namespace tsa {
namespace {

constexpr uint32_t kMaxIds = 64;      // ids one export may carry
constexpr uint32_t kMaxParts = 4;     // parts of a gated unit (one arena each)
constexpr uint32_t kQueueAuto = 0xFFFFFFFFu;
constexpr uint64_t kIndexLimit = 0x7fffffffull;

[[noreturn]] void refuse(ss_status st, const std::string& why) { fail(st, "device-gated: " + why); }

// One refusal rule: broken when `when` holds.
struct Rule {
  bool when;
  ss_status status;
  const char* why;
};

// The options, before anything is derived. Rules are tried in order; the first broken one is the open's error.
void check_options(const ss_options& o, const ss_budget& b) {
  const bool scored = o.policy == SS_POLICY_SCORED || o.policy == SS_POLICY_SCORED_AUTO;
  const bool disk = o.dg_disk_tier != 0;
  const bool q_auto = o.dg_disk_queue == kQueueAuto;
  const bool landing_chunk_ok = o.dg_landing_chunk == 0xFFFFFFFFu || o.dg_landing_chunk % 4096 == 0;
  const Rule rules[] = {
      {b.tier_mode != SS_TIER_MODE_EXCLUSIVE, SS_E_INVALID, "one home per unit: tier_mode must be EXCLUSIVE"},
      {b.pinned_backing != 0, SS_E_INVALID, "one home per unit: pinned_backing must be 0"},
      {o.policy != SS_POLICY_LRU && !scored, SS_E_INVALID, "policy must be LRU, SCORED or SCORED_AUTO"},
      {(o.dg_score_profile_len || o.dg_score_profile) && !scored, SS_E_INVALID,
       "a dg_score_profile needs policy SCORED or SCORED_AUTO"},
      {o.pin_planned != 0, SS_E_INVALID, "pin_planned must be 0 (planned residents are only where the cache starts)"},
      {!o.fill_residents, SS_E_INVALID, "fill_residents must be 1 (a resident's slot holds its only device copy)"},
      {o.readahead_units != 0, SS_E_INVALID, "readahead_units must be 0 (host read-ahead is a host-contract option)"},
      {o.spec_persistent != 0, SS_E_INVALID, "spec_persistent must be 0 (the service admits predictions itself)"},
      {o.dg_max_ids < 1 || o.dg_max_ids > kMaxIds, SS_E_INVALID, "dg_max_ids must be 1..64 (rows x top_k)"},
      {o.dg_wait_timeout_ms < 1, SS_E_INVALID, "dg_wait_timeout_ms must be at least 1"},
      {o.dg_wb_defer > 1, SS_E_INVALID, "dg_wb_defer must be 0 or 1"},
      {o.dg_wb_stream > 1, SS_E_INVALID, "dg_wb_stream must be 0 or 1"},
      {o.dg_disk_tier > 1 || o.dg_disk_prefetch > 1, SS_E_INVALID, "dg_disk_tier and dg_disk_prefetch must be 0 or 1"},
      {!disk && (o.dg_disk_prefetch || o.dg_disk_staging || (o.dg_disk_queue && !q_auto)), SS_E_INVALID,
       "dg_disk_prefetch, dg_disk_staging and dg_disk_queue apply only with dg_disk_tier = 1"},
      {o.dg_disk_staging > 256, SS_E_INVALID, "dg_disk_staging must be 0..256"},
      {o.dg_disk_queue > 64 && !q_auto, SS_E_INVALID, "dg_disk_queue must be 0..64 or SS_DG_DISK_QUEUE_AUTO"},
      {o.dg_no_admit > 1, SS_E_INVALID, "dg_no_admit must be 0 or 1"},
      {o.dg_clean_evict > 1, SS_E_INVALID, "dg_clean_evict must be 0 or 1"},
      {o.dg_bank_keep > 2, SS_E_INVALID, "dg_bank_keep must be 0, 1 or 2"},
      {o.dg_disk_queue_adapt > 1, SS_E_INVALID, "dg_disk_queue_adapt must be 0 or 1"},
      {o.dg_disk_queue_adapt && (!disk || !q_auto), SS_E_INVALID,
       "dg_disk_queue_adapt needs dg_disk_tier = 1 and dg_disk_queue = SS_DG_DISK_QUEUE_AUTO"},
      {o.dg_pf_revert_unused > 1, SS_E_INVALID, "dg_pf_revert_unused must be 0 or 1"},
      {o.dg_pf_strict_admit > 1, SS_E_INVALID, "dg_pf_strict_admit must be 0 or 1"},
      {o.dg_landing_blocks > 4096, SS_E_INVALID, "dg_landing_blocks must be 0..4096"},
      {!o.dg_landing_blocks && (o.dg_landing_max_queued || o.dg_landing_ttl || o.dg_landing_chunk), SS_E_INVALID,
       "dg_landing_max_queued, dg_landing_ttl and dg_landing_chunk apply only with dg_landing_blocks > 0"},
      {o.dg_landing_max_queued > 64, SS_E_INVALID, "dg_landing_max_queued must be 0..64"},
      {o.dg_landing_ttl > 1024, SS_E_INVALID, "dg_landing_ttl must be 0..1024"},
      {!landing_chunk_ok, SS_E_INVALID, "dg_landing_chunk must be 0, a multiple of 4096 or 0xFFFFFFFF"},
      {o.dg_landing_blocks && !disk, SS_E_INVALID, "dg_landing_blocks needs dg_disk_tier = 1"},
      {o.dg_landing_blocks && o.dg_disk_queue <= 1, SS_E_INVALID,
       "dg_landing_blocks needs dg_disk_queue > 1 (landing reads run on the reader threads)"},
      // valid for the reference, not served by this library
      {o.dg_no_admit || o.dg_pf_revert_unused || o.dg_pf_strict_admit || o.dg_prior_len || o.dg_prior,
       SS_E_UNSUPPORTED, "dg_no_admit, dg_pf_revert_unused, dg_pf_strict_admit and priors are not served by this library"},
  };
  for (const Rule& r : rules)
    if (r.when) refuse(r.status, r.why);
}

// The gated layers (every layer with units) and the one part shape they share: one arena per part.
void scan_layers(const Desc& d, DgGeometry& x) {
  x.ordinal.assign(d.layers.size(), -1);
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    if (!l.n_units) continue;
    const std::string name = "layer " + std::to_string(l.index);
    if (!l.streamable) refuse(SS_E_UNSUPPORTED, name + " has non-streamable units (every unit must be gated)");
    if (x.gated.empty()) {
      if (l.parts.size() > kMaxParts) refuse(SS_E_UNSUPPORTED, "a unit has more than 4 parts");
      for (const Part& part : l.parts) {
        if (part.bytes % 256)
          refuse(SS_E_UNSUPPORTED, "part " + part.name + " holds " + std::to_string(part.bytes) +
                                       " bytes, not a multiple of 256 (a slot of its arena is exactly its bytes)");
        x.part_offset.push_back(x.unit_bytes);
        x.part_bytes.push_back(part.bytes);
        x.unit_bytes += part.bytes;
      }
    } else {
      const Layer& first = d.layers[size_t(x.gated[0])];
      const bool same = l.parts.size() == first.parts.size() &&
                        std::equal(l.parts.begin(), l.parts.end(), first.parts.begin(),
                                   [](const Part& a, const Part& b) { return a.bytes == b.bytes; });
      if (!same) refuse(SS_E_UNSUPPORTED, name + "'s parts differ from the first gated layer's (one arena per part)");
    }
    x.ordinal[L] = int(x.gated.size());
    x.gated.push_back(int(L));
  }
  if (x.gated.empty()) refuse(SS_E_INVALID, "the descriptor has no streamable units");
  x.host_stride = host_stride(x.unit_bytes);
}

// Homes from the plan's tiers, keys in descriptor order; the spare slots each layer brings (its billed dynamic slots,
// at most its units off the device).
void place_homes(const Desc& d, const Plan& p, const ss_options& o, DgGeometry& x) {
  x.unit_base.assign(1, 0);
  uint64_t key = 0;
  for (int L : x.gated) {
    const Layer& l = d.layers[size_t(L)];
    uint32_t on_device = 0;
    for (int u = 0; u < l.n_units; ++u, ++key) {
      const uint8_t t = p.tier[size_t(d.gidx(L, u))];
      const bool file = t == SS_TIER_DISK && o.dg_disk_tier;
      if (t == SS_TIER_RESIDENT) {
        x.residents.push_back(uint32_t(key));
        ++on_device;
      } else if (t == SS_TIER_PINNED) {
        ++x.P;
      } else if (file) {
        ++x.F;
      } else {
        refuse(SS_E_CAPACITY, "unit (" + std::to_string(l.index) + ", " + std::to_string(u) +
                                  ") is neither resident nor pinned" +
                                  (o.dg_disk_tier ? "" : " (file homes need dg_disk_tier = 1)"));
      }
      if (o.dg_disk_tier) x.disk.push_back(file ? 1 : 0);
    }
    x.D += std::min<uint32_t>(p.budget.dynamic_slots_per_layer, uint32_t(l.n_units) - on_device);
    require(key < kIndexLimit, SS_E_INVALID, "device-gated: more than 2^31 - 1 gated units");
    x.unit_base.push_back(uint32_t(key));
  }
  x.keys = uint32_t(key);
  x.R = uint32_t(x.residents.size());
  if (o.dg_spare_slots) {
    if (o.dg_spare_slots > x.P + x.F)
      refuse(SS_E_INVALID, "dg_spare_slots " + std::to_string(o.dg_spare_slots) + " is more than the " +
                               std::to_string(x.P + x.F) + " units off the device");
    x.D = o.dg_spare_slots;
  }
  if (x.D < 1)
    refuse(SS_E_INVALID, "no spare slots: set dynamic_slots_per_layer or dg_spare_slots (the boundary keeps them free)");
}

// Reads in flight and staging buffers of the file tier (none without it). AUTO: three reads per read location (one
// here: a source is read from its own file), 4..8, at most an explicit staging count; staging: as given, else 8 (AUTO:
// at least its queue).
void size_disk_tier(const ss_options& o, DgGeometry& x) {
  x.disk_tier = o.dg_disk_tier != 0;
  x.disk_prefetch = o.dg_disk_prefetch != 0;
  x.bank_keep = x.disk_tier ? o.dg_bank_keep : 0;  // (no effect without the file tier)
  if (!x.disk_tier) return;
  x.L = x.F ? o.dg_landing_blocks : 0u;  // (nothing to land without file homes)
  x.landing_queued = o.dg_landing_max_queued ? o.dg_landing_max_queued : 1u;
  x.landing_ttl = o.dg_landing_ttl;
  x.landing_chunk = o.dg_landing_chunk == 0xFFFFFFFFu ? 0u : o.dg_landing_chunk ? o.dg_landing_chunk : 4ull << 20;
  if (o.dg_disk_queue == kQueueAuto) {
    constexpr uint32_t kLocations = 1;
    x.disk_queue = std::min<uint32_t>(std::max<uint32_t>(3 * kLocations, 4), 8);
    if (o.dg_disk_staging) x.disk_queue = std::min(x.disk_queue, o.dg_disk_staging);
    x.S = o.dg_disk_staging ? o.dg_disk_staging : std::max<uint32_t>(8, x.disk_queue);
  } else {
    x.disk_queue = o.dg_disk_queue ? o.dg_disk_queue : 1;
    x.S = o.dg_disk_staging ? o.dg_disk_staging : 8;
  }
}

void size_scoring(const Desc& d, const ss_options& o, DgGeometry& x) {
  if (o.policy != SS_POLICY_SCORED && o.policy != SS_POLICY_SCORED_AUTO) return;
  x.scored = true;
  const uint32_t wt = o.dg_score_w_trans, wf = o.dg_score_w_freq, wr = o.dg_score_w_recency;
  if (wt || wf || wr) {  // (all three 0: the defaults)
    if (wt > 1000 || wf > 1000 || wr > 1000 || wt + wf + wr != 1000)
      refuse(SS_E_INVALID, "dg_score_w_trans, _freq and _recency must each be 0..1000 and add up to 1000");
    x.w_trans = wt;
    x.w_freq = wf;
    x.w_rec = wr;
  }
  std::vector<uint32_t> units;
  for (int L : x.gated) units.push_back(uint32_t(d.layers[size_t(L)].n_units));
  if (score_cells(units) > uint64_t(SIZE_MAX / 8)) refuse(SS_E_INVALID, "the score tables exceed the address space");
  if (o.dg_score_profile_len || o.dg_score_profile) {
    if (!o.dg_score_profile || !o.dg_score_profile_len)
      refuse(SS_E_INVALID, "dg_score_profile needs its dg_score_profile_len and the other way round");
    x.score_identity = score_identity(d, x.gated);
    (void)check_score_profile(o.dg_score_profile, o.dg_score_profile_len, units, x.score_identity);
  }
}

// Host admission: the pinned bytes an open adds to the plan's (reference src/dg_layout.cpp:96-125 and :393-420, whose
// sum decides which budgets admit an open, so it is kept as it is): the control area as laid out for 64-id records
// (a 288-byte export record and a 272-byte prediction record per gated layer, three word arrays of the gated layers,
// seven words, and 32 layer-token part records with two part word arrays), a bounce buffer per reader (the context's
// and each file reader's, min(staging_bytes, 16 MiB) rounded up to the sources' alignment, at least 4 alignments; with
// file readers cut to the largest part plus two alignments), one unit of staging (4 KiB rounded), and the file
// tier's staging buffers and landing blocks of one host stride each.
struct HostExtra {
  uint64_t mapped = 0, bounce = 0, staging = 0, disk_staging = 0, landing = 0, total = 0;
};
HostExtra host_extra(const Desc& d, const ss_options& o, const DgGeometry& x) {
  constexpr uint64_t kRecord = 288, kPredRecord = 272, kParts = 32;
  const auto a64 = [](uint64_t v) { return (v + 63) / 64 * 64; };
  const uint64_t G = x.gated.size();
  HostExtra h;
  h.mapped = a64(G * kRecord) + a64(G * kPredRecord) + 3 * a64(G * 4) + a64(7 * 4) + a64(kParts * kRecord) +
             2 * a64(kParts * 4);
  uint64_t align = 4096, part_max = 0;
  for (const Source& src : d.sources) align = std::max(align, src.align);
  for (uint64_t pb : x.part_bytes) part_max = std::max(part_max, pb);
  const auto up = [align](uint64_t v) {
    uint64_t r = 0;
    if (__builtin_add_overflow(v, align - 1, &r)) refuse(SS_E_INVALID, "the bounce buffer overflows");
    return r / align * align;
  };
  const uint64_t want = std::min<uint64_t>(o.staging_bytes ? o.staging_bytes : 16ull << 20, 16ull << 20);
  uint64_t bounce = std::max(up(want), 4 * align);
  const uint64_t readers = 1 + (x.disk_queue > 1 ? x.disk_queue : 0);
  if (readers > 1) bounce = std::max(std::min(bounce, up(part_max + 2 * align)), 4 * align);
  h.bounce = bounce * readers;
  h.staging = (x.unit_bytes + 4095) / 4096 * 4096;
  h.disk_staging = uint64_t(x.S) * x.host_stride;
  h.landing = uint64_t(x.L) * x.host_stride;
  const uint64_t parts[] = {h.mapped, h.bounce, h.staging, h.disk_staging, h.landing};
  for (uint64_t v : parts)
    if (__builtin_add_overflow(h.total, v, &h.total)) refuse(SS_E_INVALID, "the host extras overflow");
  return h;
}

}  // namespace

DgGeometry dg_geometry(const Desc& d, const Plan& p, const ss_options& o) {
  check_options(o, p.budget);
  DgGeometry x;
  x.B = o.dg_max_ids;
  scan_layers(d, x);
  place_homes(d, p, o, x);

  // the banks and the guard take the slots the plan billed for the ring of the unit's stride
  const uint64_t stride = d.unit_stride(x.gated[0]);
  uint32_t ring = 0;
  for (const RingClass& rc : p.rings)
    if (rc.stride == stride) ring = rc.slots;
  const uint64_t banks = 2ull * x.B + 1;
  if (ring < banks)
    refuse(SS_E_CAPACITY, "two banks of " + std::to_string(x.B) + " slots and the guard need " +
                              std::to_string(banks) + " ring slots; the plan bills " + std::to_string(ring) +
                              " (ring_slots = 2 x dg_max_ids + 1)");
  // spare blocks of the unit's host stride: a write-back needs a free one
  for (const SpareClass& sc : p.spares)
    if (sc.block_bytes == x.host_stride) x.Q = sc.blocks;
  if (!x.Q)
    refuse(SS_E_CAPACITY, "the plan has no spare block (host_spare_units " + std::to_string(p.budget.host_spare_units) +
                              "): every write-back needs a free block");
  require(uint64_t(x.P) + x.Q < kIndexLimit, SS_E_INVALID, "device-gated: more than 2^31 - 1 host blocks");
  x.blocks = x.P + x.Q;
  x.I = o.dg_inclusive_blocks;
  if (x.I && x.I >= x.Q)
    refuse(SS_E_CAPACITY, "dg_inclusive_blocks " + std::to_string(x.I) + " leaves none of the " +
                              std::to_string(x.Q) + " spare blocks for write-backs (raise host_spare_units)");
  size_disk_tier(o, x);
  size_scoring(d, o, x);

  x.persistent_slots = x.R + x.D;
  const uint64_t slots = uint64_t(x.persistent_slots) + banks;
  require(slots < kIndexLimit, SS_E_INVALID, "device-gated: more than 2^31 - 1 slots");
  x.slots = uint32_t(slots);
  x.guard_slot = x.slots - 1;
  // Device admission: the plan billed resident, dynamic and ring slots; the arena replaces them. It must fit the cap
  // with the rest of the plan. (The control words counted are the reference's accounting of a context's device
  // controls: seq, abort, three error words, a miss word per gated layer, the unit bases, absent_err and four
  // layer-token words.)
  const uint64_t G = x.gated.size();
  const uint64_t ctl_bytes = 4 * (5 + G + (G + 1) + 1 + 4);
  x.arena_need = slots * x.unit_bytes + uint64_t(x.keys) * 4 + ctl_bytes;
  const uint64_t billed = p.resident + p.dynamic + p.ring;
  const uint64_t rest = p.peak >= billed ? p.peak - billed : 0;
  const uint64_t limit = p.cap > p.margin ? p.cap - p.margin : 0;
  if (rest + x.arena_need > limit)
    refuse(SS_E_CAPACITY, "the arena needs " + std::to_string(x.arena_need) + " bytes of HBM where the plan billed " +
                              std::to_string(billed) + "; with the rest of the plan that exceeds the cap less margin");
  const HostExtra h = host_extra(d, o, x);
  uint64_t host_total = 0;
  if (__builtin_add_overflow(p.pinned, h.total, &host_total)) refuse(SS_E_INVALID, "the host bytes overflow");
  if (host_total > p.budget.host_pinned_bytes)
    refuse(SS_E_CAPACITY, "the plan's pinned bytes (" + std::to_string(p.pinned) + ") plus the control area (" +
                              std::to_string(h.mapped) + "), the bounce buffers (" + std::to_string(h.bounce) +
                              "), the staging unit (" + std::to_string(h.staging) + "), the file tier's staging "
                              "buffers (" + std::to_string(h.disk_staging) + ") and the landing blocks (" +
                              std::to_string(h.landing) + ") exceed the host budget (" +
                              std::to_string(p.budget.host_pinned_bytes) + ")");
  // ... and headroom for four units beyond that: the reference's open streams its startup through a ring of four
  // buffers of at least a unit each (reference src/dg_layout.cpp:425-444, its defaults). This open stages its startup
  // through the spare blocks instead, but admits the same budgets.
  const uint64_t headroom = p.budget.host_pinned_bytes - host_total;
  if (headroom / 4 / 4096 * 4096 < x.unit_bytes)
    refuse(SS_E_CAPACITY, "the host budget leaves " + std::to_string(headroom) + " bytes beyond the open's pinned "
                              "bytes; the startup needs four units (" + std::to_string(4 * x.unit_bytes) + ")");
  return x;
}

}  // namespace tsa
