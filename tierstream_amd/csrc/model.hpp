// The model side of the serve path: the desc-v1 descriptor (what units exist and where their bytes live) and the
// placement plan (which units are resident, pinned, on disk). Same document formats and the same placement rule as
// reference src/desc.cpp and src/plan.cpp; restated here, not translated.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "json.hpp"
#include "strix_stream/ss.h"

namespace tsa {

enum class LayerKind { Dense, Moe, Blob };
enum class Tiers { Pinned, Disk, PinnedDisk, Pair };
enum class Order { Prefix, Ranked };

struct Source {
  std::string name, path;
  uint64_t align = 4096;
};

// Part p of unit u: source `source`, bytes [offset + u * stride, + bytes). A unit is its parts back to back.
struct Part {
  std::string name, format;
  int source = 0;
  uint64_t offset = 0, stride = 0, bytes = 0;
};

struct Router {
  std::string tensor, bias, format = "F32", score = "softmax";
  uint32_t rows = 0, cols = 0;
};

struct Layer {
  int index = 0;
  LayerKind kind = LayerKind::Dense;
  uint64_t fixed_bytes = 0;
  int n_units = 0, top_k = 0, n_shared = 0;
  uint64_t unit_bytes = 0;
  std::vector<Part> parts;
  bool has_router = false;
  Router router;
  std::vector<uint64_t> hash;
  std::vector<double> benefit;
  bool streamable = true;
};

struct NamedBytes {
  std::string name;
  uint64_t bytes = 0;
};

struct LookupTable {
  std::string name, placement = "file";
  int source = 0;
  uint64_t offset = 0, rows = 0, row_bytes = 0;
};

struct Desc {
  std::string model, engine, routes;
  std::vector<NamedBytes> fixed_device, host_fixed;
  uint64_t state_bytes_per_position = 0, workspace_bytes_per_row = 0;
  uint64_t unit_align = 256;
  std::vector<Source> sources;
  Order order = Order::Ranked;
  Tiers tiers = Tiers::PinnedDisk;
  uint32_t ring_slots = 0;
  std::vector<Layer> layers;
  std::vector<LookupTable> lookup_tables;
  // derived by validate()
  std::vector<int64_t> unit_base;
  int64_t total_units = 0;
  uint64_t max_unit_bytes = 0;
  int max_units_per_layer = 0;

  uint64_t unit_stride(int layer) const;  // unit bytes rounded up to unit_align (the device slot)
  uint64_t fixed_total() const;
  int64_t gidx(int layer, int unit) const { return unit_base[size_t(layer)] + unit; }
};

Desc desc_from_json(const Json& j);  // parses and validates; throws SS_E_DESC
void desc_validate(Desc& d);
Json desc_to_json(const Desc& d);

constexpr uint64_t kGiB = uint64_t(1) << 30;
constexpr uint64_t kHostStride = 4096;
constexpr uint64_t kPinnedChunk = uint64_t(1) << 30;

struct RingClass {
  uint64_t stride = 0;
  uint32_t slots = 0;
};
struct SpareClass {
  uint64_t block_bytes = 0;
  uint32_t asked = 0, blocks = 0;
};
struct PinnedLayout {
  std::vector<uint64_t> chunk_bytes;
  std::vector<int32_t> chunk_of;    // per global unit, -1 = none
  std::vector<uint64_t> offset_of;  // inside its chunk
  uint64_t total = 0;
};

struct Plan {
  std::vector<uint8_t> tier;
  ss_budget budget{};
  uint64_t cap = 0, margin = 0, fixed = 0, dynamic = 0, ring = 0, resident = 0, pinned = 0, disk = 0, peak = 0;
  uint64_t n_resident = 0, n_pinned = 0, n_disk = 0, n_pair = 0, n_backed = 0;
  std::vector<RingClass> rings;
  std::vector<SpareClass> spares;
  uint32_t dynamic_slots_per_layer = 0;
};

uint64_t host_stride(uint64_t bytes);
uint64_t plan_margin(const ss_budget& b);
bool same_budget(const ss_budget& a, const ss_budget& b);
PinnedLayout pinned_layout(const Desc& d, const std::vector<uint8_t>& tier);
std::vector<SpareClass> spare_classes(const Desc& d, const ss_budget& b, uint64_t host_left);
Plan plan_make(const Desc& d, const ss_budget& b, const std::vector<double>& benefit);
Plan plan_from_tiers(const Desc& d, const ss_budget& b, const std::vector<uint8_t>& tiers);
std::vector<uint8_t> tiers_from_json(const Desc& d, const Json& j);
Json plan_to_json(const Desc& d, const Plan& p);

}  // namespace tsa
