// desc-v1 and plan-v1. The document formats, the refusal rules and the planner's decisions are the reference's
// (src/desc.cpp:128-413, src/plan.cpp:36-477), checked document by document against it; the structure is this
// library's: a key-tracking object reader for the descriptor, overflow-checked arithmetic through the compiler's
// builtins, and a planner whose prefix search prices every split in one backward pass.
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <set>

#include "common.hpp"

namespace tsa {
namespace {

constexpr const char* kDescSchema = "strix-stream/desc-v1";
constexpr size_t kLayerLimit = 4096;
constexpr uint64_t kUnitLimit = 65536;
constexpr uint64_t kDescByteLimit = uint64_t(1) << 56;

std::string num(uint64_t v) { return std::to_string(v); }

// ---- checked sizes ----------------------------------------------------------------------------------------------------
uint64_t plus(uint64_t a, uint64_t b, const std::string& where, ss_status st = SS_E_DESC) {
  uint64_t r = 0;
  require(!__builtin_add_overflow(a, b, &r), st, where + ": a byte count overflows 64 bits");
  return r;
}
uint64_t times(uint64_t a, uint64_t b, const std::string& where, ss_status st = SS_E_DESC) {
  uint64_t r = 0;
  require(!__builtin_mul_overflow(a, b, &r), st, where + ": a byte count overflows 64 bits");
  return r;
}
bool pow2(uint64_t v) { return v != 0 && (v & (v - 1)) == 0; }

// ---- reading -----------------------------------------------------------------------------------------------------------
// One JSON object being read into the descriptor. Each key the reader asks for is noted; finish() refuses every other
// key, except the "x-" notes an adapter may leave.
class Fields {
 public:
  Fields(const Json& j, std::string path) : j_(j), path_(std::move(path)) {
    require(j.is_object(), SS_E_DESC, path_ + ": not an object");
  }
  std::string where(const char* k) const { return path_ + "." + k; }
  const Json* get(const char* k) {
    asked_.insert(k);
    return j_.find(k);
  }
  const Json& need(const char* k) {
    const Json* v = get(k);
    require(v != nullptr, SS_E_DESC, path_ + ": \"" + k + "\" is required");
    return *v;
  }
  uint64_t count(const char* k, uint64_t absent, uint64_t limit = UINT64_MAX) {
    const Json* v = get(k);
    const uint64_t x = v ? json_u64(*v, where(k)) : absent;
    require(x <= limit, SS_E_DESC, where(k) + ": " + num(x) + " exceeds " + num(limit));
    return x;
  }
  uint64_t count_needed(const char* k) { return json_u64(need(k), where(k)); }
  std::string text(const char* k, const std::string& absent = "") {
    const Json* v = get(k);
    return v ? json_str(*v, where(k)) : absent;
  }
  std::string text_needed(const char* k) { return json_str(need(k), where(k)); }
  const std::vector<Json>* list(const char* k) {
    const Json* v = get(k);
    if (!v) return nullptr;
    require(v->is_array(), SS_E_DESC, where(k) + ": not an array");
    return &v->arr;
  }
  void finish() const {
    for (const auto& kv : j_.obj)
      require(asked_.count(kv.first) || kv.first.compare(0, 2, "x-") == 0, SS_E_DESC,
              path_ + ": unknown key \"" + kv.first + "\"");
  }

 private:
  const Json& j_;
  std::string path_;
  std::set<std::string> asked_;
};

std::string item(const std::string& path, size_t i) { return path + "[" + num(i) + "]"; }

// The element formats a part may declare (the reference's list), or any "x-" private format.
bool format_known(const std::string& f) {
  static const std::set<std::string> kFormats = {
      "F32",   "F16",    "BF16",   "FP8_E4M3", "FP8_E5M2", "EXL3",   "MXFP4",  "NVFP4", "Q2_K",    "Q3_K",  "Q4_K",
      "Q5_K",  "Q6_K",   "Q8_0",   "Q4_0",     "Q4_1",     "Q5_0",   "Q5_1",   "IQ1_S", "IQ1_M",   "IQ2_XXS", "IQ2_XS",
      "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ4_NL",   "IQ4_XS",   "TQ1_0",  "TQ2_0",  "I8",    "U8",      "mixed"};
  return kFormats.count(f) || f.compare(0, 2, "x-") == 0;
}

// A 16-digit lowercase hex xxh64.
uint64_t hash_of(const std::string& s, const std::string& where) {
  require(s.size() == 16, SS_E_DESC, where + ": an xxh64 is 16 lowercase hex digits");
  uint64_t v = 0;
  for (const char c : s) {
    const bool dec = c >= '0' && c <= '9', hex = c >= 'a' && c <= 'f';
    require(dec || hex, SS_E_DESC, where + ": an xxh64 is 16 lowercase hex digits");
    v = v << 4 | uint64_t(dec ? c - '0' : c - 'a' + 10);
  }
  return v;
}
std::string hash_text(uint64_t v) {
  char b[17];
  std::snprintf(b, sizeof b, "%016llx", static_cast<unsigned long long>(v));
  return b;
}

template <class E>
E pick(const std::string& got, const std::initializer_list<std::pair<const char*, E>>& names, const std::string& where) {
  std::string all;
  for (const auto& n : names) {
    if (got == n.first) return n.second;
    all += (all.empty() ? "" : " | ") + std::string(n.first);
  }
  fail(SS_E_DESC, where + ": \"" + got + "\" is not one of " + all);
}

const std::initializer_list<std::pair<const char*, Order>> kOrders = {{"prefix", Order::Prefix}, {"ranked", Order::Ranked}};
const std::initializer_list<std::pair<const char*, Tiers>> kTierSets = {
    {"pinned", Tiers::Pinned}, {"disk", Tiers::Disk}, {"pinned|disk", Tiers::PinnedDisk}, {"pair", Tiers::Pair}};
const std::initializer_list<std::pair<const char*, LayerKind>> kKinds = {
    {"dense", LayerKind::Dense}, {"moe", LayerKind::Moe}, {"blob", LayerKind::Blob}};

template <class E>
const char* name_of(E v, const std::initializer_list<std::pair<const char*, E>>& names) {
  for (const auto& n : names)
    if (n.second == v) return n.first;
  return "?";
}

std::vector<NamedBytes> read_named(Fields& f, const char* k) {
  std::vector<NamedBytes> out;
  const std::vector<Json>* v = f.list(k);
  for (size_t i = 0; v && i < v->size(); ++i) {
    Fields e((*v)[i], item(f.where(k), i));
    out.push_back({e.text_needed("name"), e.count_needed("bytes")});
    e.finish();
  }
  return out;
}

Part read_part(const Json& j, const std::string& path) {
  Fields f(j, path);
  Part p;
  p.name = f.text("name");
  p.format = f.text_needed("format");
  p.source = int(f.count("source", 0, 1024));
  p.offset = f.count_needed("offset");
  p.bytes = f.count_needed("bytes");
  p.stride = f.count("stride", p.bytes);
  f.finish();
  return p;
}

Layer read_layer(const Json& j, const std::string& path) {
  Fields f(j, path);
  Layer l;
  const int64_t index = json_i64(f.need("index"), f.where("index"));
  require(index >= 0 && index < int64_t(kLayerLimit), SS_E_DESC, f.where("index") + ": outside 0..4095");
  l.index = int(index);
  l.kind = pick(f.text_needed("kind"), kKinds, f.where("kind"));
  l.fixed_bytes = f.count("fixed_bytes", 0);
  l.n_units = int(f.count("n_units", l.kind == LayerKind::Blob ? 1 : 0, kUnitLimit));
  l.top_k = int(f.count("top_k", 0, kUnitLimit));
  l.n_shared = int(f.count("n_shared", 0, kUnitLimit));
  l.unit_bytes = f.count("unit_bytes", 0);
  if (const Json* s = f.get("streamable")) l.streamable = json_bool(*s, f.where("streamable"));
  if (const std::vector<Json>* parts = f.list("parts"))
    for (size_t p = 0; p < parts->size(); ++p) l.parts.push_back(read_part((*parts)[p], item(f.where("parts"), p)));
  if (const Json* r = f.get("router")) {
    Fields rf(*r, f.where("router"));
    l.has_router = true;
    l.router.tensor = rf.text_needed("tensor");
    l.router.bias = rf.text("bias");
    l.router.format = rf.text("format", "F32");
    l.router.score = rf.text("score", "softmax");
    l.router.rows = uint32_t(rf.count("rows", 0, kUnitLimit));
    l.router.cols = uint32_t(rf.count("cols", 0, uint64_t(1) << 24));
    rf.finish();
  }
  if (const Json* h = f.get("hash")) {
    require(h->is_array(), SS_E_DESC, f.where("hash") + ": not an array of xxh64 strings");
    for (size_t k = 0; k < h->arr.size(); ++k)
      l.hash.push_back(hash_of(json_str(h->arr[k], item(f.where("hash"), k)), item(f.where("hash"), k)));
  }
  if (const std::vector<Json>* b = f.list("benefit"))
    for (size_t k = 0; k < b->size(); ++k) l.benefit.push_back(json_f64((*b)[k], item(f.where("benefit"), k)));
  f.finish();
  return l;
}

// ---- rules across fields ------------------------------------------------------------------------------------------------
void check_units(const Desc& d, Layer& l, const std::string& lw) {
  require(!l.parts.empty(), SS_E_DESC, lw + ": units need at least one part");
  uint64_t sum = 0;
  for (size_t p = 0; p < l.parts.size(); ++p) {
    const Part& part = l.parts[p];
    const std::string pw = item(lw + ".parts", p);
    require(part.bytes > 0, SS_E_DESC, pw + ".bytes: zero");
    require(format_known(part.format), SS_E_DESC, pw + ".format: \"" + part.format + "\" is not a known format");
    require(part.source >= 0 && size_t(part.source) < d.sources.size(), SS_E_DESC,
            pw + ".source: " + num(uint64_t(part.source)) + " names no source");
    require(l.n_units == 1 || part.stride >= part.bytes, SS_E_DESC, pw + ".stride: below bytes, so units overlap");
    sum = plus(sum, part.bytes, pw);
    plus(plus(part.offset, times(uint64_t(l.n_units - 1), part.stride, pw), pw), part.bytes, pw);  // the last byte
  }
  if (l.unit_bytes == 0) l.unit_bytes = sum;
  require(l.unit_bytes == sum, SS_E_DESC,
          lw + ".unit_bytes: " + num(l.unit_bytes) + " but the parts add up to " + num(sum));
  times(plus(l.unit_bytes, d.unit_align, lw), uint64_t(l.n_units), lw);
  require(l.hash.empty() || l.hash.size() == size_t(l.n_units), SS_E_DESC, lw + ".hash: not one per unit");
  require(l.benefit.empty() || l.benefit.size() == size_t(l.n_units), SS_E_DESC, lw + ".benefit: not one per unit");
  require(!l.has_router || l.router.rows == 0 || l.router.rows == uint32_t(l.n_units), SS_E_DESC,
          lw + ".router.rows: not n_units");
}

void check_kind(const Layer& l, const std::string& lw) {
  switch (l.kind) {
    case LayerKind::Dense:
      require(l.n_units == 0 && l.parts.empty(), SS_E_DESC, lw + ": a dense layer has fixed bytes only, no units");
      break;
    case LayerKind::Blob:
      require(l.n_units == 1, SS_E_DESC, lw + ": a blob layer is one unit");
      break;
    case LayerKind::Moe:
      require(l.n_units >= 1, SS_E_DESC, lw + ": a moe layer needs units");
      require(l.top_k >= 1 && l.top_k <= l.n_units, SS_E_DESC, lw + ".top_k: outside 1..n_units");
      break;
  }
}

}  // namespace

uint64_t Desc::unit_stride(int layer) const {
  const uint64_t b = layers[size_t(layer)].unit_bytes;
  return (b + unit_align - 1) / unit_align * unit_align;
}

uint64_t Desc::fixed_total() const {
  uint64_t t = 0;
  for (const NamedBytes& n : fixed_device) t += n.bytes;
  for (size_t L = 0; L < layers.size(); ++L)
    t += layers[L].fixed_bytes + (layers[L].streamable ? 0 : uint64_t(layers[L].n_units) * unit_stride(int(L)));
  return t;
}

Desc desc_from_json(const Json& j) {
  Fields f(j, "desc");
  const std::string schema = f.text_needed("schema");
  // the renamed project's "tierstream/" prefix reads as the same format
  require(schema == kDescSchema || schema == "tierstream/desc-v1", SS_E_DESC,
          "desc.schema: \"" + schema + "\" is not " + kDescSchema);
  Desc d;
  d.model = f.text("model");
  d.engine = f.text("engine");
  d.fixed_device = read_named(f, "fixed_device");
  d.host_fixed = read_named(f, "host_fixed");
  d.state_bytes_per_position = f.count("state_bytes_per_position", 0);
  d.workspace_bytes_per_row = f.count("workspace_bytes_per_row", 0);
  d.unit_align = f.count("unit_align", 256);
  d.ring_slots = uint32_t(f.count("ring_slots", 0, uint64_t(1) << 20));
  d.routes = f.text("routes");
  d.order = pick(f.text("order", "ranked"), kOrders, "desc.order");
  d.tiers = pick(f.text("tiers", "pinned|disk"), kTierSets, "desc.tiers");
  if (const std::vector<Json>* s = f.list("sources"))
    for (size_t i = 0; i < s->size(); ++i) {
      Fields sf((*s)[i], item("desc.sources", i));
      Source src;
      src.name = sf.text("name");
      src.path = sf.text_needed("path");
      src.align = sf.count("align", 4096);
      sf.finish();
      d.sources.push_back(src);
    }
  const Json& layers = f.need("layers");
  require(layers.is_array(), SS_E_DESC, "desc.layers: not an array");
  for (size_t i = 0; i < layers.arr.size(); ++i) d.layers.push_back(read_layer(layers.arr[i], item("desc.layers", i)));
  if (const std::vector<Json>* t = f.list("lookup_tables"))
    for (size_t i = 0; i < t->size(); ++i) {
      Fields tf((*t)[i], item("desc.lookup_tables", i));
      LookupTable lt;
      lt.name = tf.text_needed("name");
      lt.source = int(tf.count("source", 0, 1024));
      lt.offset = tf.count("offset", 0);
      lt.rows = tf.count_needed("rows");
      lt.row_bytes = tf.count_needed("row_bytes");
      lt.placement = tf.text("placement", "file");
      tf.finish();
      d.lookup_tables.push_back(lt);
    }
  f.finish();
  desc_validate(d);
  return d;
}

void desc_validate(Desc& d) {
  require(!d.layers.empty() && d.layers.size() <= kLayerLimit, SS_E_DESC, "desc.layers: needs 1..4096 layers");
  require(pow2(d.unit_align), SS_E_DESC, "desc.unit_align: not a power of two");
  for (size_t s = 0; s < d.sources.size(); ++s)
    require(pow2(d.sources[s].align) && d.sources[s].align <= (uint64_t(1) << 20), SS_E_DESC,
            item("desc.sources", s) + ".align: not a power of two up to 1 MiB");
  d.unit_base.assign(d.layers.size(), 0);
  d.total_units = 0;
  d.max_unit_bytes = 0;
  d.max_units_per_layer = 0;
  for (size_t i = 0; i < d.layers.size(); ++i) {
    Layer& l = d.layers[i];
    const std::string lw = item("desc.layers", i);
    require(l.index == int(i), SS_E_DESC, lw + ".index: layers are listed 0, 1, ... in order");
    require(l.n_units >= 0 && uint64_t(l.n_units) <= kUnitLimit, SS_E_DESC, lw + ".n_units: outside 0..65536");
    check_kind(l, lw);
    if (l.n_units > 0) {
      check_units(d, l, lw);
      if (l.streamable) {
        d.max_unit_bytes = std::max(d.max_unit_bytes, l.unit_bytes);
        d.max_units_per_layer = std::max(d.max_units_per_layer, l.n_units);
      }
    }
    d.unit_base[i] = d.total_units;
    d.total_units += l.n_units;
  }
  // everything the model could occupy, each unit at its host stride: below 2^56 bytes
  uint64_t device = 0, host = 0;
  for (const NamedBytes& n : d.fixed_device) device = plus(device, n.bytes, "desc.fixed_device");
  for (const NamedBytes& n : d.host_fixed) host = plus(host, n.bytes, "desc.host_fixed");
  uint64_t everything = plus(device, host, "desc");
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const std::string lw = item("desc.layers", L);
    everything = plus(everything, times(uint64_t(d.layers[L].n_units), plus(d.layers[L].unit_bytes, 4096, lw), lw), lw);
  }
  require(everything < kDescByteLimit, SS_E_DESC, "desc: the model's bytes reach 2^56");
  for (size_t L = 0; L < d.layers.size(); ++L) {  // the fixed device total must fit 64 bits too
    const std::string lw = item("desc.layers", L);
    device = plus(device, d.layers[L].fixed_bytes, lw + ".fixed_bytes");
    if (!d.layers[L].streamable)
      device = plus(device, times(uint64_t(d.layers[L].n_units), d.unit_stride(int(L)), lw), lw);
  }
  for (size_t i = 0; i < d.lookup_tables.size(); ++i) {
    const LookupTable& t = d.lookup_tables[i];
    const std::string tw = item("desc.lookup_tables", i);
    require(t.source >= 0 && size_t(t.source) < d.sources.size(), SS_E_DESC, tw + ".source: names no source");
    require(t.placement == "file" || t.placement == "pinned" || t.placement == "device", SS_E_DESC,
            tw + ".placement: \"" + t.placement + "\" is not file | pinned | device");
  }
}

Json desc_to_json(const Desc& d) {
  const auto str = [](const std::string& s) { return Json::string(s); };
  const auto u = [](uint64_t v) { return Json::number(v); };
  const auto i = [](int64_t v) { return Json::number_i(v); };
  const auto named = [&](const std::vector<NamedBytes>& v) {
    Json a = Json::array();
    for (const NamedBytes& n : v) {
      Json e = Json::object();
      e["name"] = str(n.name);
      e["bytes"] = u(n.bytes);
      a.push(e);
    }
    return a;
  };
  Json j = Json::object();
  j["schema"] = str(kDescSchema);
  if (!d.model.empty()) j["model"] = str(d.model);
  if (!d.engine.empty()) j["engine"] = str(d.engine);
  if (!d.routes.empty()) j["routes"] = str(d.routes);
  j["fixed_device"] = named(d.fixed_device);
  j["host_fixed"] = named(d.host_fixed);
  j["state_bytes_per_position"] = u(d.state_bytes_per_position);
  j["workspace_bytes_per_row"] = u(d.workspace_bytes_per_row);
  j["unit_align"] = u(d.unit_align);
  j["order"] = str(name_of(d.order, kOrders));
  j["tiers"] = str(name_of(d.tiers, kTierSets));
  j["ring_slots"] = u(d.ring_slots);
  j["sources"] = Json::array();
  for (const Source& s : d.sources) {
    Json e = Json::object();
    if (!s.name.empty()) e["name"] = str(s.name);
    e["path"] = str(s.path);
    e["align"] = u(s.align);
    j["sources"].push(e);
  }
  j["layers"] = Json::array();
  for (const Layer& l : d.layers) {
    Json e = Json::object();
    e["index"] = i(l.index);
    e["kind"] = str(name_of(l.kind, kKinds));
    e["fixed_bytes"] = u(l.fixed_bytes);
    if (l.top_k) e["top_k"] = i(l.top_k);
    if (l.n_shared) e["n_shared"] = i(l.n_shared);
    if (l.n_units > 0) {
      e["n_units"] = i(l.n_units);
      e["unit_bytes"] = u(l.unit_bytes);
      e["streamable"] = Json::boolean(l.streamable);
      e["parts"] = Json::array();
      for (const Part& p : l.parts) {
        Json pj = Json::object();
        if (!p.name.empty()) pj["name"] = str(p.name);
        pj["format"] = str(p.format);
        pj["source"] = i(p.source);
        pj["offset"] = u(p.offset);
        pj["stride"] = u(p.stride);
        pj["bytes"] = u(p.bytes);
        e["parts"].push(pj);
      }
      if (!l.hash.empty()) {
        e["hash"] = Json::array();
        for (uint64_t h : l.hash) e["hash"].push(str(hash_text(h)));
      }
      if (!l.benefit.empty()) {
        e["benefit"] = Json::array();
        for (double b : l.benefit) e["benefit"].push(Json::number_f(b));
      }
    }
    if (l.has_router) {
      Json r = Json::object();
      r["tensor"] = str(l.router.tensor);
      if (!l.router.bias.empty()) r["bias"] = str(l.router.bias);
      r["format"] = str(l.router.format);
      r["score"] = str(l.router.score);
      r["rows"] = u(l.router.rows);
      r["cols"] = u(l.router.cols);
      e["router"] = r;
    }
    j["layers"].push(e);
  }
  j["lookup_tables"] = Json::array();
  for (const LookupTable& t : d.lookup_tables) {
    Json e = Json::object();
    e["name"] = str(t.name);
    e["source"] = i(t.source);
    e["offset"] = u(t.offset);
    e["rows"] = u(t.rows);
    e["row_bytes"] = u(t.row_bytes);
    e["placement"] = str(t.placement);
    j["lookup_tables"].push(e);
  }
  return j;
}

// ---- the planner ----------------------------------------------------------------------------------------------------------
namespace {

std::string gib(uint64_t n) {
  char b[32];
  std::snprintf(b, sizeof b, "%.3f", double(n) / double(kGiB));
  return b;
}

bool exclusive(const ss_budget& b) { return b.tier_mode == SS_TIER_MODE_EXCLUSIVE; }
bool has_pinned_copy(uint8_t t) { return t == SS_TIER_PINNED || t == SS_TIER_RESIDENT_BACKED; }
bool on_device(uint8_t t) { return t == SS_TIER_RESIDENT || t == SS_TIER_RESIDENT_BACKED; }

// A streamable unit as the planner ranks it: model key, layer, device slot bytes, benefit.
struct Streamed {
  int64_t key;
  int layer;
  uint64_t slot;
  double value;
};

// Denser (benefit per slot byte) first; model order among equals. A total order on distinct keys.
bool denser(const Streamed& a, const Streamed& b) {
  const double inf = std::numeric_limits<double>::infinity();
  const double x = a.slot ? a.value / double(a.slot) : inf, y = b.slot ? b.value / double(b.slot) : inf;
  return x != y ? x > y : a.key < b.key;
}

// Every streamable unit in model order, valued by the caller's benefit, else the descriptor's, else 1.
std::vector<Streamed> streamable_units(const Desc& d, const std::vector<double>& benefit) {
  std::vector<Streamed> v;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    if (!l.streamable) continue;
    for (int u = 0; u < l.n_units; ++u) {
      const int64_t key = d.unit_base[L] + u;
      const double b = !benefit.empty() ? benefit[size_t(key)] : !l.benefit.empty() ? l.benefit[size_t(u)] : 1.0;
      require(std::isfinite(b) && b >= 0, SS_E_INVALID, "plan: a benefit is negative or not finite");
      v.push_back({key, int(L), d.unit_stride(int(L)), b});
    }
  }
  return v;
}

// Ring slots for a slot size: the budget's, else the descriptor's, else twice the most units of any streamable layer
// with that slot size.
uint32_t ring_slots_for(const Desc& d, const ss_budget& b, uint64_t stride) {
  if (b.ring_slots) return b.ring_slots;
  if (d.ring_slots) return d.ring_slots;
  uint32_t n = 0;
  for (size_t L = 0; L < d.layers.size(); ++L)
    if (d.layers[L].streamable && d.layers[L].n_units && d.unit_stride(int(L)) == stride)
      n = std::max(n, uint32_t(2 * d.layers[L].n_units));
  return n;
}

// One ring per distinct nonzero slot size among `slots`, by size (none with the pair tier set).
std::vector<RingClass> rings_for(const Desc& d, const ss_budget& b, const std::vector<uint64_t>& slots) {
  std::vector<RingClass> out;
  if (d.tiers == Tiers::Pair) return out;
  std::set<uint64_t> sizes(slots.begin(), slots.end());
  sizes.erase(0);
  for (uint64_t s : sizes) out.push_back({s, ring_slots_for(d, b, s)});
  return out;
}

uint64_t ring_bytes(const std::vector<RingClass>& r) {
  uint64_t t = 0;
  for (const RingClass& c : r) t += c.stride * c.slots;
  return t;
}

// The device bytes the dynamic slots take at most (before any unit is placed).
uint64_t dynamic_ceiling(const Desc& d, const ss_budget& b) {
  uint64_t t = 0;
  for (size_t L = 0; b.dynamic_slots_per_layer && L < d.layers.size(); ++L)
    if (d.layers[L].streamable && d.layers[L].n_units > 0)
      t += uint64_t(std::min<uint32_t>(b.dynamic_slots_per_layer, uint32_t(d.layers[L].n_units))) *
           d.unit_stride(int(L));
  return t;
}

// The budget's own rules and the fixed bill, before any unit is placed.
Plan open_plan(const Desc& d, const ss_budget& b) {
  require(b.device_bytes > 0, SS_E_INVALID, "plan: no device budget");
  require(b.tier_mode == SS_TIER_MODE_INCLUSIVE || b.tier_mode == SS_TIER_MODE_EXCLUSIVE, SS_E_INVALID,
          "plan: tier_mode is neither inclusive nor exclusive");
  if (exclusive(b)) {
    require(!b.pinned_backing, SS_E_INVALID,
            "plan: pinned_backing asks for the second pinned copy of residents that the exclusive mode gives up");
    require(d.tiers == Tiers::Pinned || d.tiers == Tiers::PinnedDisk, SS_E_INVALID,
            d.engine + ": the exclusive mode needs a pinned tier, and the descriptor's tiers have none");
  }
  Plan p;
  p.budget = b;
  p.cap = b.device_bytes;
  p.margin = plan_margin(b);
  p.tier.assign(size_t(d.total_units), SS_TIER_RESIDENT);
  p.dynamic_slots_per_layer = b.dynamic_slots_per_layer;
  p.fixed = d.fixed_total() + b.workspace_bytes;
  p.dynamic = dynamic_ceiling(d, b);
  require(p.cap >= p.margin + p.fixed + p.dynamic, SS_E_CAPACITY,
          d.engine + ": the " + gib(p.cap) + " GiB cap holds neither fixed " + gib(p.fixed) + " GiB + dynamic " +
              gib(p.dynamic) + " GiB + margin " + gib(p.margin) + " GiB");
  return p;
}

// Which units stay on the device. Prefix order: the longest model-order prefix that fits with the rings of the rest
// (each split priced in one backward pass). Ranked: everything if it fits, else the rings of everything first and then
// the densest units that still fit, skipping any that does not.
std::vector<char> choose_residents(const Desc& d, const ss_budget& b, const std::vector<Streamed>& units, uint64_t room,
                                   bool* ok) {
  const size_t n = units.size();
  std::vector<char> keep(n, 0);
  uint64_t all = 0;
  for (const Streamed& s : units) all += s.slot;
  *ok = true;
  if (d.order == Order::Prefix) {
    // ring[k]: the rings of units[k..n); prefix[k]: the slots of units[0..k)
    std::vector<uint64_t> ring(n + 1, 0);
    std::set<uint64_t> seen;
    for (size_t k = n; k-- > 0;) {
      ring[k] = ring[k + 1];
      if (d.tiers != Tiers::Pair && units[k].slot && seen.insert(units[k].slot).second)
        ring[k] += units[k].slot * ring_slots_for(d, b, units[k].slot);
    }
    uint64_t prefix = all;
    for (size_t k = n + 1; k-- > 0;) {
      if (prefix + ring[k] <= room) {
        std::fill(keep.begin(), keep.begin() + std::ptrdiff_t(k), char(1));
        return keep;
      }
      if (k) prefix -= units[k - 1].slot;
    }
    *ok = false;
    return keep;
  }
  if (all <= room) {
    std::fill(keep.begin(), keep.end(), char(1));
    return keep;
  }
  std::vector<uint64_t> slots;
  for (const Streamed& s : units) slots.push_back(s.slot);
  const uint64_t rings = ring_bytes(rings_for(d, b, slots));
  if (rings > room) {
    *ok = false;
    return keep;
  }
  std::vector<size_t> by_density(n);
  for (size_t i = 0; i < n; ++i) by_density[i] = i;
  std::sort(by_density.begin(), by_density.end(), [&](size_t a, size_t c) { return denser(units[a], units[c]); });
  uint64_t left = room - rings;
  for (size_t i : by_density)
    if (units[i].slot <= left) {
      keep[i] = 1;
      left -= units[i].slot;
    }
  return keep;
}

uint64_t host_budget_after_fixed(const Desc& d, const ss_budget& b) {
  uint64_t left = b.host_pinned_bytes;
  for (const NamedBytes& n : d.host_fixed) left = left > n.bytes ? left - n.bytes : 0;
  return left;
}

// pinned_backing: residents take a pinned copy, least dense first, while the host budget left after host_fixed and
// the pinned tier lasts; the first that does not fit ends it.
void back_residents(const Desc& d, const ss_budget& b, const std::vector<Streamed>& units, std::vector<uint8_t>& tier) {
  uint64_t left = host_budget_after_fixed(d, b);
  std::vector<Streamed> res;
  for (const Streamed& s : units) {
    if (tier[size_t(s.key)] == SS_TIER_PINNED) {
      const uint64_t hb = host_stride(d.layers[size_t(s.layer)].unit_bytes);
      left = left > hb ? left - hb : 0;
    } else if (tier[size_t(s.key)] == SS_TIER_RESIDENT) {
      res.push_back(s);
    }
  }
  std::sort(res.begin(), res.end(), [](const Streamed& x, const Streamed& y) { return denser(y, x); });
  for (const Streamed& s : res) {
    const uint64_t hb = host_stride(d.layers[size_t(s.layer)].unit_bytes);
    if (hb > left) return;
    tier[size_t(s.key)] = SS_TIER_RESIDENT_BACKED;
    left -= hb;
  }
}

// The bill of a complete tier assignment (made here or handed in): every tier checked, the device and host totals,
// the rings of the streamed units, the spare blocks; then both budgets.
void bill(const Desc& d, const ss_budget& b, Plan& p) {
  std::vector<uint64_t> streamed_slots;
  p.resident = p.pinned = p.disk = p.dynamic = 0;
  p.n_resident = p.n_pinned = p.n_disk = p.n_pair = p.n_backed = 0;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    const uint64_t stride = d.unit_stride(int(L));
    int on_dev = 0;
    for (int u = 0; u < l.n_units; ++u) {
      const uint8_t t = p.tier[size_t(d.unit_base[L] + u)];
      require(t <= SS_TIER_RESIDENT_BACKED, SS_E_INVALID, "plan: tier value " + num(t) + " is not a tier");
      if (!l.streamable) {
        require(t == SS_TIER_RESIDENT, SS_E_INVALID, "plan: a layer that cannot stream keeps its units resident");
        continue;
      }
      require(!(exclusive(b) && t == SS_TIER_RESIDENT_BACKED), SS_E_INVALID,
              "plan: tier B keeps a second pinned copy, which the exclusive mode gives up");
      switch (t) {
        case SS_TIER_RESIDENT_BACKED: ++p.n_backed; [[fallthrough]];
        case SS_TIER_RESIDENT:
          p.resident += stride;
          ++p.n_resident;
          ++on_dev;
          break;
        case SS_TIER_PINNED:
          ++p.n_pinned;
          streamed_slots.push_back(stride);
          break;
        case SS_TIER_DISK:
          ++p.n_disk;
          p.disk += l.unit_bytes;
          streamed_slots.push_back(stride);
          break;
        default: ++p.n_pair; break;
      }
    }
    if (l.streamable && l.n_units > 0 && b.dynamic_slots_per_layer)
      p.dynamic += uint64_t(std::min<uint32_t>(b.dynamic_slots_per_layer, uint32_t(l.n_units - on_dev))) * stride;
  }
  const uint64_t layout = pinned_layout(d, p.tier).total;
  p.pinned = layout;
  for (const NamedBytes& n : d.host_fixed) p.pinned += n.bytes;
  require(p.pinned >= layout, SS_E_INVALID, "plan: the host total overflows 64 bits");
  p.spares = spare_classes(d, b, b.host_pinned_bytes > p.pinned ? b.host_pinned_bytes - p.pinned : 0);
  for (const SpareClass& c : p.spares) {
    const uint64_t blocks = times(c.block_bytes, c.blocks, "plan: spare blocks", SS_E_INVALID);
    p.pinned = plus(p.pinned, blocks, "plan: spare blocks", SS_E_INVALID);
  }
  p.rings = rings_for(d, b, streamed_slots);
  p.ring = ring_bytes(p.rings);
  require(p.pinned <= b.host_pinned_bytes, SS_E_CAPACITY,
          d.engine + ": " + gib(p.pinned) + " GiB must be pinned but the host budget is " + gib(b.host_pinned_bytes) +
              " GiB");
  p.peak = p.fixed + p.dynamic + p.ring + p.resident;
  require(p.peak + p.margin <= p.cap, SS_E_CAPACITY,
          d.engine + ": the predicted peak " + gib(p.peak) + " GiB + margin " + gib(p.margin) + " GiB is above the " +
              gib(p.cap) + " GiB cap");
}

}  // namespace

uint64_t host_stride(uint64_t bytes) {
  require(bytes <= UINT64_MAX - (kHostStride - 1), SS_E_INVALID, "plan: a unit's host stride overflows 64 bits");
  return (bytes + kHostStride - 1) & ~(kHostStride - 1);
}

uint64_t plan_margin(const ss_budget& b) {
  return uint64_t(std::max(b.margin_gib * double(kGiB), b.margin_fraction * double(b.device_bytes)));
}

bool same_budget(const ss_budget& a, const ss_budget& b) {
  return a.device_bytes == b.device_bytes && a.host_pinned_bytes == b.host_pinned_bytes &&
         a.workspace_bytes == b.workspace_bytes && a.margin_gib == b.margin_gib &&
         a.margin_fraction == b.margin_fraction && a.dynamic_slots_per_layer == b.dynamic_slots_per_layer &&
         a.ring_slots == b.ring_slots && a.pinned_backing == b.pinned_backing && a.tier_mode == b.tier_mode &&
         a.host_spare_units == b.host_spare_units;
}

// Units with a pinned copy, in model order at 4 KiB host strides, packed into chunks of at most 1 GiB (a unit larger
// than that alone in its chunk).
PinnedLayout pinned_layout(const Desc& d, const std::vector<uint8_t>& tier) {
  PinnedLayout pl;
  pl.chunk_of.assign(size_t(d.total_units), -1);
  pl.offset_of.assign(size_t(d.total_units), 0);
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const uint64_t st = host_stride(d.layers[L].unit_bytes);
    for (int u = 0; u < d.layers[L].n_units; ++u) {
      const size_t key = size_t(d.unit_base[L] + u);
      if (!has_pinned_copy(tier[key])) continue;
      if (pl.chunk_bytes.empty() || pl.chunk_bytes.back() + st > kPinnedChunk) pl.chunk_bytes.push_back(0);
      pl.chunk_of[key] = int32_t(pl.chunk_bytes.size() - 1);
      pl.offset_of[key] = pl.chunk_bytes.back();
      pl.chunk_bytes.back() += st;
    }
  }
  for (uint64_t c : pl.chunk_bytes) pl.total = plus(pl.total, c, "plan: pinned layout", SS_E_INVALID);
  return pl;
}

// Exclusive mode: per distinct host stride of the streamable units, up to host_spare_units (default 64, at most the
// units of that stride) spare blocks, granted smallest blocks first from what is left of the host budget.
std::vector<SpareClass> spare_classes(const Desc& d, const ss_budget& b, uint64_t host_left) {
  std::vector<SpareClass> out;
  if (!exclusive(b)) return out;
  std::map<uint64_t, uint64_t> units_of;  // host stride -> streamable units
  for (const Layer& l : d.layers)
    if (l.streamable && l.n_units) units_of[host_stride(l.unit_bytes)] += uint64_t(l.n_units);
  const uint64_t want = b.host_spare_units ? b.host_spare_units : 64;
  for (const auto& kv : units_of) {  // by block size
    SpareClass c{kv.first, uint32_t(std::min(want, kv.second)), 0};
    c.blocks = uint32_t(std::min<uint64_t>(c.asked, host_left / c.block_bytes));
    host_left -= uint64_t(c.blocks) * c.block_bytes;
    out.push_back(c);
  }
  return out;
}

Plan plan_make(const Desc& d, const ss_budget& b, const std::vector<double>& benefit) {
  require(benefit.empty() || int64_t(benefit.size()) == d.total_units, SS_E_INVALID,
          "plan: the benefit list needs one value per unit (ss_desc_total_units)");
  Plan p = open_plan(d, b);
  const std::vector<Streamed> units = streamable_units(d, benefit);
  bool fits = false;
  const std::vector<char> keep = choose_residents(d, b, units, p.cap - p.margin - p.fixed - p.dynamic, &fits);
  require(fits, SS_E_CAPACITY,
          d.engine + ": nothing fits under the " + gib(p.cap) + " GiB cap once fixed " + gib(p.fixed) +
              " GiB, margin " + gib(p.margin) + " GiB and the stream rings are taken");
  // the rest by the descriptor's tier set; pinned|disk: pinned while the host budget lasts, densest first
  std::vector<Streamed> spill;
  for (size_t i = 0; i < units.size(); ++i) {
    if (keep[i]) continue;
    uint8_t& t = p.tier[size_t(units[i].key)];
    switch (d.tiers) {
      case Tiers::Pinned: t = SS_TIER_PINNED; break;
      case Tiers::Disk: t = SS_TIER_DISK; break;
      case Tiers::Pair: t = SS_TIER_PAIR; break;
      case Tiers::PinnedDisk: spill.push_back(units[i]); break;
    }
  }
  std::sort(spill.begin(), spill.end(), denser);
  uint64_t host_left = host_budget_after_fixed(d, b);
  for (const Streamed& s : spill) {
    const uint64_t hb = host_stride(d.layers[size_t(s.layer)].unit_bytes);
    const bool pin = hb <= host_left;
    p.tier[size_t(s.key)] = pin ? SS_TIER_PINNED : SS_TIER_DISK;
    if (pin) host_left -= hb;
  }
  if (b.pinned_backing) back_residents(d, b, units, p.tier);
  bill(d, b, p);
  return p;
}

Plan plan_from_tiers(const Desc& d, const ss_budget& b, const std::vector<uint8_t>& tiers) {
  require(int64_t(tiers.size()) == d.total_units, SS_E_INVALID, "plan: one tier per unit (ss_desc_total_units)");
  Plan p = open_plan(d, b);
  p.tier = tiers;
  bill(d, b, p);
  return p;
}

namespace {
constexpr char kTierLetters[] = "RPDXB";  // by ss_tier value: resident, pinned, disk, pair, resident with a pinned copy
}

Json plan_to_json(const Desc& d, const Plan& p) {
  const auto u = [](uint64_t v) { return Json::number(v); };
  Json j = Json::object();
  j["schema"] = Json::string("strix-stream/plan-v1");
  j["engine"] = Json::string(d.engine);
  j["cap_bytes"] = u(p.cap);
  j["margin_bytes"] = u(p.margin);
  j["fixed_bytes"] = u(p.fixed);
  j["dynamic_bytes"] = u(p.dynamic);
  j["dynamic_slots_per_layer"] = u(p.dynamic_slots_per_layer);
  j["ring_bytes"] = u(p.ring);
  j["rings"] = Json::array();
  for (const RingClass& c : p.rings) {
    Json r = Json::object();
    r["slot_bytes"] = u(c.stride);
    r["slots"] = u(c.slots);
    j["rings"].push(r);
  }
  j["resident_bytes"] = u(p.resident);
  j["pinned_bytes"] = u(p.pinned);
  j["disk_bytes"] = u(p.disk);
  j["peak_bytes"] = u(p.peak);
  j["n_resident"] = u(p.n_resident);
  j["n_pinned"] = u(p.n_pinned);
  j["n_disk"] = u(p.n_disk);
  j["n_pair"] = u(p.n_pair);
  j["n_backed"] = u(p.n_backed);
  if (exclusive(p.budget)) {
    j["tier_mode"] = Json::string("exclusive");
    j["spare_blocks"] = Json::array();
    for (const SpareClass& c : p.spares) {
      Json x = Json::object();
      x["block_bytes"] = u(c.block_bytes);
      x["asked"] = u(c.asked);
      x["blocks"] = u(c.blocks);
      j["spare_blocks"].push(x);
    }
  }
  j["tiers"] = Json::array();
  for (size_t L = 0; L < d.layers.size(); ++L) {
    std::string s(size_t(d.layers[L].n_units), '?');
    for (size_t u2 = 0; u2 < s.size(); ++u2) s[u2] = kTierLetters[p.tier[size_t(d.unit_base[L]) + u2]];
    j["tiers"].push(Json::string(s));
  }
  return j;
}

std::vector<uint8_t> tiers_from_json(const Desc& d, const Json& j) {
  const Json* t = j.find("tiers");
  require(t && t->is_array() && t->arr.size() == d.layers.size(), SS_E_DESC,
          "plan json: \"tiers\" is not one string per layer");
  std::vector<uint8_t> out;
  out.reserve(size_t(d.total_units));
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const std::string& s = json_str(t->arr[L], "plan.tiers");
    require(s.size() == size_t(d.layers[L].n_units), SS_E_DESC,
            "plan json: tiers[" + num(L) + "] is not one letter per unit");
    for (const char c : s) {
      const char* at = c ? std::strchr(kTierLetters, c) : nullptr;
      require(at != nullptr, SS_E_DESC, "plan json: '" + std::string(1, c) + "' is not a tier letter (R P D X B)");
      out.push_back(uint8_t(at - kTierLetters));
    }
  }
  return out;
}

}  // namespace tsa
