// desc-v1 and plan-v1: parsing, validation, the planner. The rules (and so every tier decision) are those of reference
// src/desc.cpp:128-413 and src/plan.cpp:317-477; the code is this library's own.
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
constexpr int kMaxLayers = 4096;
constexpr int kMaxUnits = 1 << 16;

// "strix-stream/<x>" also accepts the renamed "tierstream/<x>".
bool schema_ok(const std::string& got, const std::string& emitted) {
  if (got == emitted) return true;
  const std::string old = "strix-stream/";
  return emitted.rfind(old, 0) == 0 && got == "tierstream/" + emitted.substr(old.size());
}

std::string idx(const std::string& base, size_t i) { return base + "[" + std::to_string(i) + "]"; }

uint64_t add_ck(uint64_t a, uint64_t b, const std::string& w) {
  require(a <= UINT64_MAX - b, SS_E_DESC, w + ": byte arithmetic overflows 64 bits");
  return a + b;
}
uint64_t mul_ck(uint64_t a, uint64_t b, const std::string& w) {
  require(a == 0 || b <= UINT64_MAX / a, SS_E_DESC, w + ": byte arithmetic overflows 64 bits");
  return a * b;
}
uint64_t capped(uint64_t v, uint64_t max, const std::string& w) {
  require(v <= max, SS_E_DESC, w + ": " + std::to_string(v) + " is above the limit " + std::to_string(max));
  return v;
}

const Json& need(const Json& o, const char* k, const std::string& w) {
  const Json* v = o.find(k);
  require(v != nullptr, SS_E_DESC, w + ": missing \"" + k + "\"");
  return *v;
}
uint64_t u64_or(const Json& o, const char* k, const std::string& w, uint64_t d) {
  const Json* v = o.find(k);
  return v ? json_u64(*v, w + "." + k) : d;
}
std::string str_or(const Json& o, const char* k, const std::string& w, const std::string& d = "") {
  const Json* v = o.find(k);
  return v ? json_str(*v, w + "." + k) : d;
}

void only_keys(const Json& o, const std::string& w, std::initializer_list<const char*> keys) {
  require(o.is_object(), SS_E_DESC, w + ": expected an object");
  for (const auto& kv : o.obj) {
    if (kv.first.rfind("x-", 0) == 0) continue;  // adapter notes
    bool ok = false;
    for (const char* k : keys) ok = ok || kv.first == k;
    require(ok, SS_E_DESC, w + ": unknown key \"" + kv.first + "\"");
  }
}

std::vector<NamedBytes> named(const Json* v, const std::string& w) {
  std::vector<NamedBytes> out;
  if (!v) return out;
  require(v->is_array(), SS_E_DESC, w + ": expected an array");
  for (size_t i = 0; i < v->arr.size(); ++i) {
    const Json& e = v->arr[i];
    const std::string ew = idx(w, i);
    only_keys(e, ew, {"name", "bytes"});
    out.push_back({json_str(need(e, "name", ew), ew + ".name"), json_u64(need(e, "bytes", ew), ew + ".bytes")});
  }
  return out;
}

bool known_format(const std::string& f) {
  static const char* known[] = {"F32",   "F16",    "BF16",    "FP8_E4M3", "FP8_E5M2", "EXL3",   "MXFP4",  "NVFP4",
                                "Q2_K",  "Q3_K",   "Q4_K",    "Q5_K",     "Q6_K",     "Q8_0",   "Q4_0",   "Q4_1",
                                "Q5_0",  "Q5_1",   "IQ1_S",   "IQ1_M",    "IQ2_XXS",  "IQ2_XS", "IQ2_S",  "IQ3_XXS",
                                "IQ3_S", "IQ4_NL", "IQ4_XS",  "TQ1_0",    "TQ2_0",    "I8",     "U8",     "mixed"};
  for (const char* k : known)
    if (f == k) return true;
  return f.rfind("x-", 0) == 0;
}

std::string hex16(uint64_t v) {
  char b[17];
  std::snprintf(b, sizeof b, "%016llx", static_cast<unsigned long long>(v));
  return b;
}
uint64_t parse_hex16(const std::string& s, const std::string& w) {
  require(s.size() == 16, SS_E_DESC, w + ": expected 16 hex digits");
  uint64_t v = 0;
  for (char c : s) {
    v <<= 4;
    if (c >= '0' && c <= '9') v |= uint64_t(c - '0');
    else if (c >= 'a' && c <= 'f') v |= uint64_t(c - 'a' + 10);
    else fail(SS_E_DESC, w + ": expected lowercase hex digits");
  }
  return v;
}

const char* tiers_text(Tiers t) {
  switch (t) {
    case Tiers::Pinned: return "pinned";
    case Tiers::Disk: return "disk";
    case Tiers::PinnedDisk: return "pinned|disk";
    case Tiers::Pair: return "pair";
  }
  return "?";
}

std::string gib(uint64_t n) {
  char b[32];
  std::snprintf(b, sizeof b, "%.3f", double(n) / double(kGiB));
  return b;
}

}  // namespace

uint64_t Desc::unit_stride(int layer) const {
  const uint64_t b = layers[size_t(layer)].unit_bytes;
  return (b + unit_align - 1) / unit_align * unit_align;
}

uint64_t Desc::fixed_total() const {
  uint64_t t = 0;
  for (const auto& n : fixed_device) t += n.bytes;
  for (size_t L = 0; L < layers.size(); ++L) {
    t += layers[L].fixed_bytes;
    if (!layers[L].streamable) t += uint64_t(layers[L].n_units) * unit_stride(int(L));
  }
  return t;
}

Desc desc_from_json(const Json& j) {
  const std::string w = "desc";
  only_keys(j, w,
            {"schema", "model", "engine", "fixed_device", "host_fixed", "state_bytes_per_position",
             "workspace_bytes_per_row", "unit_align", "sources", "order", "tiers", "ring_slots", "routes", "layers",
             "lookup_tables"});
  require(schema_ok(json_str(need(j, "schema", w), "desc.schema"), kDescSchema), SS_E_DESC,
          std::string("desc.schema: expected \"") + kDescSchema + "\"");
  Desc d;
  d.model = str_or(j, "model", w);
  d.engine = str_or(j, "engine", w);
  d.fixed_device = named(j.find("fixed_device"), "desc.fixed_device");
  d.host_fixed = named(j.find("host_fixed"), "desc.host_fixed");
  d.state_bytes_per_position = u64_or(j, "state_bytes_per_position", w, 0);
  d.workspace_bytes_per_row = u64_or(j, "workspace_bytes_per_row", w, 0);
  d.unit_align = u64_or(j, "unit_align", w, 256);
  d.ring_slots = uint32_t(capped(u64_or(j, "ring_slots", w, 0), 1u << 20, "desc.ring_slots"));
  d.routes = str_or(j, "routes", w);
  const std::string order = str_or(j, "order", w, "ranked");
  if (order == "prefix") d.order = Order::Prefix;
  else if (order == "ranked") d.order = Order::Ranked;
  else fail(SS_E_DESC, "desc.order: expected prefix | ranked");
  const std::string tiers = str_or(j, "tiers", w, "pinned|disk");
  if (tiers == "pinned") d.tiers = Tiers::Pinned;
  else if (tiers == "disk") d.tiers = Tiers::Disk;
  else if (tiers == "pinned|disk") d.tiers = Tiers::PinnedDisk;
  else if (tiers == "pair") d.tiers = Tiers::Pair;
  else fail(SS_E_DESC, "desc.tiers: expected pinned | disk | pinned|disk | pair");

  if (const Json* s = j.find("sources")) {
    require(s->is_array(), SS_E_DESC, "desc.sources: expected an array");
    for (size_t i = 0; i < s->arr.size(); ++i) {
      const std::string sw = idx("desc.sources", i);
      only_keys(s->arr[i], sw, {"name", "path", "align"});
      Source src;
      src.name = str_or(s->arr[i], "name", sw);
      src.path = json_str(need(s->arr[i], "path", sw), sw + ".path");
      src.align = u64_or(s->arr[i], "align", sw, 4096);
      d.sources.push_back(src);
    }
  }
  const Json& layers = need(j, "layers", w);
  require(layers.is_array(), SS_E_DESC, "desc.layers: expected an array");
  for (size_t i = 0; i < layers.arr.size(); ++i) {
    const Json& lj = layers.arr[i];
    const std::string lw = idx("desc.layers", i);
    only_keys(lj, lw,
              {"index", "kind", "fixed_bytes", "n_units", "top_k", "n_shared", "unit_bytes", "parts", "router", "hash",
               "benefit", "streamable"});
    Layer l;
    const int64_t index = json_i64(need(lj, "index", lw), lw + ".index");
    require(index >= 0 && index < kMaxLayers, SS_E_DESC, lw + ".index: 0..4095");
    l.index = int(index);
    const std::string kind = json_str(need(lj, "kind", lw), lw + ".kind");
    if (kind == "dense") l.kind = LayerKind::Dense;
    else if (kind == "moe") l.kind = LayerKind::Moe;
    else if (kind == "blob") l.kind = LayerKind::Blob;
    else fail(SS_E_DESC, lw + ".kind: expected dense | moe | blob");
    l.fixed_bytes = u64_or(lj, "fixed_bytes", lw, 0);
    l.n_units = int(capped(u64_or(lj, "n_units", lw, l.kind == LayerKind::Blob ? 1 : 0), kMaxUnits, lw + ".n_units"));
    l.top_k = int(capped(u64_or(lj, "top_k", lw, 0), kMaxUnits, lw + ".top_k"));
    l.n_shared = int(capped(u64_or(lj, "n_shared", lw, 0), kMaxUnits, lw + ".n_shared"));
    l.unit_bytes = u64_or(lj, "unit_bytes", lw, 0);
    if (const Json* st = lj.find("streamable")) l.streamable = json_bool(*st, lw + ".streamable");
    if (const Json* parts = lj.find("parts")) {
      require(parts->is_array(), SS_E_DESC, lw + ".parts: expected an array");
      for (size_t p = 0; p < parts->arr.size(); ++p) {
        const Json& pj = parts->arr[p];
        const std::string pw = idx(lw + ".parts", p);
        only_keys(pj, pw, {"name", "format", "source", "offset", "stride", "bytes"});
        Part part;
        part.name = str_or(pj, "name", pw);
        part.format = json_str(need(pj, "format", pw), pw + ".format");
        part.source = int(capped(u64_or(pj, "source", pw, 0), 1024, pw + ".source"));
        part.offset = json_u64(need(pj, "offset", pw), pw + ".offset");
        part.bytes = json_u64(need(pj, "bytes", pw), pw + ".bytes");
        part.stride = u64_or(pj, "stride", pw, part.bytes);
        l.parts.push_back(part);
      }
    }
    if (const Json* r = lj.find("router")) {
      const std::string rw = lw + ".router";
      only_keys(*r, rw, {"tensor", "bias", "format", "score", "rows", "cols"});
      l.has_router = true;
      l.router.tensor = json_str(need(*r, "tensor", rw), rw + ".tensor");
      l.router.bias = str_or(*r, "bias", rw);
      l.router.format = str_or(*r, "format", rw, "F32");
      l.router.score = str_or(*r, "score", rw, "softmax");
      l.router.rows = uint32_t(capped(u64_or(*r, "rows", rw, 0), kMaxUnits, rw + ".rows"));
      l.router.cols = uint32_t(capped(u64_or(*r, "cols", rw, 0), 1u << 24, rw + ".cols"));
    }
    if (const Json* h = lj.find("hash")) {
      require(h->is_array(), SS_E_DESC, lw + ".hash: expected an array of xxh64 hex strings");
      for (size_t k = 0; k < h->arr.size(); ++k)
        l.hash.push_back(parse_hex16(json_str(h->arr[k], idx(lw + ".hash", k)), idx(lw + ".hash", k)));
    }
    if (const Json* b = lj.find("benefit")) {
      require(b->is_array(), SS_E_DESC, lw + ".benefit: expected an array");
      for (size_t k = 0; k < b->arr.size(); ++k) l.benefit.push_back(json_f64(b->arr[k], idx(lw + ".benefit", k)));
    }
    d.layers.push_back(std::move(l));
  }
  if (const Json* t = j.find("lookup_tables")) {
    require(t->is_array(), SS_E_DESC, "desc.lookup_tables: expected an array");
    for (size_t i = 0; i < t->arr.size(); ++i) {
      const std::string tw = idx("desc.lookup_tables", i);
      only_keys(t->arr[i], tw, {"name", "source", "offset", "rows", "row_bytes", "placement"});
      LookupTable lt;
      lt.name = json_str(need(t->arr[i], "name", tw), tw + ".name");
      lt.source = int(capped(u64_or(t->arr[i], "source", tw, 0), 1024, tw + ".source"));
      lt.offset = u64_or(t->arr[i], "offset", tw, 0);
      lt.rows = json_u64(need(t->arr[i], "rows", tw), tw + ".rows");
      lt.row_bytes = json_u64(need(t->arr[i], "row_bytes", tw), tw + ".row_bytes");
      lt.placement = str_or(t->arr[i], "placement", tw, "file");
      d.lookup_tables.push_back(lt);
    }
  }
  desc_validate(d);
  return d;
}

void desc_validate(Desc& d) {
  require(!d.layers.empty() && d.layers.size() <= size_t(kMaxLayers), SS_E_DESC, "desc.layers: 1..4096 layers");
  require(d.unit_align >= 1 && (d.unit_align & (d.unit_align - 1)) == 0, SS_E_DESC, "desc.unit_align: power of two");
  for (size_t s = 0; s < d.sources.size(); ++s) {
    const uint64_t a = d.sources[s].align;
    require(a >= 1 && (a & (a - 1)) == 0 && a <= (1u << 20), SS_E_DESC,
            idx("desc.sources", s) + ".align: power of two <= 1 MiB");
  }
  d.unit_base.assign(d.layers.size(), 0);
  d.total_units = 0;
  d.max_unit_bytes = 0;
  d.max_units_per_layer = 0;
  for (size_t i = 0; i < d.layers.size(); ++i) {
    Layer& l = d.layers[i];
    const std::string lw = idx("desc.layers", i);
    require(l.index == int(i), SS_E_DESC, lw + ".index: layers must be listed in order 0..n-1");
    require(l.n_units >= 0 && l.n_units <= kMaxUnits, SS_E_DESC, lw + ".n_units: 0..65536");
    if (l.kind == LayerKind::Dense)
      require(l.n_units == 0 && l.parts.empty(), SS_E_DESC, lw + ": a dense layer has no units (use fixed_bytes)");
    else if (l.kind == LayerKind::Blob)
      require(l.n_units == 1, SS_E_DESC, lw + ": a blob layer has exactly one unit");
    else {
      require(l.n_units >= 1, SS_E_DESC, lw + ": a moe layer needs n_units >= 1");
      require(l.top_k >= 1 && l.top_k <= l.n_units, SS_E_DESC, lw + ".top_k: 1..n_units");
    }
    if (l.n_units > 0) {
      require(!l.parts.empty(), SS_E_DESC, lw + ".parts: a layer with units needs parts");
      uint64_t sum = 0;
      for (size_t p = 0; p < l.parts.size(); ++p) {
        const Part& part = l.parts[p];
        const std::string pw = idx(lw + ".parts", p);
        require(part.bytes > 0, SS_E_DESC, pw + ".bytes: > 0");
        require(known_format(part.format), SS_E_DESC, pw + ".format: unknown format " + part.format);
        require(part.source >= 0 && size_t(part.source) < d.sources.size(), SS_E_DESC, pw + ".source: no such source");
        require(l.n_units == 1 || part.stride >= part.bytes, SS_E_DESC, pw + ".stride: >= bytes (units overlap)");
        sum = add_ck(sum, part.bytes, pw);
        add_ck(add_ck(part.offset, mul_ck(uint64_t(l.n_units - 1), part.stride, pw), pw), part.bytes, pw);
      }
      if (l.unit_bytes == 0) l.unit_bytes = sum;
      require(l.unit_bytes == sum, SS_E_DESC,
              lw + ".unit_bytes: " + std::to_string(l.unit_bytes) + " != sum of parts " + std::to_string(sum));
      mul_ck(add_ck(l.unit_bytes, d.unit_align, lw), uint64_t(l.n_units), lw);
      require(l.hash.empty() || l.hash.size() == size_t(l.n_units), SS_E_DESC, lw + ".hash: one per unit");
      require(l.benefit.empty() || l.benefit.size() == size_t(l.n_units), SS_E_DESC, lw + ".benefit: one per unit");
      if (l.has_router)
        require(l.router.rows == 0 || l.router.rows == uint32_t(l.n_units), SS_E_DESC,
                lw + ".router.rows: must equal n_units");
      if (l.streamable) {
        d.max_unit_bytes = std::max(d.max_unit_bytes, l.unit_bytes);
        d.max_units_per_layer = std::max(d.max_units_per_layer, l.n_units);
      }
    }
    d.unit_base[i] = d.total_units;
    d.total_units += l.n_units;
  }
  uint64_t dev = 0, host = 0;
  for (const auto& n : d.fixed_device) dev = add_ck(dev, n.bytes, "desc.fixed_device");
  for (const auto& n : d.host_fixed) host = add_ck(host, n.bytes, "desc.host_fixed");
  uint64_t all = add_ck(dev, host, "desc");
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const uint64_t st = add_ck(d.layers[L].unit_bytes, 4096, idx("desc.layers", L));
    all = add_ck(all, mul_ck(uint64_t(d.layers[L].n_units), st, idx("desc.layers", L)), idx("desc.layers", L));
  }
  require(all < (uint64_t(1) << 56), SS_E_DESC, "desc: total bytes above 2^56 (64 PiB)");
  for (size_t L = 0; L < d.layers.size(); ++L) {
    dev = add_ck(dev, d.layers[L].fixed_bytes, idx("desc.layers", L) + ".fixed_bytes");
    if (!d.layers[L].streamable)
      dev = add_ck(dev, mul_ck(uint64_t(d.layers[L].n_units), d.unit_stride(int(L)), idx("desc.layers", L)),
                   idx("desc.layers", L));
  }
  for (size_t i = 0; i < d.lookup_tables.size(); ++i) {
    const LookupTable& t = d.lookup_tables[i];
    const std::string tw = idx("desc.lookup_tables", i);
    require(t.source >= 0 && size_t(t.source) < d.sources.size(), SS_E_DESC, tw + ".source: no such source");
    require(t.placement == "file" || t.placement == "pinned" || t.placement == "device", SS_E_DESC,
            tw + ".placement: file | pinned | device");
  }
}

Json desc_to_json(const Desc& d) {
  Json j = Json::object();
  j["schema"] = Json::string(kDescSchema);
  if (!d.model.empty()) j["model"] = Json::string(d.model);
  if (!d.engine.empty()) j["engine"] = Json::string(d.engine);
  auto list = [](const std::vector<NamedBytes>& v) {
    Json a = Json::array();
    for (const auto& n : v) {
      Json e = Json::object();
      e["name"] = Json::string(n.name);
      e["bytes"] = Json::number(n.bytes);
      a.push(e);
    }
    return a;
  };
  j["fixed_device"] = list(d.fixed_device);
  j["host_fixed"] = list(d.host_fixed);
  j["state_bytes_per_position"] = Json::number(d.state_bytes_per_position);
  j["workspace_bytes_per_row"] = Json::number(d.workspace_bytes_per_row);
  j["unit_align"] = Json::number(d.unit_align);
  j["order"] = Json::string(d.order == Order::Prefix ? "prefix" : "ranked");
  j["tiers"] = Json::string(tiers_text(d.tiers));
  j["ring_slots"] = Json::number(uint64_t(d.ring_slots));
  if (!d.routes.empty()) j["routes"] = Json::string(d.routes);
  Json srcs = Json::array();
  for (const auto& s : d.sources) {
    Json e = Json::object();
    if (!s.name.empty()) e["name"] = Json::string(s.name);
    e["path"] = Json::string(s.path);
    e["align"] = Json::number(s.align);
    srcs.push(e);
  }
  j["sources"] = srcs;
  Json layers = Json::array();
  for (const auto& l : d.layers) {
    Json e = Json::object();
    e["index"] = Json::number_i(l.index);
    e["kind"] = Json::string(l.kind == LayerKind::Dense ? "dense" : l.kind == LayerKind::Moe ? "moe" : "blob");
    e["fixed_bytes"] = Json::number(l.fixed_bytes);
    if (l.n_units > 0) {
      e["n_units"] = Json::number_i(l.n_units);
      e["unit_bytes"] = Json::number(l.unit_bytes);
      e["streamable"] = Json::boolean(l.streamable);
      Json parts = Json::array();
      for (const auto& p : l.parts) {
        Json pj = Json::object();
        if (!p.name.empty()) pj["name"] = Json::string(p.name);
        pj["format"] = Json::string(p.format);
        pj["source"] = Json::number_i(p.source);
        pj["offset"] = Json::number(p.offset);
        pj["stride"] = Json::number(p.stride);
        pj["bytes"] = Json::number(p.bytes);
        parts.push(pj);
      }
      e["parts"] = parts;
      if (!l.hash.empty()) {
        Json h = Json::array();
        for (uint64_t v : l.hash) h.push(Json::string(hex16(v)));
        e["hash"] = h;
      }
      if (!l.benefit.empty()) {
        Json b = Json::array();
        for (double v : l.benefit) b.push(Json::number_f(v));
        e["benefit"] = b;
      }
    }
    if (l.top_k) e["top_k"] = Json::number_i(l.top_k);
    if (l.n_shared) e["n_shared"] = Json::number_i(l.n_shared);
    if (l.has_router) {
      Json r = Json::object();
      r["tensor"] = Json::string(l.router.tensor);
      if (!l.router.bias.empty()) r["bias"] = Json::string(l.router.bias);
      r["format"] = Json::string(l.router.format);
      r["score"] = Json::string(l.router.score);
      r["rows"] = Json::number(uint64_t(l.router.rows));
      r["cols"] = Json::number(uint64_t(l.router.cols));
      e["router"] = r;
    }
    layers.push(e);
  }
  j["layers"] = layers;
  Json tables = Json::array();
  for (const auto& t : d.lookup_tables) {
    Json e = Json::object();
    e["name"] = Json::string(t.name);
    e["source"] = Json::number_i(t.source);
    e["offset"] = Json::number(t.offset);
    e["rows"] = Json::number(t.rows);
    e["row_bytes"] = Json::number(t.row_bytes);
    e["placement"] = Json::string(t.placement);
    tables.push(e);
  }
  j["lookup_tables"] = tables;
  return j;
}

// ---------------------------------------------------------------------------------------------------------------------
// Planner. Units are streamable (layer, unit) pairs in model order; "bytes" is the device slot (unit stride).
namespace {

struct Cand {
  int64_t g;
  int layer;
  uint64_t bytes;
  double benefit;
};

double per_byte(const Cand& c) {
  return c.bytes ? c.benefit / double(c.bytes) : std::numeric_limits<double>::infinity();
}
// Higher benefit per byte first; model order breaks ties.
bool before(const Cand& a, const Cand& b) {
  const double x = per_byte(a), y = per_byte(b);
  if (x != y) return x > y;
  return a.g < b.g;
}

std::vector<Cand> candidates(const Desc& d, const std::vector<double>& benefit) {
  std::vector<Cand> v;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    if (!l.streamable) continue;
    for (int u = 0; u < l.n_units; ++u) {
      const int64_t g = d.unit_base[L] + u;
      const double b = !benefit.empty() ? benefit[size_t(g)] : !l.benefit.empty() ? l.benefit[size_t(u)] : 1.0;
      require(std::isfinite(b) && b >= 0, SS_E_INVALID, "plan: benefit must be finite and >= 0");
      v.push_back({g, int(L), d.unit_stride(int(L)), b});
    }
  }
  return v;
}

uint64_t dynamic_upper(const Desc& d, const ss_budget& b) {
  if (!b.dynamic_slots_per_layer) return 0;
  uint64_t t = 0;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    if (l.streamable && l.n_units > 0)
      t += uint64_t(std::min<uint32_t>(b.dynamic_slots_per_layer, uint32_t(l.n_units))) * d.unit_stride(int(L));
  }
  return t;
}

// One ring per distinct slot size among the streamed units; slots: the budget's, else the descriptor's, else twice the
// most units of any layer with that slot size. Sorted by slot size.
std::vector<RingClass> rings_of(const Desc& d, const ss_budget& b, const std::vector<Cand>& streamed) {
  std::vector<RingClass> out;
  if (d.tiers == Tiers::Pair) return out;
  for (const Cand& c : streamed) {
    if (!c.bytes) continue;
    bool seen = false;
    for (const RingClass& r : out) seen = seen || r.stride == c.bytes;
    if (seen) continue;
    uint32_t slots = b.ring_slots ? b.ring_slots : d.ring_slots;
    if (!slots)
      for (size_t L = 0; L < d.layers.size(); ++L)
        if (d.layers[L].streamable && d.layers[L].n_units && d.unit_stride(int(L)) == c.bytes)
          slots = std::max(slots, uint32_t(2 * d.layers[L].n_units));
    out.push_back({c.bytes, slots});
  }
  std::sort(out.begin(), out.end(), [](const RingClass& x, const RingClass& y) { return x.stride < y.stride; });
  return out;
}

uint64_t ring_total(const std::vector<RingClass>& r) {
  uint64_t t = 0;
  for (const RingClass& c : r) t += c.stride * c.slots;
  return t;
}

bool excl(const ss_budget& b) { return b.tier_mode == SS_TIER_MODE_EXCLUSIVE; }
bool pinned_copy(uint8_t t) { return t == SS_TIER_PINNED || t == SS_TIER_RESIDENT_BACKED; }

uint64_t spare_total(const std::vector<SpareClass>& s) {
  uint64_t t = 0;
  for (const SpareClass& c : s) {
    require(c.blocks == 0 || c.block_bytes <= (UINT64_MAX - t) / c.blocks, SS_E_INVALID,
            "plan: spare block bytes overflow");
    t += c.block_bytes * c.blocks;
  }
  return t;
}

// The totals every consumer bills, from the tiers alone.
void totals(const Desc& d, const ss_budget& b, Plan& p) {
  std::vector<Cand> streamed;
  p.resident = p.pinned = p.disk = p.dynamic = 0;
  p.n_resident = p.n_pinned = p.n_disk = p.n_pair = p.n_backed = 0;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const Layer& l = d.layers[L];
    int planned = 0;
    for (int u = 0; u < l.n_units; ++u) {
      const int64_t g = d.unit_base[L] + u;
      const uint8_t t = p.tier[size_t(g)];
      require(t <= SS_TIER_RESIDENT_BACKED, SS_E_INVALID, "plan: bad tier value");
      if (!l.streamable) {
        require(t == SS_TIER_RESIDENT, SS_E_INVALID, "plan: a non-streamable layer's units must be resident");
        continue;
      }
      require(!(excl(b) && t == SS_TIER_RESIDENT_BACKED), SS_E_INVALID,
              "plan: tier B (resident with a pinned copy) is the second copy the exclusive tier mode removes");
      if (t == SS_TIER_RESIDENT || t == SS_TIER_RESIDENT_BACKED) {
        p.resident += d.unit_stride(int(L));
        ++p.n_resident;
        ++planned;
        if (t == SS_TIER_RESIDENT_BACKED) ++p.n_backed;
        continue;
      }
      if (t != SS_TIER_PAIR) streamed.push_back({g, int(L), d.unit_stride(int(L)), 0.0});
      if (t == SS_TIER_PINNED) {
        ++p.n_pinned;
      } else if (t == SS_TIER_DISK) {
        p.disk += l.unit_bytes;
        ++p.n_disk;
      } else {
        ++p.n_pair;
      }
    }
    if (l.streamable && l.n_units > 0 && b.dynamic_slots_per_layer)
      p.dynamic += uint64_t(std::min<uint32_t>(b.dynamic_slots_per_layer, uint32_t(l.n_units - planned))) *
                   d.unit_stride(int(L));
  }
  const uint64_t layout = pinned_layout(d, p.tier).total;
  p.pinned = layout;
  for (const auto& n : d.host_fixed) p.pinned += n.bytes;
  require(p.pinned >= layout, SS_E_INVALID, "plan: host byte total overflows");
  p.spares = spare_classes(d, b, b.host_pinned_bytes > p.pinned ? b.host_pinned_bytes - p.pinned : 0);
  p.pinned += spare_total(p.spares);
  p.rings = rings_of(d, b, streamed);
  p.ring = ring_total(p.rings);
  require(p.pinned <= b.host_pinned_bytes, SS_E_CAPACITY,
          d.engine + ": " + gib(p.pinned) + " GiB must be pinned on the host, above the host budget " +
              gib(b.host_pinned_bytes) + " GiB; raise the cap or the host budget");
  p.peak = p.fixed + p.dynamic + p.ring + p.resident;
  require(p.peak + p.margin <= p.cap, SS_E_CAPACITY,
          d.engine + ": predicted peak " + gib(p.peak) + " GiB above the cap " + gib(p.cap) + " GiB - margin " +
              gib(p.margin) + " GiB");
}

Plan start_plan(const Desc& d, const ss_budget& b) {
  require(b.device_bytes > 0, SS_E_INVALID, "plan: device budget must be > 0");
  require(b.tier_mode == SS_TIER_MODE_INCLUSIVE || b.tier_mode == SS_TIER_MODE_EXCLUSIVE, SS_E_INVALID,
          "plan: tier_mode must be SS_TIER_MODE_INCLUSIVE or SS_TIER_MODE_EXCLUSIVE");
  if (excl(b)) {
    require(!b.pinned_backing, SS_E_INVALID,
            "plan: pinned_backing keeps a second pinned copy of residents, which the exclusive tier mode removes");
    require(d.tiers == Tiers::Pinned || d.tiers == Tiers::PinnedDisk, SS_E_INVALID,
            d.engine + ": the exclusive tier mode needs a descriptor whose tiers allow pinned");
  }
  Plan p;
  p.budget = b;
  p.cap = b.device_bytes;
  p.margin = plan_margin(b);
  p.tier.assign(size_t(d.total_units), SS_TIER_RESIDENT);
  p.dynamic_slots_per_layer = b.dynamic_slots_per_layer;
  p.fixed = d.fixed_total() + b.workspace_bytes;
  p.dynamic = dynamic_upper(d, b);
  require(p.cap >= p.margin + p.fixed + p.dynamic, SS_E_CAPACITY,
          d.engine + ": fixed device memory " + gib(p.fixed) + " GiB + dynamic slots " + gib(p.dynamic) +
              " GiB + margin " + gib(p.margin) + " GiB exceeds the " + gib(p.cap) + " GiB cap");
  return p;
}

// RESIDENT -> RESIDENT_BACKED while the host budget left after host_fixed and the pinned tier lasts, lowest benefit
// per byte first, stopping at the first that does not fit.
void give_backing(const Desc& d, const ss_budget& b, const std::vector<double>& benefit, std::vector<uint8_t>& tier) {
  uint64_t left = b.host_pinned_bytes;
  for (const auto& n : d.host_fixed) left = left > n.bytes ? left - n.bytes : 0;
  std::vector<Cand> res;
  for (const Cand& c : candidates(d, benefit)) {
    const uint8_t t = tier[size_t(c.g)];
    if (t == SS_TIER_PINNED) {
      const uint64_t hb = host_stride(d.layers[size_t(c.layer)].unit_bytes);
      left = left > hb ? left - hb : 0;
    } else if (t == SS_TIER_RESIDENT) {
      res.push_back(c);
    }
  }
  std::stable_sort(res.begin(), res.end(), [](const Cand& x, const Cand& y) { return before(y, x); });
  for (const Cand& c : res) {
    const uint64_t hb = host_stride(d.layers[size_t(c.layer)].unit_bytes);
    if (hb > left) break;
    tier[size_t(c.g)] = SS_TIER_RESIDENT_BACKED;
    left -= hb;
  }
}

}  // namespace

uint64_t host_stride(uint64_t bytes) {
  require(bytes <= UINT64_MAX - (kHostStride - 1), SS_E_INVALID, "plan: unit bytes overflow the host stride");
  return (bytes + kHostStride - 1) / kHostStride * kHostStride;
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

PinnedLayout pinned_layout(const Desc& d, const std::vector<uint8_t>& tier) {
  // model order, 4 KiB strides, chunks of at most 1 GiB (a larger unit alone in its chunk)
  PinnedLayout pl;
  pl.chunk_of.assign(size_t(d.total_units), -1);
  pl.offset_of.assign(size_t(d.total_units), 0);
  uint64_t used = 0;
  bool open = false;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const uint64_t st = host_stride(d.layers[L].unit_bytes);
    for (int u = 0; u < d.layers[L].n_units; ++u) {
      const int64_t g = d.unit_base[L] + u;
      if (!pinned_copy(tier[size_t(g)])) continue;
      if (!open || (used > 0 && used + st > kPinnedChunk)) {
        if (open) pl.chunk_bytes.push_back(used);
        used = 0;
        open = true;
      }
      pl.chunk_of[size_t(g)] = int32_t(pl.chunk_bytes.size());
      pl.offset_of[size_t(g)] = used;
      used += st;
    }
  }
  if (open) pl.chunk_bytes.push_back(used);
  for (uint64_t c : pl.chunk_bytes) {
    require(pl.total <= UINT64_MAX - c, SS_E_INVALID, "plan: pinned layout overflows");
    pl.total += c;
  }
  return pl;
}

std::vector<SpareClass> spare_classes(const Desc& d, const ss_budget& b, uint64_t host_left) {
  std::vector<SpareClass> out;
  if (!excl(b)) return out;
  std::vector<std::pair<uint64_t, uint64_t>> per;  // host stride -> streamable units of that stride
  for (const Layer& l : d.layers) {
    if (!l.streamable || !l.n_units) continue;
    const uint64_t hs = host_stride(l.unit_bytes);
    bool found = false;
    for (auto& x : per)
      if (x.first == hs) {
        x.second += uint64_t(l.n_units);
        found = true;
      }
    if (!found) per.push_back({hs, uint64_t(l.n_units)});
  }
  for (const auto& x : per) {
    const uint64_t want = b.host_spare_units ? b.host_spare_units : 64;
    out.push_back({x.first, uint32_t(std::min<uint64_t>(want, x.second)), 0});
  }
  std::sort(out.begin(), out.end(), [](const SpareClass& x, const SpareClass& y) { return x.block_bytes < y.block_bytes; });
  for (SpareClass& c : out) {  // smallest blocks first
    c.blocks = uint32_t(std::min<uint64_t>(c.asked, host_left / c.block_bytes));
    host_left -= uint64_t(c.blocks) * c.block_bytes;
  }
  return out;
}

Plan plan_make(const Desc& d, const ss_budget& b, const std::vector<double>& benefit) {
  require(benefit.empty() || int64_t(benefit.size()) == d.total_units, SS_E_INVALID,
          "plan: benefit needs one value per unit (ss_desc_total_units)");
  Plan p = start_plan(d, b);
  const std::vector<Cand> units = candidates(d, benefit);
  uint64_t room = p.cap - p.margin - p.fixed - p.dynamic;
  std::vector<char> chosen(units.size(), 0);
  uint64_t total = 0;
  for (const Cand& c : units) total += c.bytes;
  bool ok = false;
  if (d.order == Order::Prefix) {
    // the longest prefix that fits together with the rings of what is left
    std::vector<Cand> rest;
    for (size_t k = units.size() + 1; k-- > 0;) {
      rest.assign(units.begin() + std::ptrdiff_t(k), units.end());
      if (total + ring_total(rings_of(d, b, rest)) <= room) {
        for (size_t i = 0; i < k; ++i) chosen[i] = 1;
        ok = true;
        break;
      }
      if (k) total -= units[k - 1].bytes;
    }
  } else if (total <= room) {
    std::fill(chosen.begin(), chosen.end(), char(1));
    ok = true;
  } else {
    const uint64_t ring = ring_total(rings_of(d, b, units));
    if (ring <= room) {
      room -= ring;
      std::vector<size_t> order(units.size());
      for (size_t i = 0; i < order.size(); ++i) order[i] = i;
      std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t c) { return before(units[a], units[c]); });
      uint64_t used = 0;
      for (size_t i : order)
        if (used + units[i].bytes <= room) {
          chosen[i] = 1;
          used += units[i].bytes;
        }
      ok = true;
    }
  }
  require(ok, SS_E_CAPACITY,
          d.engine + ": nothing fits under the " + gib(p.cap) + " GiB cap: fixed " + gib(p.fixed) + " GiB + margin " +
              gib(p.margin) + " GiB + the stream rings exceed it");
  uint64_t host_left = b.host_pinned_bytes;
  for (const auto& n : d.host_fixed) host_left = host_left > n.bytes ? host_left - n.bytes : 0;
  std::vector<Cand> spill;
  for (size_t i = 0; i < units.size(); ++i) {
    if (chosen[i]) continue;
    const Cand& c = units[i];
    uint8_t& t = p.tier[size_t(c.g)];
    switch (d.tiers) {
      case Tiers::Pinned: {
        t = SS_TIER_PINNED;
        const uint64_t hb = host_stride(d.layers[size_t(c.layer)].unit_bytes);
        host_left = host_left > hb ? host_left - hb : 0;
        break;
      }
      case Tiers::Disk: t = SS_TIER_DISK; break;
      case Tiers::Pair: t = SS_TIER_PAIR; break;
      case Tiers::PinnedDisk: spill.push_back(c); break;
    }
  }
  std::stable_sort(spill.begin(), spill.end(), before);
  for (const Cand& c : spill) {
    const uint64_t hb = host_stride(d.layers[size_t(c.layer)].unit_bytes);
    if (hb <= host_left) {
      p.tier[size_t(c.g)] = SS_TIER_PINNED;
      host_left -= hb;
    } else {
      p.tier[size_t(c.g)] = SS_TIER_DISK;
    }
  }
  if (b.pinned_backing) give_backing(d, b, benefit, p.tier);
  totals(d, b, p);
  return p;
}

Plan plan_from_tiers(const Desc& d, const ss_budget& b, const std::vector<uint8_t>& tiers) {
  require(int64_t(tiers.size()) == d.total_units, SS_E_INVALID, "plan: one tier per unit (ss_desc_total_units)");
  Plan p = start_plan(d, b);
  p.tier = tiers;
  totals(d, b, p);
  return p;
}

Json plan_to_json(const Desc& d, const Plan& p) {
  Json j = Json::object();
  j["schema"] = Json::string("strix-stream/plan-v1");
  j["engine"] = Json::string(d.engine);
  j["cap_bytes"] = Json::number(p.cap);
  j["margin_bytes"] = Json::number(p.margin);
  j["fixed_bytes"] = Json::number(p.fixed);
  j["dynamic_bytes"] = Json::number(p.dynamic);
  j["dynamic_slots_per_layer"] = Json::number(uint64_t(p.dynamic_slots_per_layer));
  j["ring_bytes"] = Json::number(p.ring);
  Json rings = Json::array();
  for (const RingClass& c : p.rings) {
    Json r = Json::object();
    r["slot_bytes"] = Json::number(c.stride);
    r["slots"] = Json::number(uint64_t(c.slots));
    rings.push(r);
  }
  j["rings"] = rings;
  j["resident_bytes"] = Json::number(p.resident);
  j["pinned_bytes"] = Json::number(p.pinned);
  j["disk_bytes"] = Json::number(p.disk);
  j["peak_bytes"] = Json::number(p.peak);
  j["n_resident"] = Json::number(p.n_resident);
  j["n_pinned"] = Json::number(p.n_pinned);
  j["n_disk"] = Json::number(p.n_disk);
  j["n_pair"] = Json::number(p.n_pair);
  j["n_backed"] = Json::number(p.n_backed);
  if (p.budget.tier_mode == SS_TIER_MODE_EXCLUSIVE) {
    j["tier_mode"] = Json::string("exclusive");
    Json sp = Json::array();
    for (const SpareClass& c : p.spares) {
      Json x = Json::object();
      x["block_bytes"] = Json::number(c.block_bytes);
      x["asked"] = Json::number(uint64_t(c.asked));
      x["blocks"] = Json::number(uint64_t(c.blocks));
      sp.push(x);
    }
    j["spare_blocks"] = sp;
  }
  Json layers = Json::array();
  for (size_t L = 0; L < d.layers.size(); ++L) {
    std::string s;
    for (int u = 0; u < d.layers[L].n_units; ++u) s += "RPDXB"[p.tier[size_t(d.unit_base[L] + u)]];
    layers.push(Json::string(s));
  }
  j["tiers"] = layers;
  return j;
}

std::vector<uint8_t> tiers_from_json(const Desc& d, const Json& j) {
  static const char kLetters[] = "RPDXB";
  const Json* t = j.find("tiers");
  require(t && t->is_array() && t->arr.size() == d.layers.size(), SS_E_DESC,
          "plan json: \"tiers\" needs one string per layer");
  std::vector<uint8_t> out;
  for (size_t L = 0; L < d.layers.size(); ++L) {
    const std::string& s = json_str(t->arr[L], "plan.tiers");
    require(s.size() == size_t(d.layers[L].n_units), SS_E_DESC,
            "plan json: tiers[" + std::to_string(L) + "] needs one letter per unit");
    for (char c : s) {
      const char* k = c ? std::strchr(kLetters, c) : nullptr;
      require(k != nullptr, SS_E_DESC, "plan json: tier letters are R P D X B");
      out.push_back(uint8_t(k - kLetters));
    }
  }
  return out;
}

}  // namespace tsa
