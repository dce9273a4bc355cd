// The strix-stream / tierstream C ABI of the serve path: descriptor, plan, context, host-contract forward, stats, and
// the device-gated calls. Versioned-struct reading and the status conventions follow reference src/capi.cpp:101-243.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <mutex>
#include <sstream>

#include "capi_internal.hpp"
#include "dg_ctx.hpp"
#include "host_ctx.hpp"
#include "tierstream_amd/tsa_test.h"

ss_ctx::~ss_ctx() = default;

namespace tsa {

bool ctx_poisoned(const ss_ctx* c) { return c->dg ? c->dg->poisoned() : c->host->poisoned(); }
void ctx_poison(ss_ctx* c) {
  if (c->dg) c->dg->poison();
  else c->host->poison();
}

namespace {

// Contexts open now, in open order. A process that exits with one still open (an engine that failed and never called
// ss_close) would otherwise tear the HIP runtime down under a live service thread, reader threads and streams: the
// first ss_open registers an exit handler, and handlers registered after a library was loaded run before that
// library's own finalizers, so the handler closes what is left while the runtime still works. A handler never throws.
std::mutex g_open_mu;
std::vector<ss_ctx*>* g_open = nullptr;  // allocated once and never freed: it is read by the exit handler

void close_open_contexts() noexcept {
  std::vector<ss_ctx*> left;
  {
    std::lock_guard<std::mutex> lk(g_open_mu);
    if (g_open) left.swap(*g_open);
  }
  for (auto it = left.rbegin(); it != left.rend(); ++it) {
    try {
      delete *it;
    } catch (...) {
    }
  }
}

void track_open(ss_ctx* c) {
  std::lock_guard<std::mutex> lk(g_open_mu);
  if (!g_open) {
    g_open = new std::vector<ss_ctx*>();
    std::atexit(close_open_contexts);
  }
  g_open->push_back(c);
}

void untrack(ss_ctx* c) {
  std::lock_guard<std::mutex> lk(g_open_mu);
  if (!g_open) return;
  const auto it = std::find(g_open->begin(), g_open->end(), c);
  if (it != g_open->end()) g_open->erase(it);
}

void budget_defaults(ss_budget* b) {
  std::memset(static_cast<void*>(b), 0, sizeof *b);
  b->struct_size = uint32_t(sizeof *b);
  b->margin_gib = 2.0;
  b->margin_fraction = 0.03;
}

void options_defaults(ss_options* o) {
  std::memset(static_cast<void*>(o), 0, sizeof *o);
  o->struct_size = uint32_t(sizeof *o);
  o->backend = SS_BACKEND_HIP;  // this library's only backend (the reference defaults to CPU)
  o->policy = SS_POLICY_LRU;
  o->lookahead_budget = 2;
  o->reader_threads = 2;
  o->staging_buffers = 4;
  o->staging_bytes = uint64_t(256) << 20;
  o->copy_piece_bytes = uint64_t(64) << 20;
  o->fill_residents = 1;
  o->score_window = 16;
  o->pin_planned = 1;
  o->direct_io = 1;
  o->forward_mode = SS_FORWARD_HOST;
  o->dg_prefetch_reserve = 0xFFFFFFFFu;
  o->dg_prefetch_per_layer = 4;
  o->dg_prefetch_per_token = 48;
  o->dg_wait_timeout_ms = 10000;
  o->dg_spare_target = 0xFFFFFFFFu;
  o->dg_wb_defer = 1;
  o->dg_wb_stream = 1;
  o->dg_score_w_trans = 700;
  o->dg_score_w_freq = 200;
  o->dg_score_w_recency = 100;
  o->drive_readers = 4;
  o->weight_verify = 0;
}

void clear_reserved(ss_budget& b) { b.reserved0 = 0; }
void clear_reserved(ss_options& o) {
  o.reserved0 = o.reserved1 = o.reserved2 = o.reserved3 = o.reserved4 = o.reserved5 = o.reserved6 = o.reserved7 = 0;
}

// An input struct: the library's defaults, then min(struct_size, sizeof) bytes of the caller's.
template <class T>
T versioned(const T* in, void (*defaults)(T*), const char* what) {
  T v;
  defaults(&v);
  if (!in) return v;
  require(in->struct_size >= 2 * sizeof(uint32_t), SS_E_INVALID,
          std::string(what) + ": struct_size not set (fill the struct with its *_defaults function)");
  std::memcpy(static_cast<void*>(&v), in, std::min<size_t>(in->struct_size, sizeof(T)));
  v.struct_size = uint32_t(sizeof(T));
  clear_reserved(v);
  return v;
}

template <class T>
void sized_defaults(T* out, uint32_t size, void (*defaults)(T*)) {
  if (!out || size < sizeof(uint32_t)) return;
  T v;
  defaults(&v);
  v.struct_size = std::min<uint32_t>(size, uint32_t(sizeof(T)));
  std::memcpy(static_cast<void*>(out), &v, v.struct_size);
}

void need(bool ok, const char* m) { require(ok, SS_E_INVALID, m); }

ss_status give_text(const std::string& s, char** out, size_t* len) {
  if (!out) {
    set_last_error("null output");
    return SS_E_INVALID;
  }
  char* p = static_cast<char*>(std::malloc(s.size() + 1));
  if (!p) {
    set_last_error("out of host memory");
    return SS_E_NOMEM;
  }
  std::memcpy(p, s.data(), s.size());
  p[s.size()] = '\0';
  *out = p;
  if (len) *len = s.size();
  return SS_OK;
}

std::string read_file(const char* path) {
  need(path != nullptr, "null path");
  std::ifstream f(path, std::ios::binary);
  require(bool(f), SS_E_IO, std::string("cannot open ") + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

HostCtx& host_of(const ss_ctx* c, const char* fn) {
  if (c->dg) fail(SS_E_INVALID, std::string(fn) + ": refused in device-gated mode (use the ss_dg_* calls)");
  return *c->host;
}
DgCtx& dg_of(const ss_ctx* c, const char* fn) {
  if (!c->dg) fail(SS_E_INVALID, std::string(fn) + ": the context is not device-gated");
  return *c->dg;
}

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" {

// ---- descriptor ----
ss_status ss_desc_from_json(const char* text, size_t len, ss_desc** out) {
  return guard([&] {
    need(text && out, "ss_desc_from_json: null argument");
    *out = new ss_desc{desc_from_json(json_parse(std::string(text, len)))};
  });
}
ss_status ss_desc_from_file(const char* path, ss_desc** out) {
  return guard([&] {
    need(out != nullptr, "ss_desc_from_file: null argument");
    *out = new ss_desc{desc_from_json(json_parse(read_file(path)))};
  });
}
ss_status ss_desc_from_model(const char* path, ss_desc** out) { return ss_desc_from_file(path, out); }
void ss_desc_free(ss_desc* d) { delete d; }
int ss_desc_n_layers(const ss_desc* d) { return d ? int(d->d.layers.size()) : 0; }
int ss_desc_layer_units(const ss_desc* d, int layer) {
  if (!d || layer < 0 || size_t(layer) >= d->d.layers.size()) return -1;
  return d->d.layers[size_t(layer)].n_units;
}
uint64_t ss_desc_unit_bytes(const ss_desc* d, int layer) {
  if (!d || layer < 0 || size_t(layer) >= d->d.layers.size()) return 0;
  return d->d.layers[size_t(layer)].unit_bytes;
}
ss_status ss_desc_to_json(const ss_desc* d, char** out, size_t* len) {
  std::string s;
  const ss_status st = guard([&] {
    need(d != nullptr, "ss_desc_to_json: null descriptor");
    s = json_dump(desc_to_json(d->d));
  });
  return st != SS_OK ? st : give_text(s, out, len);
}
int64_t ss_desc_unit_index(const ss_desc* d, int layer, int unit) {
  if (!d || layer < 0 || size_t(layer) >= d->d.layers.size()) return -1;
  if (unit < 0 || unit >= d->d.layers[size_t(layer)].n_units) return -1;
  return d->d.unit_base[size_t(layer)] + unit;
}
int64_t ss_desc_total_units(const ss_desc* d) { return d ? d->d.total_units : 0; }

// ---- plan ----
void ss_budget_defaults_sized(ss_budget* b, uint32_t size) { sized_defaults(b, size, budget_defaults); }
ss_status ss_plan_make(const ss_desc* d, const ss_budget* b, const double* benefit, size_t n, ss_plan** out) {
  return guard([&] {
    need(d && b && out, "ss_plan_make: null argument");
    need(benefit || n == 0, "ss_plan_make: null benefit with n > 0");
    const ss_budget bb = versioned(b, budget_defaults, "ss_plan_make budget");
    std::vector<double> ben;
    if (benefit) ben.assign(benefit, benefit + n);
    *out = new ss_plan{plan_make(d->d, bb, ben), d};
  });
}
ss_status ss_plan_from_tiers(const ss_desc* d, const ss_budget* b, const uint8_t* tiers, size_t n, ss_plan** out) {
  return guard([&] {
    need(d && b && tiers && out, "ss_plan_from_tiers: null argument");
    const ss_budget bb = versioned(b, budget_defaults, "ss_plan_from_tiers budget");
    *out = new ss_plan{plan_from_tiers(d->d, bb, std::vector<uint8_t>(tiers, tiers + n)), d};
  });
}
ss_status ss_plan_from_json(const ss_desc* d, const ss_budget* b, const char* text, size_t len, ss_plan** out) {
  return guard([&] {
    need(d && b && text && out, "ss_plan_from_json: null argument");
    const std::vector<uint8_t> tiers = tiers_from_json(d->d, json_parse(std::string(text, len)));  // before the budget
    const ss_budget bb = versioned(b, budget_defaults, "ss_plan_from_json budget");
    *out = new ss_plan{plan_from_tiers(d->d, bb, tiers), d};
  });
}
void ss_plan_free(ss_plan* p) { delete p; }
ss_tier ss_plan_unit_tier(const ss_plan* p, int layer, int unit) {
  const int64_t g = p ? ss_desc_unit_index(p->desc, layer, unit) : -1;
  return g < 0 ? SS_TIER_PAIR : ss_tier(p->p.tier[size_t(g)]);
}
void ss_plan_get_totals(const ss_plan* p, ss_plan_totals* o) {
  if (!p || !o) return;
  *o = ss_plan_totals{};
  o->fixed_bytes = p->p.fixed;
  o->margin_bytes = p->p.margin;
  o->resident_bytes = p->p.resident;
  o->dynamic_bytes = p->p.dynamic;
  o->ring_bytes = p->p.ring;
  o->peak_device_bytes = p->p.peak;
  o->pinned_bytes = p->p.pinned;
  o->disk_bytes = p->p.disk;
  o->n_resident = p->p.n_resident;
  o->n_pinned = p->p.n_pinned;
  o->n_disk = p->p.n_disk;
}
ss_status ss_plan_to_json(const ss_plan* p, char** out, size_t* len) {
  std::string s;
  const ss_status st = guard([&] {
    need(p != nullptr, "ss_plan_to_json: null plan");
    s = json_dump(plan_to_json(p->desc->d, p->p));
  });
  return st != SS_OK ? st : give_text(s, out, len);
}

// ---- context ----
void ss_options_defaults_sized(ss_options* o, uint32_t size) { sized_defaults(o, size, options_defaults); }

ss_status ss_open(const ss_desc* d, const ss_budget* budget, const ss_plan* plan, const ss_options* opt,
                  ss_ctx** out) {
  return guard([&] {
    need(d && budget && out, "ss_open: null argument");
    need(!plan || plan->desc == d, "ss_open: plan was made from another descriptor");
    const ss_options o = versioned(opt, options_defaults, "ss_open options");
    require(o.backend == SS_BACKEND_HIP, SS_E_UNSUPPORTED,
            "ss_open: this library is the MI355X (discrete HIP) backend; backend must be SS_BACKEND_HIP");
    const ss_budget bb = versioned(budget, budget_defaults, "ss_open budget");
    need(!plan || same_budget(plan->p.budget, bb), "ss_open: the plan was made with another budget");
    const Plan p = plan ? plan->p : plan_make(d->d, bb, {});
    need(o.forward_mode == SS_FORWARD_HOST || o.forward_mode == SS_FORWARD_DEVICE_GATED,
         "ss_open: unknown forward_mode");
    auto c = std::make_unique<ss_ctx>();
    if (o.forward_mode == SS_FORWARD_DEVICE_GATED) {
      c->dg = open_dg_ctx(d->d, p, o);
    } else {
      need(o.policy == SS_POLICY_LRU || o.policy == SS_POLICY_SCORED, "ss_open: SCORED_AUTO needs device-gated mode");
      c->host = std::make_unique<HostCtx>(d->d, bb, p, o);
    }
    track_open(c.get());
    *out = c.release();
  });
}

void ss_close(ss_ctx* c) {
  if (!c) return;
  untrack(c);
  delete c;
}

int ss_source_direct(const ss_ctx* c, int source) {
  if (!c) return -1;
  if (c->dg) return source < 0 || source >= c->dg->n_sources() ? -1 : c->dg->source_direct(source) ? 1 : 0;
  if (source < 0 || source >= c->host->n_sources()) return -1;
  return c->host->source_direct(source) ? 1 : 0;
}

ss_status ss_seed(ss_ctx* c, int layer, const int32_t* units, int n) {
  return ctx_guard(c, [&] { host_of(c, "ss_seed").seed(layer, units, n); });
}
ss_status ss_begin(ss_ctx* c, const uint32_t* rows, int n_layers) {
  return ctx_guard(c, [&] {
    if (c->dg) c->dg->begin(rows, n_layers);
    else c->host->begin(rows, n_layers);
  });
}
ss_status ss_layer_routes(ss_ctx* c, int layer, const int32_t* ids, int n) {
  return ctx_guard(c, [&] { host_of(c, "ss_layer_routes").routes(layer, ids, n); });
}
ss_status ss_layer_routes_dev(ss_ctx* c, int layer, const int32_t* ids_dev, int n, void* stream) {
  return ctx_guard(c, [&] { host_of(c, "ss_layer_routes_dev").routes_dev(layer, ids_dev, n, stream); });
}
ss_status ss_layer_all(ss_ctx* c, int layer) {
  return ctx_guard(c, [&] { host_of(c, "ss_layer_all").routes_all(layer); });
}
ss_status ss_prefetch(ss_ctx* c, int layer, const int32_t* ids, int n, ss_prefetch_kind kind) {
  return ctx_guard(c, [&] {
    need(kind == SS_PREFETCH_CERTAIN || kind == SS_PREFETCH_SPECULATIVE, "ss_prefetch: unknown kind");
    host_of(c, "ss_prefetch").prefetch(layer, ids, n, kind == SS_PREFETCH_SPECULATIVE);
  });
}
ss_status ss_prefetch_layer(ss_ctx* c, int layer) {
  return ctx_guard(c, [&] { host_of(c, "ss_prefetch_layer").prefetch_layer(layer); });
}
ss_status ss_host_prefetch(ss_ctx* c, int layer, const int32_t* ids, int n) {
  return ctx_guard(c, [&] { host_of(c, "ss_host_prefetch").host_prefetch(layer, ids, n); });
}
ss_status ss_host_prefetch_layer(ss_ctx* c, int layer) {
  return ctx_guard(c, [&] { host_of(c, "ss_host_prefetch_layer").host_prefetch_layer(layer); });
}
ss_status ss_lookahead_select(const float* scores, int rows, int n_experts, int top_k, int32_t* out, int max_out,
                              int* n_out) {
  return guard([&] { lookahead_select(scores, rows, n_experts, top_k, out, max_out, n_out); });
}
ss_status ss_acquire(ss_ctx* c, int layer, void* stream, ss_layer_view* out) {
  return ctx_guard(c, [&] { host_of(c, "ss_acquire").acquire(layer, stream, true, out); });
}
ss_status ss_acquire_groups(ss_ctx* c, int layer, void* stream, ss_layer_view* out) {
  return ctx_guard(c, [&] { host_of(c, "ss_acquire_groups").acquire(layer, stream, false, out); });
}
ss_status ss_group_wait(ss_ctx* c, int layer, int group, void* stream) {
  return ctx_guard(c, [&] { host_of(c, "ss_group_wait").group_wait(layer, group, stream); });
}
ss_status ss_release(ss_ctx* c, int layer, void* stream) {
  return ctx_guard(c, [&] { host_of(c, "ss_release").release(layer, stream); });
}
ss_status ss_end(ss_ctx* c) {
  return ctx_guard(c, [&] {
    if (c->dg) c->dg->end();
    else c->host->end();
  });
}
ss_status ss_check_unit(ss_ctx* c, int layer, int unit) {
  return ctx_guard(c, [&] { host_of(c, "ss_check_unit").check_unit(layer, unit); });
}

// ---- stats (also on a poisoned context) ----
ss_status ss_stats_layer(const ss_ctx* c, int layer, ss_layer_stats* out) {
  return guard([&] {
    need(c && out, "ss_stats_layer: null argument");
    if (c->dg) {
      *out = c->dg->layer_stats(layer);
      return;
    }
    need(layer >= 0 && layer < c->host->n_layers(), "ss_stats_layer: layer out of range");
    *out = c->host->stats(layer);
  });
}
ss_status ss_stats_total(const ss_ctx* c, ss_layer_stats* out) {
  return guard([&] {
    need(c && out, "ss_stats_total: null argument");
    *out = c->dg ? c->dg->total_stats() : c->host->total();
  });
}
void ss_stats_reset(ss_ctx* c) {
  if (!c) return;
  if (c->dg) c->dg->stats_reset();
  else c->host->stats_reset();
}
void ss_set_stats_hook(ss_ctx* c, ss_stats_hook hook, void* user) {
  if (!c) return;
  if (c->dg) c->dg->set_hook(hook, user);
  else if (c->host) c->host->set_hook(hook, user);
}
ss_status ss_stats_to_json(const ss_ctx* c, char** out_json, size_t* out_len) {
  std::string s;
  const ss_status st = guard([&] {
    need(c != nullptr, "ss_stats_to_json: null context");
    s = json_dump(c->dg ? c->dg->stats_json() : c->host->stats_json());
  });
  return st != SS_OK ? st : give_text(s, out_json, out_len);
}
// Any thread (reference include/strix_stream/ss.h:573-615): the first call arms the publication.
ss_status ss_stats_snapshot_sized(const ss_ctx* c, ss_layer_stats* total_out, ss_snapshot_info* info_out,
                                  uint32_t info_size) {
  return guard([&] {
    need(c != nullptr, "ss_stats_snapshot: null context");
    need(total_out || info_out, "ss_stats_snapshot: no output");
    need(!info_out || info_size >= sizeof(uint32_t), "ss_stats_snapshot: info_size below struct_size");
    ss_layer_stats t{};
    ss_snapshot_info i{};
    need(c->dg ? c->dg->snapshot(&t, &i) : c->host->snapshot(&t, &i),
         "no stats snapshot published yet (armed now: published at the next completed ss_end or reset between "
         "forwards)");
    if (total_out) *total_out = t;
    if (info_out) {
      i.struct_size = std::min<uint32_t>(info_size, uint32_t(sizeof i));
      std::memcpy(static_cast<void*>(info_out), &i, i.struct_size);
    }
  });
}
ss_status ss_stats_snapshot_json(const ss_ctx* c, char** out_json, size_t* out_len) {
  std::string s;
  const ss_status st = guard([&] {
    need(c != nullptr, "ss_stats_snapshot_json: null context");
    Json j;
    need(c->dg ? c->dg->snapshot_json(&j) : c->host->snapshot_json(&j),
         "no stats snapshot published yet (armed now: published at the next completed ss_end or reset between "
         "forwards)");
    s = json_dump(j);
  });
  return st != SS_OK ? st : give_text(s, out_json, out_len);
}
ss_status ss_stats_exclusive_sized(const ss_ctx* c, ss_exclusive_stats* out, uint32_t size) {
  return guard([&] {
    need(c && out, "ss_stats_exclusive: null argument");
    need(size >= sizeof(uint32_t), "ss_stats_exclusive: size below struct_size");
    ss_exclusive_stats x = c->dg ? c->dg->exclusive_stats() : c->host->exclusive_stats();
    x.struct_size = std::min<uint32_t>(size, uint32_t(sizeof x));
    std::memcpy(static_cast<void*>(out), &x, x.struct_size);
  });
}

// ---- device-gated ----
ss_status ss_dg_get_device_view_sized(const ss_ctx* c, ss_dg_device_view* out, uint32_t size) {
  return guard([&] {
    need(c && out, "ss_dg_get_device_view: null argument");
    need(size >= 2 * sizeof(uint32_t), "ss_dg_get_device_view: size");
    ss_dg_device_view v = dg_of(c, "ss_dg_get_device_view").device_view();
    v.struct_size = std::min<uint32_t>(size, uint32_t(sizeof v));
    std::memcpy(static_cast<void*>(out), &v, v.struct_size);
  });
}
int ss_dg_gated_index(const ss_ctx* c, int layer) { return c && c->dg ? c->dg->gated_index(layer) : -1; }
ss_status ss_dg_enqueue_begin(ss_ctx* c, void* stream) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_enqueue_begin").enqueue_begin(stream); });
}
ss_status ss_dg_enqueue_export(ss_ctx* c, int g, const int32_t* ids_dev, int n, int n_pred, void* stream) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_enqueue_export").enqueue_export(g, ids_dev, n, n_pred, stream); });
}
ss_status ss_dg_enqueue_predict(ss_ctx* c, int g, const int32_t* ids_dev, int n, void* stream) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_enqueue_predict").enqueue_predict(g, ids_dev, n, stream); });
}
ss_status ss_dg_enqueue_wait(ss_ctx* c, int g, void* stream) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_enqueue_wait").enqueue_wait(g, stream); });
}
ss_status ss_dg_enqueue_end(ss_ctx* c, void* stream) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_enqueue_end").enqueue_end(stream); });
}
ss_status ss_dg_residency(ss_ctx* c, ss_dg_unit* out, uint32_t cap, uint32_t* total) {
  return ctx_guard(c, [&] {
    need(total != nullptr && (out || cap == 0), "ss_dg_residency: null argument");
    *total = dg_of(c, "ss_dg_residency").residency(out, cap);
  });
}
ss_status ss_dg_set_budgets(ss_ctx* c, uint32_t spare_target, uint32_t per_layer, uint32_t per_token) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_set_budgets").set_budgets(spare_target, per_layer, per_token); });
}
ss_status ss_dg_keep(ss_ctx* c, int g, const int32_t* ids, int n) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_keep").keep(g, ids, n); });
}
ss_status ss_dg_set_sched(ss_ctx* c, uint32_t wb_defer, uint32_t flush_ready) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_set_sched").set_sched(wb_defer, flush_ready); });
}
ss_status ss_dg_set_clean_evict(ss_ctx* c, uint32_t on) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_set_clean_evict").set_clean_evict(on); });
}
ss_status ss_dg_timeline_sized(const ss_ctx* c, int g, ss_dg_layer_timeline* out, uint32_t size) {
  return guard([&] {
    need(c && out && size >= sizeof(uint32_t), "ss_dg_timeline: bad argument");
    ss_dg_layer_timeline t;
    dg_of(c, "ss_dg_timeline").timeline(g, &t);
    t.struct_size = std::min<uint32_t>(size, uint32_t(sizeof t));
    std::memcpy(static_cast<void*>(out), &t, t.struct_size);
  });
}
ss_status ss_dg_boundary_timeline_sized(const ss_ctx* c, ss_dg_boundary_timeline* out, uint32_t size) {
  return guard([&] {
    need(c && out && size >= sizeof(uint32_t), "ss_dg_boundary_timeline: bad argument");
    ss_dg_boundary_timeline t;
    dg_of(c, "ss_dg_boundary_timeline").boundary_timeline(&t);
    t.struct_size = std::min<uint32_t>(size, uint32_t(sizeof t));
    std::memcpy(static_cast<void*>(out), &t, t.struct_size);
  });
}
ss_status ss_dg_end_rows(ss_ctx* c, uint32_t rows) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_end_rows").end(rows); });
}
ss_status ss_dg_set_policy(ss_ctx* c, ss_policy policy) {
  return ctx_guard(c, [&] { dg_of(c, "ss_dg_set_policy").set_policy(policy); });
}
ss_status ss_stats_dg_sized(const ss_ctx* c, ss_dg_stats* out, uint32_t size) {
  return guard([&] {
    need(c && out, "ss_stats_dg: null argument");
    need(size >= sizeof(uint32_t), "ss_stats_dg: size");
    ss_dg_stats s = dg_of(c, "ss_stats_dg").stats();
    s.struct_size = std::min<uint32_t>(size, uint32_t(sizeof s));
    std::memcpy(static_cast<void*>(out), &s, s.struct_size);
  });
}

// ---- test hooks (tsa_test.h) ----
ss_status tsa_test_region_of(const ss_ctx* c, uint64_t addr, int* kind, int* index, uint64_t* offset) {
  return guard([&] {
    need(c && kind && index && offset, "tsa_test_region_of: null argument");
    const Region r = host_of(c, "tsa_test_region_of").region_of(addr);
    *kind = r.kind;
    *index = r.index;
    *offset = r.offset;
  });
}
ss_status tsa_test_dg_table(const ss_ctx* c, int32_t* out, uint32_t cap, uint32_t* n) {
  return guard([&] {
    need(c && n && (out || cap == 0), "tsa_test_dg_table: null argument");
    *n = dg_of(c, "tsa_test_dg_table").host_table(out, cap);
  });
}
uint64_t tsa_test_verify_failures(const ss_ctx* c) {
  if (!c) return 0;
  return c->dg ? c->dg->verify_failures() : c->host->verify_failures();
}
int tsa_test_dg_hsa_copies(const ss_ctx* c) { return c && c->dg && c->dg->hsa_copies() ? 1 : 0; }
ss_status tsa_test_host_copies(const ss_ctx* c, uint64_t* units, uint64_t* copies) {
  return guard([&] {
    need(c && units && copies, "tsa_test_host_copies: null argument");
    need(c->host != nullptr, "tsa_test_host_copies: a host-contract context");
    c->host->copy_counts(units, copies);
  });
}
ss_status tsa_test_host_waits(const ss_ctx* c, uint64_t* issued, uint64_t* skipped) {
  return guard([&] {
    need(c && issued && skipped, "tsa_test_host_waits: null argument");
    need(c->host != nullptr, "tsa_test_host_waits: a host-contract context");
    c->host->wait_counts(issued, skipped);
  });
}
ss_status ss_test_hold_readers(ss_ctx* c, int hold) {
  return guard([&] {
    need(c != nullptr && c->host != nullptr, "ss_test_hold_readers: a host-contract context");
    c->host->test_hold_readers(hold != 0);
  });
}
ss_status ss_test_ra_quiesce(ss_ctx* c) {
  return guard([&] {
    need(c != nullptr && c->host != nullptr, "ss_test_ra_quiesce: a host-contract context");
    c->host->test_ra_quiesce();
  });
}
ss_status ss_test_inject(ss_ctx* c, int what) {
  return ctx_guard(c, [&] { host_of(c, "ss_test_inject").test_inject(what); });
}
ss_status ss_test_check_exclusive(ss_ctx* c) {
  return guard([&] {  // a broken rule is reported (SS_E_INVALID) and poisons nothing
    need(c != nullptr, "ss_test_check_exclusive: null context");
    host_of(c, "ss_test_check_exclusive").check_exclusive();
  });
}
ss_status ss_test_dg_check(ss_ctx* c) {
  return guard([&] {  // a broken invariant is reported (SS_E_BACKEND) and poisons nothing
    need(c != nullptr, "ss_test_dg_check: null context");
    dg_of(c, "ss_test_dg_check").test_check();
  });
}
ss_status ss_test_dg_stop_service(ss_ctx* c) {
  return ctx_guard(c, [&] { dg_of(c, "ss_test_dg_stop_service").test_stop_service(); });
}
ss_status tsa_test_profile_enable(ss_ctx* c, int on) {
  return guard([&] {
    need(c != nullptr, "tsa_test_profile_enable: null context");
    need(on >= 0 && on <= (TSA_TEST_PROF_COPY | TSA_TEST_PROF_WRITEBACK | TSA_TEST_PROF_VERIFY),
         "tsa_test_profile_enable: on is 0, 1 or a mask of TSA_TEST_PROF_*");
    if (c->dg) c->dg->profile_enable(on);
    else c->host->profile_enable(on);
  });
}
ss_status tsa_test_profile_read(ss_ctx* c, int wait, tsa_test_profile* out) {
  return guard([&] {
    need(c && out, "tsa_test_profile_read: null argument");
    *out = c->dg ? c->dg->profile_read(wait != 0) : c->host->profile_read(wait != 0);
  });
}
ss_status tsa_test_dg_stamps(const ss_ctx* c, uint64_t* out, uint32_t cap, uint32_t* n) {
  return guard([&] {
    need(c && n && (out || cap == 0), "tsa_test_dg_stamps: null argument");
    *n = dg_of(c, "tsa_test_dg_stamps").stamps(out, cap);
  });
}
ss_status tsa_test_dg_corrupt_block(ss_ctx* c, int gated, int unit, uint64_t offset) {
  return guard([&] {
    need(c != nullptr, "tsa_test_dg_corrupt_block: null context");
    dg_of(c, "tsa_test_dg_corrupt_block").corrupt_block(gated, unit, offset);
  });
}

}  // extern "C"
