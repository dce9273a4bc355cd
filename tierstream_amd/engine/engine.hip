// The synthetic engine the tests and the benchmark drive libtierstream_amd with (not part of the product): what an
// inference engine does around the serve path, with the model math replaced by a checksum of every routed unit's
// bytes read through the library's tables. The checksum kernels read HBM like a batch-1 MoE layer reads its experts
// (every byte of every routed unit once), so in the benchmark they stand in for the expert compute.
//
// Checksum of a unit: sum over its little-endian 32-bit words w_j of w_j * ((j mod 251) + 1), mod 2^64 (words counted
// from the unit's first byte, across its parts; a unit's bytes are a multiple of 4 in every workload here).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <string>
#include <vector>

#include "strix_stream/ss.h"
#include "tierstream/ts.h"
#include "tierstream_amd/tsa_test.h"

namespace {

constexpr int kThreads = 256;
constexpr uint64_t kChunk = 256 * 1024;  // bytes per workgroup

// Words [first_word, first_word + n_words) of a unit, read from p (16-byte aligned; units below 16 GiB, so word indexes
// fit 32 bits). The read is shaped like a batch-1 expert GEMV's: 16-byte loads, four per lane in flight, every byte
// once; the weight of word j is (j mod 251) + 1, carried from word to word instead of divided per word.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g4_t;

__device__ __forceinline__ uint64_t sum4(u32x4 v, uint32_t m) {  // m = (index of v.x) mod 251
  uint64_t s = uint64_t(v.x) * (m + 1);
  m = m == 250u ? 0u : m + 1u;
  s += uint64_t(v.y) * (m + 1);
  m = m == 250u ? 0u : m + 1u;
  s += uint64_t(v.z) * (m + 1);
  m = m == 250u ? 0u : m + 1u;
  return s + uint64_t(v.w) * (m + 1);
}

__device__ __forceinline__ uint64_t sum_words(const uint32_t* p, uint64_t first_word, uint64_t n_words) {
  constexpr uint32_t kU = 4;
  g4_t* q = reinterpret_cast<g4_t*>(reinterpret_cast<uintptr_t>(p));
  const uint32_t w0 = uint32_t(first_word), nq = uint32_t(n_words / 4);
  uint64_t s = 0;
  uint32_t i = threadIdx.x;
  for (; i + (kU - 1) * kThreads < nq; i += kU * kThreads) {
    u32x4 v[kU];
#pragma unroll
    for (uint32_t k = 0; k < kU; ++k) v[k] = q[i + k * kThreads];
#pragma unroll
    for (uint32_t k = 0; k < kU; ++k) s += sum4(v[k], (w0 + 4 * (i + k * kThreads)) % 251u);
  }
  for (; i < nq; i += kThreads) s += sum4(q[i], (w0 + 4 * i) % 251u);
  for (uint32_t j = 4 * nq + threadIdx.x; j < uint32_t(n_words); j += kThreads)  // a tail of 1-3 words
    s += uint64_t(p[j]) * ((w0 + j) % 251u + 1);
  return s;
}

__device__ __forceinline__ void block_add(uint64_t s, unsigned long long* out) {
  for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
  __shared__ uint64_t part[kThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t t = 0;
    for (int w = 0; w < kThreads / 64; ++w) t += part[w];
    atomicAdd(out, (unsigned long long)t);
  }
}

// Host contract: blockIdx.y = routed unit i (its table entry table_dev[ids[i]]); blockIdx.x = a chunk of its bytes.
__global__ __launch_bounds__(kThreads) void checksum_table(const uint64_t* table_dev, const int32_t* ids, uint64_t bytes,
                                                           unsigned long long* out) {
  const int32_t u = ids[blockIdx.y];
  const uint64_t a = table_dev[u];
  const uint64_t off = uint64_t(blockIdx.x) * kChunk;
  if (a == 0 || off >= bytes) return;
  const uint64_t n = (bytes - off < kChunk ? bytes - off : kChunk) / 4;
  block_add(sum_words(reinterpret_cast<const uint32_t*>(a + off), off / 4, n), out + blockIdx.y);
}

// Device-gated: the slot from ss_dg_slot, then each part at base + slot * stride.
__global__ __launch_bounds__(kThreads) void checksum_dg(ss_dg_device_view v, uint32_t g, const int32_t* ids,
                                                        unsigned long long* out, unsigned long long* start) {
  __shared__ int32_t slot_s;
  if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0) start[g] = wall_clock64();  // the layer's compute began
  if (threadIdx.x == 0) slot_s = ss_dg_slot(&v, g, ids[blockIdx.y]);
  __syncthreads();
  const int32_t slot = slot_s;
  uint64_t b = blockIdx.x, word0 = 0;
  for (uint32_t p = 0; p < v.n_parts; ++p) {  // chunk b of the unit: each part has its own whole chunks
    const uint64_t pb = v.parts[p].bytes, nb = (pb + kChunk - 1) / kChunk;
    if (b < nb) {
      const uint64_t off = b * kChunk;
      const uint64_t n = (pb - off < kChunk ? pb - off : kChunk) / 4;
      const uint32_t* base = reinterpret_cast<const uint32_t*>(static_cast<const char*>(v.parts[p].base) +
                                                               uint64_t(slot) * v.parts[p].stride + off);
      block_add(sum_words(base, word0 + off / 4, n), out + blockIdx.y);
      return;
    }
    b -= nb;
    word0 += pb / 4;
  }
}

// Resident-first reads before layer g's wait (ss_dg_slot_if_ready): one workgroup per routed id resolves the slot
// once; a published slot's unit is checksummed in full into out[i] and ready[i] = 1, an unpublished one leaves both 0.
// A slot entry is published only once its unit's bytes are complete, so every ready checksum must be exact.
__global__ __launch_bounds__(kThreads) void checksum_early_dg(ss_dg_device_view v, uint32_t g, const int32_t* ids,
                                                              unsigned long long* out, uint32_t* ready) {
  __shared__ int32_t slot_s;
  if (threadIdx.x == 0) slot_s = ss_dg_slot_if_ready(&v, g, ids[blockIdx.x]);
  __syncthreads();
  const int32_t slot = slot_s;
  if (slot < 0) return;
  uint64_t word0 = 0, s = 0;
  for (uint32_t p = 0; p < v.n_parts; ++p) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(static_cast<const char*>(v.parts[p].base) +
                                                             uint64_t(slot) * v.parts[p].stride);
    s += sum_words(base, word0, v.parts[p].bytes / 4);
    word0 += v.parts[p].bytes / 4;
  }
  block_add(s, out + blockIdx.x);
  if (threadIdx.x == 0) ready[blockIdx.x] = 1;
}

ss_status ck(hipError_t e) { return e == hipSuccess ? SS_OK : SS_E_BACKEND; }
#define TSE_CK(x)                                          \
  do {                                                     \
    const ss_status s_ = (x);                              \
    if (s_ != SS_OK) return s_;                            \
  } while (0)
#define TSE_HIP(x) TSE_CK(ck(x))

uint32_t chunks_of(uint64_t bytes) { return uint32_t((bytes + kChunk - 1) / kChunk); }

double ms_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

}  // namespace

extern "C" {

// Host contract: `steps` forwards over every layer with units. routes[step][layer][max_ids] (-1 = none);
// mode 0 = ss_layer_routes + ss_acquire, 1 = ss_layer_all + ss_acquire, 2 = ss_layer_routes + ss_acquire_groups with
// one ss_group_wait per group; mode | 0x10: a new engine stream for every forward, the last one destroyed after its
// forward (an engine that does not keep one stream; a new stream may reuse the old handle); mode | 0x20: the null
// stream, for the ss_* calls (nullptr) and the engine's own work; host_lookahead H > 0: after each layer's routes, ss_host_prefetch_layer of the next H
// layers with units; prefetch (same shape as routes, may be NULL): after layer l's acquire, ss_prefetch of layer l + 1
// with its row, CERTAIN on even steps and SPECULATIVE on odd ones (the next layer's ids while this one holds its slots).
// Outputs (may be NULL): checksums[step][layer][max_ids] of the routed ids (0 for -1),
// tables[step][layer][max_units] = the layer's table_host, stats[step] = the forward's totals, step_ms[step].
__attribute__((visibility("default"))) ss_status tse_host_run_ex(ss_ctx* c, const ss_desc* d, int steps,
                                                                 const int32_t* routes, const int32_t* prefetch,
                                                                 int max_ids, int max_units, int mode,
                                                                 int host_lookahead, uint64_t* checksums,
                                                                 uint64_t* tables, ss_layer_stats* stats,
                                                                 double* step_ms) {
  const int L = ss_desc_n_layers(d);
  const bool null_stream = (mode & 0x20) != 0;
  const bool fresh_streams = (mode & 0x10) != 0 && !null_stream;
  mode &= 0xF;
  hipStream_t s = nullptr;
  if (!null_stream) TSE_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  int32_t* ids_dev = nullptr;
  int32_t* ids_host = nullptr;  // pinned: a layer's id copy needs no host wait (the step's end waits for them all)
  unsigned long long* out_dev = nullptr;
  ss_status st = SS_OK;
  if (hipMalloc(&ids_dev, 4ull * max_ids * L) != hipSuccess || hipMalloc(&out_dev, 8ull * max_ids * L) != hipSuccess ||
      hipHostMalloc(&ids_host, 4ull * max_ids * L, hipHostMallocDefault) != hipSuccess)
    st = SS_E_NOMEM;
  for (int step = 0; st == SS_OK && step < steps; ++step) {
    if (fresh_streams && step > 0) {  // (the last forward's work on s has completed: it was synchronized)
      (void)hipStreamDestroy(s);
      s = nullptr;
      if ((st = ck(hipStreamCreateWithFlags(&s, hipStreamNonBlocking))) != SS_OK) break;
    }
    const auto t0 = std::chrono::steady_clock::now();
    ss_layer_stats before{};
    ss_stats_total(c, &before);
    if ((st = ss_begin(c, nullptr, 0)) != SS_OK) break;
    if ((st = ck(hipMemsetAsync(out_dev, 0, 8ull * max_ids * L, s))) != SS_OK) break;
    for (int l = 0; st == SS_OK && l < L; ++l) {
      const int nu = ss_desc_layer_units(d, l);
      if (nu <= 0) continue;
      const int32_t* r = routes + (size_t(step) * L + l) * max_ids;
      int n = 0;
      while (n < max_ids && r[n] >= 0) ++n;
      if (mode == 1) st = ss_layer_all(c, l);
      else st = ss_layer_routes(c, l, r, n);
      for (int h = l + 1, left = host_lookahead; st == SS_OK && left > 0 && h < L; ++h)
        if (ss_desc_layer_units(d, h) > 0) {
          st = ss_host_prefetch_layer(c, h);
          --left;
        }
      if (st != SS_OK) break;
      ss_layer_view v{};
      st = mode == 2 ? ss_acquire_groups(c, l, s, &v) : ss_acquire(c, l, s, &v);
      if (st != SS_OK) break;
      if (mode == 2)
        for (int gi = 1; st == SS_OK && gi < v.n_groups; ++gi) st = ss_group_wait(c, l, gi, s);
      if (st != SS_OK) break;
      if (prefetch && l + 1 < L && ss_desc_layer_units(d, l + 1) > 0) {
        const int32_t* q = prefetch + (size_t(step) * L + l + 1) * max_ids;
        int m = 0;
        while (m < max_ids && q[m] >= 0) ++m;
        if (m && (st = ss_prefetch(c, l + 1, q, m, step % 2 ? SS_PREFETCH_SPECULATIVE : SS_PREFETCH_CERTAIN)) != SS_OK)
          break;
      }
      const int n_read = mode == 1 ? std::min(nu, max_ids) : n;
      int32_t* rid = ids_host + size_t(l) * max_ids;
      for (int i = 0; i < n_read; ++i) rid[i] = mode == 1 ? i : r[i];
      if (n_read > 0) {
        st = ck(hipMemcpyAsync(ids_dev + size_t(l) * max_ids, rid, 4ull * n_read, hipMemcpyHostToDevice, s));
        if (st == SS_OK) {
          hipLaunchKernelGGL(checksum_table, dim3(chunks_of(ss_desc_unit_bytes(d, l)), n_read), dim3(kThreads), 0, s,
                             v.table_dev, ids_dev + size_t(l) * max_ids, ss_desc_unit_bytes(d, l),
                             out_dev + size_t(l) * max_ids);
          st = ck(hipGetLastError());
        }
      }
      if (st == SS_OK && tables)
        std::memcpy(tables + (size_t(step) * L + l) * max_units, v.table_host, 8ull * std::min(nu, max_units));
      if (st == SS_OK) st = ss_release(c, l, s);
    }
    if (st == SS_OK) st = ck(hipStreamSynchronize(s));
    const ss_status end_st = ss_end(c);
    if (st == SS_OK) st = end_st;
    if (st != SS_OK) break;
    if (step_ms) step_ms[step] = ms_since(t0);
    if (stats) {
      ss_layer_stats after{};
      ss_stats_total(c, &after);
      ss_layer_stats& o = stats[step];
      o = after;
      o.routed -= before.routed, o.hits -= before.hits, o.admitted -= before.admitted;
      o.transient -= before.transient, o.evicted -= before.evicted, o.prefetched -= before.prefetched;
      o.spec_issued -= before.spec_issued, o.spec_used -= before.spec_used, o.spec_dropped -= before.spec_dropped;
      o.bytes_pinned -= before.bytes_pinned, o.bytes_disk -= before.bytes_disk, o.wait_ns -= before.wait_ns;
    }
    if (checksums) {
      std::vector<unsigned long long> all(size_t(max_ids) * L);
      if ((st = ck(hipMemcpyAsync(all.data(), out_dev, 8ull * max_ids * L, hipMemcpyDeviceToHost, s))) != SS_OK ||
          (st = ck(hipStreamSynchronize(s))) != SS_OK)
        break;
      std::memcpy(checksums + size_t(step) * L * max_ids, all.data(), 8ull * max_ids * L);
    }
  }
  (void)hipStreamSynchronize(s);
  (void)hipFree(ids_dev);
  (void)hipFree(out_dev);
  (void)hipHostFree(ids_host);
  if (s) (void)hipStreamDestroy(s);
  return st;
}

__attribute__((visibility("default"))) ss_status tse_host_run(ss_ctx* c, const ss_desc* d, int steps,
                                                              const int32_t* routes, int max_ids, int max_units,
                                                              int mode, uint64_t* checksums, uint64_t* tables,
                                                              ss_layer_stats* stats, double* step_ms) {
  return tse_host_run_ex(c, d, steps, routes, nullptr, max_ids, max_units, mode, 0, checksums, tables, stats,
                         step_ms);
}

// ---- device-gated ----
struct TseDg {
  ss_ctx* c = nullptr;
  uint32_t G = 0, n_ids = 0, max_chunks = 0;
  uint32_t n_pred = 0;  // ids predicted at each layer for the next one (0: no predictions)
  uint32_t rows = 1;  // the verify rows each token closes (above one: ss_dg_end_rows instead of ss_end)
  bool checksum = true, dg = true;
  bool early = false;  // resident-first reads before every wait (checksum_early_dg)
  hipStream_t s = nullptr;
  int32_t* ids_dev = nullptr;               // [G][64]
  int32_t* pred_dev = nullptr;              // [G][64]: row g predicts layer g + 1
  unsigned long long* out_dev = nullptr;    // [G][64]
  unsigned long long* start_dev = nullptr;  // [G]: wall clock at each layer's first checksum workgroup
  unsigned long long* early_dev = nullptr;  // [G][64]: resident-first checksums
  uint32_t* ready_dev = nullptr;            // [G][64]: 1 where the early read found a published slot
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  ss_dg_device_view view{};

  ~TseDg() {
    if (s) (void)hipStreamSynchronize(s);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipFree(ids_dev);
    (void)hipFree(pred_dev);
    (void)hipFree(out_dev);
    (void)hipFree(start_dev);
    (void)hipFree(early_dev);
    (void)hipFree(ready_dev);
    if (s) (void)hipStreamDestroy(s);
  }
};

static ss_status tse_enqueue_token(TseDg* e) {
  if (e->dg) TSE_CK(ss_dg_enqueue_begin(e->c, e->s));
  for (uint32_t g = 0; g < e->G; ++g) {
    const int np = e->n_pred && g + 1 < e->G ? int(e->n_pred) : 0;
    if (e->dg) TSE_CK(ss_dg_enqueue_export(e->c, int(g), e->ids_dev + 64 * g, int(e->n_ids), np, e->s));
    if (e->dg && np) TSE_CK(ss_dg_enqueue_predict(e->c, int(g), e->pred_dev + 64 * g, np, e->s));
    if (e->early) {
      hipLaunchKernelGGL(checksum_early_dg, dim3(e->n_ids), dim3(kThreads), 0, e->s, e->view, g, e->ids_dev + 64 * g,
                         e->early_dev + 64 * g, e->ready_dev + 64 * g);
      TSE_HIP(hipGetLastError());
    }
    if (e->dg) TSE_CK(ss_dg_enqueue_wait(e->c, int(g), e->s));
    if (e->checksum) {
      hipLaunchKernelGGL(checksum_dg, dim3(e->max_chunks, e->n_ids), dim3(kThreads), 0, e->s, e->view, g,
                         e->ids_dev + 64 * g, e->out_dev + 64 * g, e->start_dev);
      TSE_HIP(hipGetLastError());
    }
  }
  if (e->dg) TSE_CK(ss_dg_enqueue_end(e->c, e->s));
  return SS_OK;
}

// A device-gated engine: n_ids routed ids per gated layer per token, captured once into a hipGraph (use_graph = 1) or
// enqueued per token. checksum = 0 leaves out the checksum kernels; dg = 0 leaves out the gating kernels (a baseline
// graph for the wait overhead: the same checksum kernels, nothing gated).
__attribute__((visibility("default"))) ss_status tse_dg_create_pred(ss_ctx* c, uint32_t n_ids, uint32_t n_pred,
                                                                    int use_graph, int checksum, int dg, void** out);
__attribute__((visibility("default"))) ss_status tse_dg_create(ss_ctx* c, uint32_t n_ids, int use_graph, int checksum,
                                                               int dg, void** out) {
  return tse_dg_create_pred(c, n_ids, 0, use_graph, checksum, dg, out);
}

// As tse_dg_create, with n_pred (<= 64) ids predicted at every gated layer but the last for the next one (each token's
// predictions come with its routes, tse_dg_token_pred).
__attribute__((visibility("default"))) ss_status tse_dg_create_ex(ss_ctx* c, uint32_t n_ids, uint32_t n_pred,
                                                                  int use_graph, int checksum, int dg, int early,
                                                                  void** out);
__attribute__((visibility("default"))) ss_status tse_dg_create_pred(ss_ctx* c, uint32_t n_ids, uint32_t n_pred,
                                                                    int use_graph, int checksum, int dg, void** out) {
  return tse_dg_create_ex(c, n_ids, n_pred, use_graph, checksum, dg, 0, out);
}

// As tse_dg_create_pred; early = 1 adds resident-first reads through ss_dg_slot_if_ready before every layer's wait
// (tse_dg_early reads the last token's results back).
__attribute__((visibility("default"))) ss_status tse_dg_create_ex(ss_ctx* c, uint32_t n_ids, uint32_t n_pred,
                                                                  int use_graph, int checksum, int dg, int early,
                                                                  void** out) {
  if (n_ids < 1 || n_ids > 64 || n_pred > 64) return SS_E_INVALID;
  auto* e = new TseDg;
  e->c = c;
  e->n_ids = n_ids;
  e->n_pred = n_pred;
  e->checksum = checksum != 0;
  e->dg = dg != 0;
  e->early = early != 0;
  ss_status st = ss_dg_get_device_view(c, &e->view);
  if (st != SS_OK) {
    delete e;
    return st;
  }
  e->G = e->view.n_gated;
  uint32_t chunks = 0;
  for (uint32_t p = 0; p < e->view.n_parts; ++p) chunks += chunks_of(e->view.parts[p].bytes);
  e->max_chunks = chunks;
  if (hipStreamCreateWithFlags(&e->s, hipStreamNonBlocking) != hipSuccess ||
      hipMalloc(&e->ids_dev, 4ull * 64 * e->G) != hipSuccess || hipMalloc(&e->pred_dev, 4ull * 64 * e->G) != hipSuccess ||
      hipMalloc(&e->out_dev, 8ull * 64 * e->G) != hipSuccess ||
      hipMalloc(&e->start_dev, 8ull * e->G) != hipSuccess ||
      (e->early && (hipMalloc(&e->early_dev, 8ull * 64 * e->G) != hipSuccess ||
                    hipMalloc(&e->ready_dev, 4ull * 64 * e->G) != hipSuccess))) {
    delete e;
    return SS_E_NOMEM;
  }
  (void)hipMemset(e->out_dev, 0, 8ull * 64 * e->G);
  (void)hipMemset(e->ids_dev, 0, 4ull * 64 * e->G);
  (void)hipMemset(e->pred_dev, 0, 4ull * 64 * e->G);
  (void)hipMemset(e->start_dev, 0, 8ull * e->G);
  if (use_graph) {
    st = ck(hipStreamBeginCapture(e->s, hipStreamCaptureModeThreadLocal));
    if (st == SS_OK) {
      const ss_status qs = tse_enqueue_token(e);
      const ss_status es = ck(hipStreamEndCapture(e->s, &e->graph));
      st = qs != SS_OK ? qs : es;
    }
    if (st == SS_OK) st = ck(hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0));
    if (st != SS_OK) {
      delete e;
      return st;
    }
  }
  *out = e;
  return SS_OK;
}

// One token: routes (host, [G][n_ids]) uploaded, ss_begin, the graph (or the kernels), ss_end. checksums
// ([G][n_ids]) and token_ms (begin -> end) may be NULL.
__attribute__((visibility("default"))) ss_status tse_dg_token_pred(void* h, const int32_t* routes, const int32_t* preds,
                                                                   uint64_t* checksums, double* token_ms);
__attribute__((visibility("default"))) ss_status tse_dg_token(void* h, const int32_t* routes, uint64_t* checksums,
                                                              double* token_ms) {
  return tse_dg_token_pred(h, routes, nullptr, checksums, token_ms);
}

// The token's routes (and predictions) on the device and its output words cleared, before ss_begin.
static ss_status stage_token(TseDg* e, const int32_t* routes, const int32_t* preds) {
  std::vector<int32_t> ids(size_t(64) * e->G, 0);
  for (uint32_t g = 0; g < e->G; ++g)
    for (uint32_t i = 0; i < e->n_ids; ++i) ids[64 * g + i] = routes[size_t(g) * e->n_ids + i];
  TSE_HIP(hipMemcpyAsync(e->ids_dev, ids.data(), 4ull * ids.size(), hipMemcpyHostToDevice, e->s));
  if (e->n_pred) {
    std::vector<int32_t> pv(size_t(64) * e->G, 0);
    for (uint32_t g = 0; preds && g < e->G; ++g)
      for (uint32_t i = 0; i < e->n_pred; ++i) pv[64 * g + i] = preds[size_t(g) * e->n_pred + i];
    TSE_HIP(hipMemcpyAsync(e->pred_dev, pv.data(), 4ull * pv.size(), hipMemcpyHostToDevice, e->s));
    TSE_HIP(hipStreamSynchronize(e->s));  // (pv is a local)
  }
  if (e->checksum) TSE_HIP(hipMemsetAsync(e->out_dev, 0, 8ull * 64 * e->G, e->s));
  if (e->early) {
    TSE_HIP(hipMemsetAsync(e->early_dev, 0, 8ull * 64 * e->G, e->s));
    TSE_HIP(hipMemsetAsync(e->ready_dev, 0, 4ull * 64 * e->G, e->s));
  }
  TSE_HIP(hipStreamSynchronize(e->s));
  return SS_OK;
}

// ss_begin and the token's kernels enqueued, nothing more: the token stays open (an engine that fails mid-token).
__attribute__((visibility("default"))) ss_status tse_dg_token_open(void* h, const int32_t* routes) {
  TseDg* e = static_cast<TseDg*>(h);
  TSE_CK(stage_token(e, routes, nullptr));
  if (e->dg) TSE_CK(ss_begin(e->c, nullptr, 0));
  return e->exec ? ck(hipGraphLaunch(e->exec, e->s)) : tse_enqueue_token(e);
}

// preds ([G][n_pred], row g for layer g + 1; the last row unused) may be NULL: zeros are predicted then.
__attribute__((visibility("default"))) ss_status tse_dg_token_pred(void* h, const int32_t* routes, const int32_t* preds,
                                                                   uint64_t* checksums, double* token_ms) {
  TseDg* e = static_cast<TseDg*>(h);
  TSE_CK(stage_token(e, routes, preds));
  const auto t0 = std::chrono::steady_clock::now();
  if (e->dg) TSE_CK(ss_begin(e->c, nullptr, 0));
  ss_status st = e->exec ? ck(hipGraphLaunch(e->exec, e->s)) : tse_enqueue_token(e);
  const ss_status end_st = !e->dg          ? ck(hipStreamSynchronize(e->s))
                            : e->rows > 1 ? ss_dg_end_rows(e->c, e->rows)
                                          : ss_end(e->c);
  if (token_ms) *token_ms = ms_since(t0);
  (void)hipStreamSynchronize(e->s);
  if (st == SS_OK) st = end_st;
  // the checksums also when the token failed (a failed token's reads after its abort are the guard slot's zeros)
  if (checksums) {
    std::vector<unsigned long long> out(size_t(64) * e->G);
    // on the engine's stream (the null stream would wait for the library's blocking copy streams)
    TSE_HIP(hipMemcpyAsync(out.data(), e->out_dev, 8ull * out.size(), hipMemcpyDeviceToHost, e->s));
    TSE_HIP(hipStreamSynchronize(e->s));
    for (uint32_t g = 0; g < e->G; ++g)
      for (uint32_t i = 0; i < e->n_ids; ++i) checksums[size_t(g) * e->n_ids + i] = out[64 * g + i];
  }
  return st;
}

// ss_dg_slot / ts_dg_slot on the device over a synthetic view (no context): slot_of[n_keys], unit_base[n_gated + 1],
// the guard slot, an abort word and an absent_err word (with_absent = 0: the view has no absent_err). Query i resolves
// id[i] of gated layer g[i] (every g[i] < n_gated); out_ss / out_ts get both results, *absent the absent_err word.
__global__ void slot_probe(ss_dg_device_view v, const uint32_t* g, const int32_t* id, uint32_t n, int32_t* out_ss,
                           int32_t* out_ts) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out_ss[i] = ss_dg_slot(&v, g[i], id[i]);
  out_ts[i] = ts_dg_slot(&v, g[i], id[i]);
}

__attribute__((visibility("default"))) ss_status tse_slot_probe(const int32_t* slot_of, uint32_t n_keys,
                                                                const uint32_t* unit_base, uint32_t n_gated,
                                                                uint32_t guard, uint32_t aborted, int with_absent,
                                                                const uint32_t* g, const int32_t* id, uint32_t n,
                                                                int32_t* out_ss, int32_t* out_ts, uint32_t* absent) {
  for (uint32_t i = 0; i < n; ++i)
    if (g[i] >= n_gated) return SS_E_INVALID;
  for (uint32_t k = 0; k <= n_gated; ++k)
    if (unit_base[k] > n_keys || (k && unit_base[k] < unit_base[k - 1])) return SS_E_INVALID;
  int32_t *d_slot = nullptr, *d_id = nullptr, *d_ss = nullptr, *d_ts = nullptr;
  uint32_t *d_base = nullptr, *d_g = nullptr, *d_words = nullptr;
  ss_status st = SS_OK;
  if (hipMalloc(&d_slot, 4ull * (n_keys ? n_keys : 1)) != hipSuccess || hipMalloc(&d_base, 4ull * (n_gated + 1)) != hipSuccess ||
      hipMalloc(&d_g, 4ull * n) != hipSuccess || hipMalloc(&d_id, 4ull * n) != hipSuccess ||
      hipMalloc(&d_ss, 4ull * n) != hipSuccess || hipMalloc(&d_ts, 4ull * n) != hipSuccess ||
      hipMalloc(&d_words, 8) != hipSuccess)
    st = SS_E_NOMEM;
  const uint32_t words[2] = {aborted, 0};
  if (st == SS_OK) {
    st = ck(hipMemcpy(d_slot, slot_of, 4ull * n_keys, hipMemcpyHostToDevice));
    if (st == SS_OK) st = ck(hipMemcpy(d_base, unit_base, 4ull * (n_gated + 1), hipMemcpyHostToDevice));
    if (st == SS_OK) st = ck(hipMemcpy(d_g, g, 4ull * n, hipMemcpyHostToDevice));
    if (st == SS_OK) st = ck(hipMemcpy(d_id, id, 4ull * n, hipMemcpyHostToDevice));
    if (st == SS_OK) st = ck(hipMemcpy(d_words, words, 8, hipMemcpyHostToDevice));
  }
  if (st == SS_OK) {
    ss_dg_device_view v;
    std::memset(&v, 0, sizeof v);
    v.struct_size = uint32_t(sizeof v);
    v.protocol = SS_DG_PROTOCOL;
    v.n_gated = n_gated;
    v.guard_slot = guard;
    v.slots = guard + 1;
    v.slot_of = d_slot;
    v.unit_base = d_base;
    v.abort = d_words;
    v.absent_err = with_absent ? d_words + 1 : nullptr;
    hipLaunchKernelGGL(slot_probe, dim3((n + 63) / 64), dim3(64), 0, nullptr, v, d_g, d_id, n, d_ss, d_ts);
    st = ck(hipGetLastError());
    if (st == SS_OK) st = ck(hipDeviceSynchronize());
    if (st == SS_OK) st = ck(hipMemcpy(out_ss, d_ss, 4ull * n, hipMemcpyDeviceToHost));
    if (st == SS_OK) st = ck(hipMemcpy(out_ts, d_ts, 4ull * n, hipMemcpyDeviceToHost));
    uint32_t back[2] = {0, 0};
    if (st == SS_OK) st = ck(hipMemcpy(back, d_words, 8, hipMemcpyDeviceToHost));
    if (absent) *absent = back[1];
  }
  (void)hipFree(d_slot);
  (void)hipFree(d_base);
  (void)hipFree(d_g);
  (void)hipFree(d_id);
  (void)hipFree(d_ss);
  (void)hipFree(d_ts);
  (void)hipFree(d_words);
  return st;
}

// The last token's resident-first reads: sums[G][n_ids] and ready[G][n_ids] (an engine created with early = 1).
__attribute__((visibility("default"))) ss_status tse_dg_early(void* h, uint64_t* sums, uint32_t* ready) {
  TseDg* e = static_cast<TseDg*>(h);
  if (!e || !e->early) return SS_E_INVALID;
  std::vector<unsigned long long> s(size_t(64) * e->G);
  std::vector<uint32_t> r(size_t(64) * e->G);
  TSE_HIP(hipMemcpyAsync(s.data(), e->early_dev, 8ull * s.size(), hipMemcpyDeviceToHost, e->s));
  TSE_HIP(hipMemcpyAsync(r.data(), e->ready_dev, 4ull * r.size(), hipMemcpyDeviceToHost, e->s));
  TSE_HIP(hipStreamSynchronize(e->s));
  for (uint32_t g = 0; g < e->G; ++g)
    for (uint32_t i = 0; i < e->n_ids; ++i) {
      sums[size_t(g) * e->n_ids + i] = s[64 * g + i];
      ready[size_t(g) * e->n_ids + i] = r[64 * g + i];
    }
  return SS_OK;
}

// The verify rows each later token closes (1: ss_end; more: ss_dg_end_rows, e.g. a speculative step's rows).
__attribute__((visibility("default"))) ss_status tse_dg_set_rows(void* h, uint32_t rows) {
  if (!h || rows < 1) return SS_E_INVALID;
  static_cast<TseDg*>(h)->rows = rows;
  return SS_OK;
}

// The last token's per-layer compute-start stamps (wall clock, 100 MHz ticks), [G].
__attribute__((visibility("default"))) ss_status tse_dg_stamps(void* h, uint64_t* out) {
  TseDg* e = static_cast<TseDg*>(h);
  TSE_HIP(hipStreamSynchronize(e->s));
  TSE_HIP(hipMemcpy(out, e->start_dev, 8ull * e->G, hipMemcpyDeviceToHost));
  return SS_OK;
}

__attribute__((visibility("default"))) void tse_dg_destroy(void* h) {
  delete static_cast<TseDg*>(h);
}

}  // extern "C"
