// MarkOrder against vector clocks (a test hook, CPU only): random records, waits and stream replacements over a few
// stream handles and events. Each stream's knowledge is a vector clock (per stream, the highest mark it follows; a
// replaced handle names a new stream with a clock of its own); the reference applies every wait, the checked side only
// the waits MarkOrder says are needed. After every step both clocks of every live stream must be equal: a skipped wait
// was implied by one already given.
#include <cstdint>
#include <map>
#include <random>
#include <vector>

#include "stream_order.hpp"
#include "tierstream_amd/tsa_test.h"

namespace tsa {
namespace {

using Clock = std::map<uint32_t, uint64_t>;  // stream (incarnation) -> mark

void join(Clock& a, const Clock& b) {
  for (const auto& [k, v] : b) {
    uint64_t& x = a[k];
    if (v > x) x = v;
  }
}

// mode 0: MarkOrder as built. 1: a planted mistake (any earlier wait for the same stream counts, whatever its mark).
// 2: a planted mistake (a replaced handle is not forgotten).
uint64_t run(uint32_t seed, uint32_t n_ops, uint32_t n_handles, int mode, uint64_t* skipped) {
  std::mt19937_64 rng(seed);
  const uint32_t n_events = 2 * n_handles + 1;
  MarkOrder<uint32_t, uint32_t> order;
  std::vector<uint32_t> inc(n_handles);  // each handle's current stream
  for (uint32_t h = 0; h < n_handles; ++h) inc[h] = h;
  uint32_t next_inc = n_handles;
  std::vector<std::map<uint32_t, int>> waited_any(n_handles);  // mode 1's rule: per handle, streams waited for at all
  std::vector<Clock> full(n_handles), kept(n_handles);
  std::map<uint32_t, uint64_t> marks;
  std::vector<int64_t> ev_stream(n_events, -1);
  std::vector<Clock> ev_full(n_events), ev_kept(n_events);
  *skipped = 0;
  for (uint32_t op = 0; op < n_ops; ++op) {
    const uint32_t h = uint32_t(rng() % n_handles);
    const uint32_t kind = uint32_t(rng() % 16);
    const uint32_t e = uint32_t(rng() % n_events);
    if (kind < 7) {  // record e on h
      const uint64_t k = ++marks[inc[h]];
      full[h][inc[h]] = kept[h][inc[h]] = k;
      ev_stream[e] = inc[h];
      ev_full[e] = full[h];
      ev_kept[e] = kept[h];
      order.recorded(e, h);
    } else if (kind < 15) {  // h waits for e
      if (ev_stream[e] < 0) continue;  // never recorded: the runtime's no-op
      join(full[h], ev_full[e]);
      const uint32_t x = uint32_t(ev_stream[e]);
      bool need = order.needs_wait(h, e);
      if (mode == 1) need = x != inc[h] && !waited_any[h].count(x);
      if (need) {
        join(kept[h], ev_kept[e]);
        order.waited(h, e);
        waited_any[h][x] = 1;
      } else {
        ++*skipped;
      }
    } else {  // h now names a new stream, which follows nothing
      inc[h] = next_inc++;
      full[h].clear();
      kept[h].clear();
      waited_any[h].clear();
      if (mode != 2) order.forget(h);
    }
    for (uint32_t t = 0; t < n_handles; ++t)
      if (full[t] != kept[t]) return op + 1;
  }
  return 0;
}

}  // namespace
}  // namespace tsa

extern "C" ss_status tsa_test_stream_order(uint32_t seed, uint32_t n_ops, uint32_t n_streams, int mode,
                                           uint64_t* counts) {
  if (n_streams < 1 || n_streams > 16 || mode < 0 || mode > 2 || !counts) return SS_E_INVALID;
  counts[0] = tsa::run(seed, n_ops, n_streams, mode, &counts[1]);
  return SS_OK;
}
