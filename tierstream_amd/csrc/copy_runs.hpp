// Runs of host-to-device unit copies that can go as one copy: consecutive orders of one layer whose sources lie in one
// pinned allocation and whose destinations lie in one device allocation, each a step of exactly one slot further on
// both sides (a step of at least the unit size and under twice it: slots and blocks sit one stride apart, the stride
// under the unit size plus its alignment), so no slot or block of another unit lies inside the copied span.
#pragma once

#include <cstddef>
#include <cstdint>

namespace tsa {

struct CopyRunItem {
  int32_t layer = 0;
  int32_t src_alloc = -1;  // -1: not from a pinned allocation (never merged)
  int32_t dst_alloc = -1;
  uint64_t src = 0, dst = 0;  // addresses
};

// The end (exclusive) of the run that starts at items[first]; cap bounds the run's span in bytes (at least one unit).
inline size_t copy_run_end(const CopyRunItem* items, size_t count, size_t first, uint64_t unit_bytes, uint64_t cap) {
  const CopyRunItem& a = items[first];
  const int64_t n = int64_t(unit_bytes);
  int64_t stride = 0;
  size_t j = first + 1;
  for (; j < count; ++j) {
    const CopyRunItem& p = items[j - 1];
    const CopyRunItem& q = items[j];
    if (a.src_alloc < 0 || q.layer != a.layer || q.src_alloc != a.src_alloc || q.dst_alloc != a.dst_alloc) break;
    const int64_t ds = int64_t(q.dst - p.dst), sd = int64_t(q.src - p.src);
    if (ds != sd || ds < n || ds >= 2 * n || (stride && ds != stride)) break;
    if (uint64_t(ds) * (j - first) + unit_bytes > cap) break;
    stride = ds;
  }
  return j;
}

}  // namespace tsa
