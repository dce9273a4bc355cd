// ss_lookahead_select (reference include/strix_stream/ss.h:496-499, src/capi.cpp:577-612): from `rows` router score
// rows of the next layer, the union of each row's top_k experts, ordered by the best rank an expert reached in any
// row, then by its best score at that rank, then by id.
//
// Each row's top_k comes from one nth_element over an index buffer (O(n_experts)) followed by a sort of the k winners
// only; an expert's (best rank, best score at that rank) pair is folded in per row. Scores order descending with the
// lower id first on ties; a NaN orders below every number (the selection stays a strict weak order), which only
// matters to callers that pass NaN.
#include <algorithm>
#include <cmath>
#include <vector>

#include "capi_internal.hpp"

namespace tsa {
namespace {

// x strictly above y (NaN below every number, NaNs equal)
bool above(float x, float y) {
  const bool nx = std::isnan(x), ny = std::isnan(y);
  if (nx || ny) return ny && !nx;
  return x > y;
}

// a before b in one row: the higher score, then the lower id
struct RowOrder {
  const float* s;
  bool operator()(int a, int b) const {
    if (above(s[a], s[b])) return true;
    if (above(s[b], s[a])) return false;
    return a < b;
  }
};

}  // namespace

void lookahead_select(const float* scores, int rows, int n_experts, int top_k, int32_t* out, int max_out,
                      int* n_out) {
  require(scores && out && n_out && rows >= 0 && n_experts > 0 && top_k > 0 && top_k <= n_experts && max_out >= 0,
          SS_E_INVALID, "ss_lookahead_select: bad argument");
  struct Best {
    int rank;
    float score;
  };
  std::vector<Best> best(size_t(n_experts), Best{top_k, 0.0f});  // rank top_k: never selected
  std::vector<int> order(static_cast<size_t>(n_experts));
  for (int r = 0; r < rows; ++r) {
    const RowOrder before{scores + size_t(r) * size_t(n_experts)};
    for (int e = 0; e < n_experts; ++e) order[size_t(e)] = e;
    const auto kth = order.begin() + top_k;
    if (top_k < n_experts) std::nth_element(order.begin(), kth - 1, order.end(), before);
    std::sort(order.begin(), kth, before);
    for (int k = 0; k < top_k; ++k) {
      const int e = order[size_t(k)];
      const float v = before.s[e];
      Best& b = best[size_t(e)];
      if (k < b.rank || (k == b.rank && above(v, b.score))) b = Best{k, v};
    }
  }
  std::vector<int> chosen;
  for (int e = 0; e < n_experts; ++e)
    if (best[size_t(e)].rank < top_k) chosen.push_back(e);
  std::sort(chosen.begin(), chosen.end(), [&](int a, int b) {
    const Best& x = best[size_t(a)];
    const Best& y = best[size_t(b)];
    if (x.rank != y.rank) return x.rank < y.rank;
    if (above(x.score, y.score)) return true;
    if (above(y.score, x.score)) return false;
    return a < b;
  });
  const int n = std::min(int(chosen.size()), max_out);
  std::copy(chosen.begin(), chosen.begin() + n, out);
  *n_out = n;
}

}  // namespace tsa
