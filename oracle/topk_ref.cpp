// Oracle (test infrastructure only): CPU top-k by magnitude in the exact order
// torch.topk returns on CPU for a 1-D float32 input, largest=True, sorted=True.
//
// Follows the reference call site codec.py:533-535 (torch.topk(abs_flat, k)),
// whose CPU kernel keeps a queue of (value, index) pairs in index order and
// selects with libstdc++:
//   * k * 64 <= n : std::partial_sort(q, q + k, q + n, cmp)
//   * otherwise   : std::nth_element(q, q + k - 1, q + n, cmp); std::sort(q, q + k - 1, cmp)
// with cmp(a, b) = (isnan(a.v) && !isnan(b.v)) || a.v > b.v.
// Calling the same library routines reproduces the tie order at the threshold,
// which is not lowest-index-first.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <utility>
#include <vector>

extern "C" int ts_oracle_topk(const float* vals, int64_t n, int64_t k, float* out_vals, int64_t* out_idx) {
  if (n < 0 || k < 0 || k > n) return 1;
  if (k == 0) return 0;
  typedef std::pair<float, int64_t> elem_t;
  std::vector<elem_t> q(n);
  for (int64_t i = 0; i < n; ++i) q[i] = elem_t(vals[i], i);
  auto cmp = [](const elem_t& x, const elem_t& y) -> bool {
    return (std::isnan(x.first) && !std::isnan(y.first)) || (x.first > y.first);
  };
  if (k * 64 <= n) {
    std::partial_sort(q.begin(), q.begin() + k, q.end(), cmp);
  } else {
    std::nth_element(q.begin(), q.begin() + k - 1, q.end(), cmp);
    std::sort(q.begin(), q.begin() + k - 1, cmp);
  }
  for (int64_t i = 0; i < k; ++i) { out_vals[i] = q[i].first; out_idx[i] = q[i].second; }
  return 0;
}

// Sequential float32 accumulation in index order: out[idx[i]] += src[i].
// The reference's Lloyd-Max step uses CPU index_add_ (codec.py:351-352),
// which adds one source at a time in index order.
extern "C" void ts_oracle_index_add_f32(float* out, const int64_t* idx, const float* src, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[idx[i]] += src[i];
}
