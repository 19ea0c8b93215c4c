// CPU oracle for the integer/selection part of the Q38 MoE path. TEST INFRASTRUCTURE ONLY:
// loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the
// product library never links or calls it.
//
// oracle_topk: restatement of torch's CPU top-k loop, ATen/native/TopKImpl.h:45-76 (torch
//   2.10 header installed in this image; the reference pins torch 2.7.1, whose loop is the same):
//   queue[j] = (value_j, j); if k*64 <= n: std::partial_sort(q, q+k, q+n, cmp) else
//   std::nth_element(q, q+k-1, q+n, cmp) then std::sort(q, q+k-1, cmp), with
//   cmp(x, y) = (isnan(x.first) && !isnan(y.first)) || x.first > y.first  (largest = true).
//   The libstdc++ algorithms are the specification, so they are called, not re-implemented.
// oracle_permute: stable counting sort of pair ids, the closed form of
//   torch.sort(ids, stable=True) + searchsorted in q38/inference.py:163-171.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <utility>
#include <vector>

extern "C" {

void oracle_topk(const float* values, int64_t rows, int64_t n, int64_t k, float* out_values,
                 int64_t* out_indices) {
  using elem_t = std::pair<float, int64_t>;
  std::vector<elem_t> queue(n);
  auto cmp = [](const elem_t& x, const elem_t& y) -> bool {
    return (std::isnan(x.first) && !std::isnan(y.first)) || (x.first > y.first);
  };
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = values + r * n;
    for (int64_t j = 0; j < n; ++j) queue[j] = elem_t(v[j], j);
    if (k * 64 <= n) {
      std::partial_sort(queue.begin(), queue.begin() + k, queue.end(), cmp);
    } else {
      std::nth_element(queue.begin(), queue.begin() + k - 1, queue.end(), cmp);
      std::sort(queue.begin(), queue.begin() + k - 1, cmp);
    }
    for (int64_t j = 0; j < k; ++j) {
      out_values[r * k + j] = queue[j].first;
      out_indices[r * k + j] = queue[j].second;
    }
  }
}

// ids [P]; ids outside [0, E) are dropped. counts/starts [E], perm [sum(counts)].
void oracle_permute(const int64_t* ids, int64_t P, int32_t E, int32_t* counts, int32_t* starts,
                    int32_t* perm) {
  std::vector<int64_t> cursor(E, 0);
  for (int32_t e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t p = 0; p < P; ++p)
    if (ids[p] >= 0 && ids[p] < E) counts[ids[p]]++;
  int64_t run = 0;
  for (int32_t e = 0; e < E; ++e) {
    starts[e] = (int32_t)run;
    cursor[e] = run;
    run += counts[e];
  }
  for (int64_t p = 0; p < P; ++p)
    if (ids[p] >= 0 && ids[p] < E) perm[cursor[ids[p]]++] = (int32_t)p;
}

}  // extern "C"
