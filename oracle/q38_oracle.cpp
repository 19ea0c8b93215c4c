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
// oracle_softmax_rows: torch 2.10's CPU softmax over the last dimension in fp32 (the AVX512
//   kernel that torch.softmax(z, dim=-1) dispatches to on this image), restated from its measured
//   behaviour: the row max; e_i = SLEEF's expf_u10 (the published xexpf algorithm, with the fused
//   multiply-adds of its vector form) of x_i - max; the sum in the order of a 16-lane vector
//   reduction (accumulator l adds x_l, x_{l+16}, ... in turn, then lanes fold l^8, l^4, l^2, l^1;
//   rows narrower than 16 sum left to right); p_i = e_i * (1 / sum). tests/test_oracle.py checks
//   it bit for bit against torch.softmax; the router kernel computes its probabilities this way.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <utility>
#include <vector>

namespace {

float sleef_expf_u10(float d) {
  const float qf = std::rint(d * 1.442695040888963407359924681001892137426645954152985934135449406931f);
  const int q = (int)qf;
  float s = std::fma(qf, -0.693145751953125f, d);
  s = std::fma(qf, -1.428606765330187045e-06f, s);
  float u = 0.000198527617612853646278381f;
  u = std::fma(u, s, 0.00139304355252534151077271f);
  u = std::fma(u, s, 0.00833336077630519866943359f);
  u = std::fma(u, s, 0.0416664853692054748535156f);
  u = std::fma(u, s, 0.166666671633720397949219f);
  u = std::fma(u, s, 0.5f);
  const float s2 = s * s;
  u = 1.0f + std::fma(s2, u, s);
  const int q1 = q >> 1, q2 = q - q1;
  uint32_t b1 = (uint32_t)(q1 + 127) << 23, b2 = (uint32_t)(q2 + 127) << 23;
  float f1, f2;
  std::memcpy(&f1, &b1, 4);
  std::memcpy(&f2, &b2, 4);
  u = u * f1;
  u = u * f2;
  if (d < -104.0f) u = 0.0f;
  if (d > 100.0f) u = INFINITY;
  return std::isnan(d) ? d : u;
}

// max propagating NaN, as the vector maximum does
float max_nan(float a, float b) { return (std::isnan(a) || std::isnan(b)) ? NAN : (a > b ? a : b); }

// reduction in the order of a 16-lane vector reduce: accumulators, then folds l^8, l^4, l^2, l^1
template <typename Op>
float reduce16(const float* x, int64_t n, Op op) {
  if (n < 16) {
    float a = x[0];
    for (int64_t i = 1; i < n; ++i) a = op(a, x[i]);
    return a;
  }
  float acc[16];
  for (int l = 0; l < 16; ++l) acc[l] = x[l];
  for (int64_t d = 16; d < n; d += 16)
    for (int l = 0; l < 16 && d + l < n; ++l) acc[l] = op(acc[l], x[d + l]);
  for (int s = 8; s >= 1; s >>= 1) {
    float nxt[16];
    for (int l = 0; l < 16; ++l) nxt[l] = op(acc[l], acc[l ^ s]);
    std::memcpy(acc, nxt, sizeof(acc));
  }
  return acc[0];
}

}  // namespace

extern "C" {

void oracle_softmax_rows(const float* x, int64_t rows, int64_t n, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    float* yr = out + r * n;
    const float m = reduce16(xr, n, max_nan);
    for (int64_t i = 0; i < n; ++i) yr[i] = sleef_expf_u10(xr[i] - m);
    const float s = reduce16(yr, n, [](float a, float b) { return a + b; });
    const float rs = 1.0f / s;
    for (int64_t i = 0; i < n; ++i) yr[i] = yr[i] * rs;
  }
}

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
