// Router (R1-R2): bf16 logits on MFMA, fp32 softmax, top-k with torch-CPU tie semantics,
// renormalisation, shared-expert gate logit and the per-block expert histogram, in one pass.
//
// Reference semantics: Qwen3_8MoeTopKRouter.forward (modeling_qwen3_8_moe.py:805-813) with the
// tie order of torch's CPU topk (ATen/native/TopKImpl.h:45-76):
//   queue[j] = (value_j, j); std::nth_element(q, q+k-1, q+n, cmp); std::sort(q, q+k-1, cmp)
//   cmp(x, y) = (isnan(x) && !isnan(y)) || x > y
// (std::partial_sort when k*64 <= n). The selection here replays libstdc++'s introselect step by
// step, with each Hoare partition evaluated wave-parallel (one lane per queue slot), so indices
// match the CPU library bit for bit. Rows whose k+1 largest values are all distinct have a unique
// answer and take a fast path (k rounds of a group-wide maximum over 8 lanes per token).
//
// Selection compares the fp32 probabilities themselves, computed bit for bit as torch's CPU
// softmax computes them (torch_softmax_* below), so rows whose distinct logits collapse to equal
// probabilities (x - max rounding to one value, or exp / the 1/sum scaling merging neighbours) tie
// exactly where the CPU's do.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int KMAX = 8;

// ---- torch 2.10 CPU softmax over a row of fp32 values (the AVX512 kernel torch dispatches to),
// restated operation by operation; verified bit for bit against torch.softmax on the CPU over
// millions of rows of widths 1..64, wide ranges, +-inf and NaN (tests/test_oracle.py restates it
// in C and checks it there):
//   m = max(x); e_i = expf_u10(x_i - m); s = sum of e_i in the order of a 16-lane vector
//   reduction (lane l accumulates e_l, e_{l+16}, e_{l+32}, e_{l+48} in turn, then the lanes are
//   folded l ^ 8, l ^ 4, l ^ 2, l ^ 1; rows narrower than 16 sum left to right); p_i = e_i * (1/s).
// expf_u10 is SLEEF's single-precision u10 exponential (the published xexpf algorithm: round
// x/ln2 to an integer q, two-part Cody-Waite reduction, degree-6 polynomial, scale by 2^q in two
// halves; 0 below -104, inf above 100), fused multiply-adds where SLEEF's vector form uses them.
__device__ __forceinline__ float torch_cpu_expf(float d) {
#pragma clang fp contract(off)
  const float qf = __builtin_rintf(d * 1.442695040888963407359924681001892137426645954152985934135449406931f);
  const int q = (int)qf;
  float s = __builtin_fmaf(qf, -0.693145751953125f, d);
  s = __builtin_fmaf(qf, -1.428606765330187045e-06f, s);
  float u = 0.000198527617612853646278381f;
  u = __builtin_fmaf(u, s, 0.00139304355252534151077271f);
  u = __builtin_fmaf(u, s, 0.00833336077630519866943359f);
  u = __builtin_fmaf(u, s, 0.0416664853692054748535156f);
  u = __builtin_fmaf(u, s, 0.166666671633720397949219f);
  u = __builtin_fmaf(u, s, 0.5f);
  const float s2 = s * s;
  u = 1.0f + __builtin_fmaf(s2, u, s);
  const int q1 = q >> 1, q2 = q - q1;
  u = u * __int_as_float((q1 + 127) << 23);
  u = u * __int_as_float((q2 + 127) << 23);
  u = d < -104.0f ? 0.0f : u;
  u = d > 100.0f ? __builtin_inff() : u;
  return __builtin_isnan(d) ? d : u;
}

// torch's CPU sum over the last dimension of a contiguous [rows, k] fp32 tensor (the top-k
// renormalisation, modeling:810), as measured bit for bit against torch.sum on the CPU: k in 5..7
// take the 4-way interleaved row sum ((v0 + v4 [+ v5 [+ v6]]) + v1 + v2 + v3, left to right);
// every other k <= 8 sums left to right.
template <int K>
__device__ __forceinline__ float torch_topk_sum(const float* v) {
  float t;
  if constexpr (K >= 5 && K <= 7) {
    t = v[0] + v[4];
#pragma unroll
    for (int r = 5; r < K; ++r) t = t + v[r];
    t = t + v[1];
    t = t + v[2];
    t = t + v[3];
  } else {
    t = v[0];
#pragma unroll
    for (int r = 1; r < K; ++r) t = t + v[r];
  }
  return t;
}

// The selection's comparator (torch's topk on the CPU: NaN above every number). NANS = false is the
// same order for rows without NaN, whose probabilities are all numbers (finite, or -inf in the
// unused slots past E): the replay of such rows, nearly all of them, skips the NaN tests.
template <bool NANS = true>
__device__ __forceinline__ bool cmp_gt(float a, float b) {
  if constexpr (NANS) return (__builtin_isnan(a) && !__builtin_isnan(b)) || (a > b);
  else return a > b;
}

// Whole-wave reductions without LDS traffic: DPP within rows of 16 lanes (xor 1, xor 2, half-row
// and row mirrors), then the gfx950 row-pair and half-wave swaps.
__device__ __forceinline__ float dpp_f(float v, int ctrl) {
  switch (ctrl) {  // ctrl must be an immediate
    case 0xb1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));
    case 0x4e: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));
    case 0x141: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
  }
}
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_f(v, 0xb1));   // quad_perm [1,0,3,2]: lane ^ 1
  v = op(v, dpp_f(v, 0x4e));   // quad_perm [2,3,0,1]: lane ^ 2
  v = op(v, dpp_f(v, 0x141));  // row_half_mirror: quads of each 8 lanes
  v = op(v, dpp_f(v, 0x140));  // row_mirror: halves of each row of 16
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  v = op(__int_as_float(r16[0]), __int_as_float(r16[1]));  // rows 0|1 and 2|3
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return op(__int_as_float(r32[0]), __int_as_float(r32[1]));  // lanes 0-31 | 32-63
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    uint32_t lo = __shfl_xor((unsigned)(uint32_t)k, o);
    uint32_t hi = __shfl_xor((unsigned)(uint32_t)(k >> 32), o);
    uint64_t other = ((uint64_t)hi << 32) | lo;
    k = other > k ? other : k;
  }
  return k;
}

// Wave-uniform broadcast of lane `src`'s value (v_readlane; src must be wave-uniform).
__device__ __forceinline__ float lane_f(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ int lane_i(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// Number of set bits of m below the calling lane (v_mbcnt).
__device__ __forceinline__ int bits_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Swap queue slots a and b (wave-uniform).
__device__ __forceinline__ void swap_slots(float& qv, int& qi, int lane, int a, int b) {
  const float va = lane_f(qv, a), vb = lane_f(qv, b);
  const int ia = lane_i(qi, a), ib = lane_i(qi, b);
  if (lane == a) {
    qv = vb;
    qi = ib;
  } else if (lane == b) {
    qv = va;
    qi = ia;
  }
}

// libstdc++ __insertion_sort (a stable insertion sort) of slots [lo, hi), hi - lo <= KMAX. Under
// the strict weak order cmp_gt its result is the stable descending sort, so the element in slot p
// moves to lo + (the number of slots in [lo, hi) holding a cmp-greater value, plus those before p
// holding an equivalent one). Every lane computes that rank against the n values (read as
// scalars) and one forward permute places the elements; lanes outside [lo, hi) keep theirs.
template <bool NANS>
__device__ void insertion_sort_slots(float& qv, int& qi, int lane, int lo, int hi) {
  const int n = hi - lo;
  if (n <= 1) return;
  int rank = 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < n) {  // wave-uniform
      const float vj = lane_f(qv, lo + j);
      const bool gt = cmp_gt<NANS>(vj, qv);
      const bool equiv = !gt && !cmp_gt<NANS>(qv, vj);
      rank += (gt || (equiv && lo + j < lane)) ? 1 : 0;
    }
  }
  const int dst = (lane >= lo && lane < hi) ? lo + rank : lane;
  qv = __int_as_float(__builtin_amdgcn_ds_permute(dst << 2, __float_as_int(qv)));
  qi = __builtin_amdgcn_ds_permute(dst << 2, qi);
}

// libstdc++ __adjust_heap + __push_heap on LDS arrays based at `first` (single lane).
template <bool NANS>
__device__ void heap_adjust(float* v, int* id, int first, int hole, int len, float val, int vid) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (cmp_gt<NANS>(v[first + second], v[first + second - 1])) second--;
    v[first + hole] = v[first + second];
    id[first + hole] = id[first + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    v[first + hole] = v[first + second - 1];
    id[first + hole] = id[first + second - 1];
    hole = second - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && cmp_gt<NANS>(v[first + parent], val)) {
    v[first + hole] = v[first + parent];
    id[first + hole] = id[first + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  v[first + hole] = val;
  id[first + hole] = vid;
}

// libstdc++ __heap_select(first, middle, last) followed by iter_swap(first, nth): the
// depth-limit exit of __introselect. Runs on one lane over an LDS copy of the queue.
template <bool NANS>
__device__ void heap_select_slots(float& qv, int& qi, int lane, int first, int middle, int last,
                                  int nth, float* sv, int* si) {
  sv[lane] = qv;
  si[lane] = qi;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane == 0) {
    const int len = middle - first;
    if (len >= 2) {
      int parent = (len - 2) / 2;
      while (true) {
        heap_adjust<NANS>(sv, si, first, parent, len, sv[first + parent], si[first + parent]);
        if (parent == 0) break;
        parent--;
      }
    }
    for (int i = middle; i < last; ++i) {
      if (cmp_gt<NANS>(sv[i], sv[first])) {
        const float val = sv[i];
        const int vid = si[i];
        sv[i] = sv[first];
        si[i] = si[first];
        heap_adjust<NANS>(sv, si, first, 0, len, val, vid);
      }
    }
    const float tv = sv[first];
    const int ti = si[first];
    sv[first] = sv[nth];
    si[first] = si[nth];
    sv[nth] = tv;
    si[nth] = ti;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  qv = sv[lane];
  qi = si[lane];
}

// std::nth_element(q, q+k-1, q+n, cmp) then std::sort(q, q+k-1, cmp), with queue slot = lane.
template <bool NANS>
__device__ void nth_element_then_sort(float& qv, int& qi, int lane, int n, int k, float* sv,
                                      int* si) {
  const int nth = k - 1;
  int first = 0, last = n;
  int depth = 2 * (31 - __clz(n));
  bool sorted_tail = true;
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_slots<NANS>(qv, qi, lane, first, nth + 1, last, nth, sv, si);
      sorted_tail = false;
      break;
    }
    --depth;
    // __unguarded_partition_pivot: median of (first+1, mid, last-1) moved to first.
    const int mid = first + (last - first) / 2;
    const float a = lane_f(qv, first + 1), b = lane_f(qv, mid), c = lane_f(qv, last - 1);
    int s;
    if (cmp_gt<NANS>(a, b)) {
      if (cmp_gt<NANS>(b, c)) s = mid;
      else if (cmp_gt<NANS>(a, c)) s = last - 1;
      else s = first + 1;
    } else if (cmp_gt<NANS>(a, c)) {
      s = first + 1;
    } else if (cmp_gt<NANS>(b, c)) {
      s = last - 1;
    } else {
      s = mid;
    }
    swap_slots(qv, qi, lane, first, s);
    const float pv = lane_f(qv, first);
    // __unguarded_partition(first+1, last, pivot=first): the i-th left stop (slot holding a value
    // not cmp-greater than the pivot) swaps with the i-th right stop (value the pivot is not
    // cmp-greater than; the pivot slot itself guards the scan) while left < right. Lane i learns
    // li = the i-th left stop and ri = the i-th right stop counted from the right by a forward
    // permute (each stop sends its position to the lane of its rank; lane 63 is never a rank a
    // left stop or a partial right-stop set reaches, so the other lanes send there).
    const bool isl = lane > first && lane < last && !cmp_gt<NANS>(qv, pv);
    const bool isg = lane >= first && lane < last && !cmp_gt<NANS>(pv, qv);
    const uint64_t le = ballot64(isl);
    const uint64_t ge = ballot64(isg);
    const int nl = __popcll(le), nr = __popcll(ge);
    const int lrank = bits_below(le);
    const int grank = nr - 1 - bits_below(ge);
    const int lp = __builtin_amdgcn_ds_permute((isl ? lrank : 63) << 2, lane);
    const int rp = __builtin_amdgcn_ds_permute((isg ? grank : 63) << 2, lane);
    const int li = lane < nl ? lp : 64;
    const int ri = lane < nr ? rp : -1;
    const int sw = __popcll(ballot64(lane < nl && lane < nr && li < ri));
    int cut;
    if (sw == 0) {
      cut = lane_i(li, 0);
    } else {
      const int l_next = sw < nl ? lane_i(li, sw) : (1 << 20);
      const int r_last = lane_i(ri, sw - 1);
      cut = min(l_next, r_last);
    }
    // The i-th left stop takes the i-th right stop's slot and vice versa, for i < sw.
    const int from_r = __builtin_amdgcn_ds_bpermute((isl ? lrank : lane) << 2, ri);
    const int from_l = __builtin_amdgcn_ds_bpermute((isg ? grank : lane) << 2, li);
    int src = lane;
    if (isl && lrank < sw) src = from_r;
    else if (isg && grank < sw) src = from_l;
    qv = __int_as_float(__builtin_amdgcn_ds_bpermute((src & 63) << 2, __float_as_int(qv)));
    qi = __builtin_amdgcn_ds_bpermute((src & 63) << 2, qi);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  if (sorted_tail) insertion_sort_slots<NANS>(qv, qi, lane, first, last);
  // std::sort on k-1 <= 16 elements is __insertion_sort.
  insertion_sort_slots<NANS>(qv, qi, lane, 0, k - 1);
}

// Selection and renormalisation for one token held by the calling wave, from its fp32
// probabilities: p of expert `lane` (lanes >= E ignored); all_nan when the row's softmax is NaN
// everywhere. The selection replays libstdc++ on them. Lane r < K receives the r-th selected expert
// and its renormalised weight.
template <int K>
__device__ void select_token(float p, bool all_nan, int lane, int E, int& out_idx, float& out_w, float* sv,
                             int* si) {
  const bool valid = lane < E;
  float qv = valid ? p : -INFINITY;
  int qi = lane;

  if (K * 64 <= E) {
    // std::partial_sort path (K == 1, E == 64): first slot whose value is cmp-greater than all
    // before it = lowest-index maximum (slot 0 when every value is NaN).
    int best = 0;
    if (!all_nan) {
      const uint64_t key = valid ? ((uint64_t)order_key(qv) << 32) | (uint32_t)(63 - lane) : 0ull;
      best = 63 - (int)(uint32_t)wave_max_u64(key);
    }
    qi = best;
  } else if (all_nan) {
    nth_element_then_sort<true>(qv, qi, lane, E, K, sv, si);
  } else {
    nth_element_then_sort<false>(qv, qi, lane, E, K, sv, si);
  }
  // Renormalise over the selected probabilities with torch's row-sum order, then divide.
  const float pr = __shfl(p, qi & 63);
  float v[K];
#pragma unroll
  for (int r = 0; r < K; ++r) v[r] = lane_f(pr, r);
  out_idx = qi;
  out_w = pr / torch_topk_sum<K>(v);
}

// Route one token held by the calling wave. z: selection input of expert `lane` (bf16 logit plus
// the optional bias; lanes >= E ignored). The fp32 probabilities follow torch's CPU softmax bit
// for bit; then select_token.
template <int K>
__device__ void route_token(float z, int lane, int E, int& out_idx, float& out_w, float* sv, int* si) {
  const bool valid = lane < E;
  z = z + 0.0f;  // -0 -> +0 (the CPU adds the bias or a zero the same way; exp(+-0) is 1 either way)
  const bool has_nan = ballot64(valid && __builtin_isnan(z)) != 0ull;
  const float m = wave_max(valid ? z : -INFINITY);
  const bool all_nan = has_nan || !__builtin_isfinite(m);  // softmax is NaN everywhere then
  float p;
  if (all_nan) {
    p = __builtin_nanf("");
  } else {
    const float ex = valid ? torch_cpu_expf(z - m) : 0.0f;
    float sum;
    if (E >= 16) {
      // Lane l < 16 accumulates experts l, l+16, l+32, l+48 (absent ones add +0, exactly), then
      // the 16 partial sums fold l ^ 8, l ^ 4, l ^ 2, l ^ 1.
      float acc = ex;
      acc = acc + __shfl(ex, (lane + 16) & 63);
      acc = acc + __shfl(ex, (lane + 32) & 63);
      acc = acc + __shfl(ex, (lane + 48) & 63);
      acc = acc + __shfl_xor(acc, 8);
      acc = acc + __shfl_xor(acc, 4);
      acc = acc + __shfl_xor(acc, 2);
      acc = acc + __shfl_xor(acc, 1);
      sum = lane_f(acc, 0);
    } else {
      sum = lane_f(ex, 0);
      for (int e = 1; e < E; ++e) sum = sum + lane_f(ex, e);
    }
    p = ex * (1.0f / sum);
  }
  select_token<K>(p, all_nan, lane, E, out_idx, out_w, sv, si);
}

constexpr int ROUTE_TOKENS = 64;   // tokens per histogram row (and per block, unless TOK = 128)
constexpr int ROUTE_KCHUNK = 1024; // router-weight K columns staged in LDS at a time
constexpr int ROUTE_WROWS = 65;    // 64 expert rows + the shared-expert gate row

// Router weight chunk in LDS: row n (expert, or 64 = shared gate), 16-byte chunk c of the
// current K chunk stored at slot c ^ (n & 15): the 16 rows of a B fragment read distinct banks.
__device__ __forceinline__ int wr_slot(int n, int c) { return n * (ROUTE_KCHUNK / 8) + (c ^ (n & 15)); }

constexpr int SEL_LANES = 8;  // lanes per token in the selection fast path
// Outcomes of group_select: selected; tie (the row's probabilities are left in LDS for the
// replay); NaN or a non-finite maximum (the replay starts from the logits).
enum { SEL_DONE = 0, SEL_REPLAY_PROBS = 1, SEL_REPLAY_LOGITS = 2 };

// Value of lane (lane ^ O) for O in {1, 2, 4}, by DPP (no LDS round trip): quad permutes for 1 and
// 2; for 4, the half-row mirror (lane i of each 8 takes 7 - i) followed by the quad reverse (i takes
// 3 - i within its quad), whose composition is i -> i ^ 4.
template <int O>
__device__ __forceinline__ int xor_lanes(int v) {
  static_assert(O == 1 || O == 2 || O == 4, "xor_lanes: O in {1, 2, 4}");
  if constexpr (O == 1) return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);
  else if constexpr (O == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);
  else return __builtin_amdgcn_update_dpp(0, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false), 0x1b, 0xf, 0xf, false);
}
template <int O>
__device__ __forceinline__ float xor_lanes_f(float v) { return __int_as_float(xor_lanes<O>(__float_as_int(v))); }


// Per-token selection by a group of SEL_LANES lanes (lane s of the group holds experts s,
// s + SEL_LANES, ...). The group computes the row's fp32 probabilities as torch's CPU softmax does
// (the 16 partial sums of its vector reduction are lanes s and s + 8 of the two interleaved
// halves of each lane's experts, folded l ^ 8 locally, then across lanes ^ 4, ^ 2, ^ 1). Then k
// rounds of a group-wide maximum: each round takes the largest remaining probability (a local max
// over the lane's 8, then three lane exchanges), counts how often it occurs in the row and removes
// every occurrence. A count above one among the first k rounds means the k+1 largest values are
// not all distinct. Returns SEL_DONE with the k largest in descending order when they are; else
// (or when the row has a NaN / non-finite max, or fewer than k experts) the token needs the
// libstdc++ replay. Every lane of the group returns the same answer.
template <int KP1>
__device__ __forceinline__ int group_select(float* row, const float* bias, int E, int s,
                                            int* out_idx, float* out_w) {
  constexpr int K = KP1 - 1;
  constexpr int PER = 64 / SEL_LANES;  // 8 values per lane
  static_assert(SEL_LANES == 8, "the reductions below are for 8 lanes per token");
  float z[PER];
  int nan = 0;
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = s + SEL_LANES * j;
    z[j] = -INFINITY;
    if (e < E) {
      z[j] = row[e] + (bias != nullptr ? bias[e] : 0.0f) + 0.0f;
      nan |= __builtin_isnan(z[j]);
      mx = fmaxf(mx, z[j]);
    }
  }
  mx = fmaxf(mx, xor_lanes_f<1>(mx));
  mx = fmaxf(mx, xor_lanes_f<2>(mx));
  mx = fmaxf(mx, xor_lanes_f<4>(mx));
  nan |= xor_lanes<1>(nan);
  nan |= xor_lanes<2>(nan);
  nan |= xor_lanes<4>(nan);
  if (nan || !__builtin_isfinite(mx)) return SEL_REPLAY_LOGITS;
  float ex[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) ex[j] = s + SEL_LANES * j < E ? torch_cpu_expf(z[j] - mx) : 0.0f;
  float sum;
  if (E >= 16) {
    float a = ex[0], b = ex[1];
#pragma unroll
    for (int j = 2; j < PER; j += 2) {
      a = a + ex[j];
      b = b + ex[j + 1];
    }
    sum = a + b;
    sum = sum + xor_lanes_f<4>(sum);
    sum = sum + xor_lanes_f<2>(sum);
    sum = sum + xor_lanes_f<1>(sum);
  } else {
    // Rows narrower than one vector: left to right over the experts.
    sum = 0.0f;
    for (int e = 0; e < E; ++e) {
      const float ee = torch_cpu_expf(row[e] + (bias != nullptr ? bias[e] : 0.0f) + 0.0f - mx);
      sum = e == 0 ? ee : sum + ee;
    }
  }
  const float rs = 1.0f / sum;
  float lv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) lv[j] = s + SEL_LANES * j < E ? ex[j] * rs : -INFINITY;
  const int lim = min(K, E - 1);
  bool tie = false;
  float v[K];
  int id[K];
#pragma unroll
  for (int r = 0; r < K; ++r) {
    float m = lv[0];
#pragma unroll
    for (int j = 1; j < PER; ++j) m = fmaxf(m, lv[j]);
    m = fmaxf(m, xor_lanes_f<1>(m));
    m = fmaxf(m, xor_lanes_f<2>(m));
    m = fmaxf(m, xor_lanes_f<4>(m));
    int c = 0, ix = 64;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const bool eq = lv[j] == m;
      c += eq ? 1 : 0;
      ix = eq ? min(ix, s + SEL_LANES * j) : ix;
      lv[j] = eq ? -INFINITY : lv[j];
    }
    c += xor_lanes<1>(c);
    c += xor_lanes<2>(c);
    c += xor_lanes<4>(c);
    ix = min(ix, xor_lanes<1>(ix));
    ix = min(ix, xor_lanes<2>(ix));
    ix = min(ix, xor_lanes<4>(ix));
    if (r < lim && c > 1) tie = true;            // v[r] == v[r + 1]
    if (r == K - 1 && m == -INFINITY) tie = true;  // fewer than k experts: replay
    v[r] = m;
    id[r] = ix;
  }
  if (tie) {
    // The replay starts from these probabilities: they replace the row's logits in LDS (the
    // logits output, when requested, has read them all before the selection starts).
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (s + SEL_LANES * j < E) row[s + SEL_LANES * j] = ex[j] * rs;
    return SEL_REPLAY_PROBS;
  }
  const float tot = torch_topk_sum<K>(v);
#pragma unroll
  for (int r = 0; r < K; ++r) {
    out_idx[r] = id[r];
    out_w[r] = v[r] / tot;
  }
  return SEL_DONE;
}


// One block = TOK tokens (64, or 128 when a launch would need more than one round of 64-token
// blocks), 16 waves. Phase 1: logits on 16x16x32 MFMA, router weights (+ the shared-expert gate row
// as column 64) staged in LDS per 1024-wide K chunk by all waves; every wave multiplies one
// 16-token group over one K part of the chunk (4 parts with 64 tokens, 2 with 128), its x rows
// loaded straight into registers with the whole part in flight, and the parts' partial sums are
// added in K-part order through LDS. Phase 2: bf16-rounded logits to LDS.
// Phase 3: eight lanes per token select top-k (unique answer when the k+1 largest values are
// distinct). Phase 4: tokens with ties are replayed wave-parallel through libstdc++'s algorithm,
// one per wave: sixteen at a time.
constexpr int ROUTE_THREADS = 1024;  // 16 waves: all multiply (K split), select and replay ties

// KT = k (1..KMAX) as a template parameter: each instantiation carries only its own selection
// network, which keeps the kernel's code within the instruction cache.
// F32IO: the fp32 path (fp32 models): logits come in as fp32 (logits_in, computed by the fp32
// router GEMM) and the renormalised weights leave as fp32 (no bf16 rounding, modeling:812 with
// the fp32 logits dtype); x is unused.
// SPLITK (T <= 16, one 64-token block; bf16, logits computed here): phase 1 is a split-K product
// instead of the staged one, see below.
template <int KT, bool F32IO, int TOK = ROUTE_TOKENS, bool SPLITK = false>
__global__ __launch_bounds__(ROUTE_THREADS) void route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const uint16_t* __restrict__ wsg, const void* __restrict__ logits_in,
    const float* __restrict__ bias, uint16_t* __restrict__ logits_out,
    int32_t* __restrict__ idx_out, void* __restrict__ w_out,
    uint16_t* __restrict__ gate_out, int32_t* __restrict__ hist, int64_t T, int h, int E, int k) {
  static_assert(TOK == 64 || TOK == 128, "64 or 128 tokens per block");
  static_assert(!SPLITK || (TOK == 64 && !F32IO), "split-K logits: one 64-token block, bf16");
  // Staged router weights (phase 1) and logits (from phase 2 on). With 128 tokens both do not fit
  // side by side: they share one LDS area, and the logits are written once every wave has finished
  // its MFMAs.
  // Logit row stride 72 (= 8 mod 64 banks): the selection's 8 lanes x 8 tokens per wave read 64
  // distinct banks.
  constexpr bool ALIAS = TOK > 64;
  constexpr int W_BYTES = ROUTE_WROWS * (ROUTE_KCHUNK / 8) * 16, L_BYTES = TOK * 72 * 4;
  __shared__ __attribute__((aligned(16)))
  uint8_t s_wl[ALIAS ? (W_BYTES > L_BYTES ? W_BYTES : L_BYTES) : W_BYTES + L_BYTES];
  u32x4_t* const s_w = reinterpret_cast<u32x4_t*>(s_wl);
  float (*const s_logit)[72] = reinterpret_cast<float (*)[72]>(s_wl + (ALIAS ? 0 : W_BYTES));
  __shared__ float s_bias[64];
  __shared__ int s_hist[TOK / 64][64];  // per 64-token histogram row
  __shared__ int s_ties[TOK];
  __shared__ int s_nties;
  __shared__ float s_sv[ROUTE_THREADS / 64][64];
  __shared__ int s_si[ROUTE_THREADS / 64][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // the same, as a scalar
  const int64_t tb = (int64_t)blockIdx.x * TOK;
  if (tid < TOK) s_hist[tid >> 6][tid & 63] = 0;
  if (tid < 64) s_bias[tid] = (bias != nullptr && tid < E) ? bias[tid] : 0.0f;
  if (tid == 0) s_nties = 0;

  if constexpr (SPLITK) {
    // At most 16 tokens (decode, short chunks): staging the 133 KB of router weights in LDS for one
    // 16-token MFMA wave would serialise the copy and the multiply in one workgroup. Instead every
    // wave multiplies the 16 token rows by all 64 + 1 weight rows over its eighth of K, both operands
    // loaded from global memory straight into MFMA registers (all its loads in flight at once),
    // and the eight partial sums are added in wave order through LDS, then rounded to bf16 as the
    // staged product's logits are. Same products, another fp32 summation order.
    const int kw = h / (ROUTE_THREADS / 64);  // multiple of 32 (h % 512 == 0)
    const int64_t trow = (lane & 15) < T ? (lane & 15) : T - 1;
    const uint16_t* const xa = x + trow * (int64_t)h + 8 * (lane >> 4);
    const uint16_t* wrow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 16 * j + (lane & 15);
      wrow[j] = wr + (int64_t)(n < E ? n : 0) * h + 8 * (lane >> 4);
    }
    const uint16_t* const grow = wsg != nullptr ? wsg + 8 * (lane >> 4) : nullptr;
    f32x4_t acc[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int kbeg = wave_u * kw;
#pragma unroll 4
    for (int kk = 0; kk < kw; kk += 32) {
      const int kq = kbeg + kk;
      const u32x4_t a = ld16(xa + kq);
      u32x4_t b[5];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = ld16(wrow[j] + kq);
      b[4] = grow != nullptr ? ld16(grow + kq) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 5; ++j) acc[j] = mfma16x16x32(a, b[j], acc[j]);
    }
    f32x4_t* const part = reinterpret_cast<f32x4_t*>(s_wl);  // [wave][tile][lane], 40 KB
#pragma unroll
    for (int j = 0; j < 5; ++j) part[(wave * 5 + j) * 64 + lane] = acc[j];
    __syncthreads();
    if (tid < 5 * 64) {
      const int j = tid >> 6, l = tid & 63;
      f32x4_t sum = part[j * 64 + l];
      for (int w = 1; w < ROUTE_THREADS / 64; ++w) sum += part[(w * 5 + j) * 64 + l];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 4 * (l >> 4) + i, col = 16 * j + (l & 15);
        if (j < 4) {
          if (col < E) s_logit[tok][col] = round_bf16(sum[i]);
        } else if ((l & 15) == 0 && wsg != nullptr) {
          s_logit[tok][64] = round_bf16(sum[i]);
        }
      }
    }
  } else if (!F32IO && logits_in == nullptr) {
    const int ntile = (E + 15) >> 4;
    const bool gate_tile = wsg != nullptr;
    const int nrows_w = gate_tile ? ROUTE_WROWS : 64;
    f32x4_t acc[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Every wave multiplies: token group g (16 tokens) over K part kp of each chunk (SPW of its 32
    // steps); the NKP partial sums of a token group are added in K-part order below.
    constexpr int G = TOK / 16, NKP = (ROUTE_THREADS / 64) / G, SPW = 32 / NKP;
    const int g = wave & (G - 1), kp = wave / G;
    const int64_t trow = tb + g * 16 + (lane & 15);
    const uint16_t* xa = x + (trow < T ? trow : T - 1) * (int64_t)h + 8 * (lane >> 4);
    // Tiles of experts >= E (and the gate tile without wsg) multiply LDS rows that are never
    // filled; their columns are never stored. Computing them keeps the MFMA loop branch-free.
    for (int k0 = 0; k0 < h; k0 += ROUTE_KCHUNK) {
      const int kc = min(ROUTE_KCHUNK, h - k0);  // multiple of 64
      __syncthreads();                            // previous chunk fully consumed
      const bool full = kc == ROUTE_KCHUNK;
      // Router weights -> LDS in 1 KiB row segments: segment q = (row n, half part) fills slots
      // n * 128 + part * 64 + lane, lane l holding the 16-byte chunk the swizzle puts in slot l. A
      // chunk narrower than 512 columns leaves slots past kc/8 unused; their lanes copy chunk 0.
      // Each block starts at a different segment so that the blocks, which all copy the same
      // weights at once, spread over the L2 channels.
      const int halves = (kc + 511) / 512;        // 1 KiB row segments in this chunk: 1 or 2
      const int nseg = nrows_w * halves;
      const int seg0 = (int)((blockIdx.x * 37u) % (unsigned)nseg);
      auto seg_src = [&](int q, int& slot) -> const uint16_t* {
        int qq = q + seg0;
        qq = qq >= nseg ? qq - nseg : qq;
        const int n = halves == 2 ? qq >> 1 : qq, part = halves == 2 ? qq & 1 : 0;
        const uint16_t* src = n < 64 ? (n < E ? wr + (int64_t)n * h : nullptr) : wsg;
        const int c = (part * 64 + lane) ^ (n & 15);
        slot = n * (ROUTE_KCHUNK / 8) + part * 64 + lane;
        return src == nullptr ? nullptr : src + k0 + (c < kc / 8 ? c : 0) * 8;
      };
      u32x4_t a[SPW];  // this wave's x rows over its K part of a full chunk
      if constexpr (!ALIAS) {
        // 64-token blocks: the x loads go first; then every wave copies weight segments
        // (asynchronous copies; spread over every wave they arrive sooner). The multiply starts
        // once both are in.
        if (full) {
#pragma unroll
          for (int s = 0; s < SPW; ++s) a[s] = ld16(xa + k0 + (kp * SPW + s) * 32);
        }
        for (int q = wave_u; q < nseg; q += ROUTE_THREADS / 64) {
          int slot;
          const uint16_t* src = seg_src(q, slot);
          if (src != nullptr) load_lds16(src, &s_w[slot - lane]);
        }
        wait_vmcnt0();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        // 128-token blocks: every wave multiplies and copies weight segments asynchronously, issued
        // before its x loads so that they are not queued behind them.
        for (int q = wave_u; q < nseg; q += ROUTE_THREADS / 64) {
          int slot;
          const uint16_t* src = seg_src(q, slot);
          if (src != nullptr) load_lds16(src, &s_w[slot - lane]);
        }
        if (full) {
#pragma unroll
          for (int s = 0; s < SPW; ++s) a[s] = ld16(xa + k0 + (kp * SPW + s) * 32);
        }
        wait_vmcnt0();
        __syncthreads();
      }
      if (full) {
        // Weight fragments of step s + 1 are read from LDS while step s multiplies. Fragment (j, s)
        // of this lane is wr_slot(16 j + lr, 4 s + lq): with s = 4 m + r its byte offset is
        // 32768 j + 256 m + (2048 lr + 64 (r ^ (lr >> 2)) + 16 (lq ^ (lr & 3))), so four per-lane
        // bases and immediate offsets cover all 32 steps (the gate row 64 is the same in every
        // lane: 131072 + 64 s + 16 lq).
        const uint8_t* const sb = reinterpret_cast<const uint8_t*>(s_w);
        const uint32_t lr = lane & 15, lq = lane >> 4;
        // (The empty asm keeps each base in one register: folded into the constants, every step's
        // address would be a register of its own.)
        // This wave's steps start at kp * SPW (a multiple of 4): its part's offset joins the bases.
        const uint8_t* fb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          uint32_t off = 2048u * lr + 64u * ((uint32_t)r ^ (lr >> 2)) + 16u * (lq ^ (lr & 3u)) +
                         64u * (uint32_t)(kp * SPW);
          asm volatile("" : "+v"(off));
          fb[r] = sb + off;
        }
        uint32_t goff = (uint32_t)wr_slot(64, 0) * 16u + 16u * lq + 64u * (uint32_t)(kp * SPW);
        asm volatile("" : "+v"(goff));
        const uint8_t* const gb = sb + goff;
        // Fragment reads one step ahead (two buffers); with 128-token blocks a wave's 16 steps of x
        // already take 64 registers, so its reads run in the step itself.
        constexpr int NB = SPW > 8 ? 1 : 2;
        u32x4_t bf[NB][5];
        auto bload = [&](int s, u32x4_t(&d)[5]) {
#pragma unroll
          for (int j = 0; j < 4; ++j) d[j] = *reinterpret_cast<const u32x4_t*>(fb[s & 3] + (32768 * j + 256 * (s >> 2)));
          d[4] = *reinterpret_cast<const u32x4_t*>(gb + 64 * s);
        };
        if constexpr (NB == 2) bload(0, bf[0]);
#pragma unroll
        for (int s = 0; s < SPW; ++s) {
          if constexpr (NB == 2) {
            if (s + 1 < SPW) bload(s + 1, bf[(s + 1) & 1]);
          } else {
            bload(s, bf[0]);
          }
          __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of this step's MFMAs
#pragma unroll
          for (int j = 0; j < 5; ++j) acc[j] = mfma16x16x32(a[s], bf[NB == 2 ? (s & 1) : 0][j], acc[j]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        // Narrow last chunk (h not a multiple of the chunk): one 32-wide slice at a time, slice s
        // to K part s % NKP.
        for (int s = kp; s < kc / 32; s += NKP) {
          const u32x4_t as = ld16(xa + k0 + s * 32);
          const int c = 4 * s + (lane >> 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = mfma16x16x32(as, s_w[wr_slot(16 * j + (lane & 15), c)], acc[j]);
          acc[4] = mfma16x16x32(as, s_w[wr_slot(64, c)], acc[4]);
        }
      }
    }
    // Partial sums through the staged-weight area (every wave's MFMAs have read it), added in K-part
    // order; with 128-token blocks the logits share that area, so the sums are formed in registers
    // before any logit is written.
    __syncthreads();
    f32x4_t* const part = reinterpret_cast<f32x4_t*>(s_wl);  // [wave][tile][lane]
#pragma unroll
    for (int j = 0; j < 5; ++j) part[(wave * 5 + j) * 64 + lane] = acc[j];
    __syncthreads();
    constexpr int NENT = G * 5 * 64, NPT = (NENT + ROUTE_THREADS - 1) / ROUTE_THREADS;
    f32x4_t sum[NPT];
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int e_ = tid + u * ROUTE_THREADS;
      if (e_ < NENT) {
        const int gg = e_ / 320, j = (e_ / 64) % 5, l = e_ & 63;
        sum[u] = part[(gg * 5 + j) * 64 + l];
#pragma unroll
        for (int q = 1; q < NKP; ++q) sum[u] += part[((q * G + gg) * 5 + j) * 64 + l];
      }
    }
    if (ALIAS) __syncthreads();
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int e_ = tid + u * ROUTE_THREADS;
      if (e_ < NENT) {
        const int gg = e_ / 320, j = (e_ / 64) % 5, l = e_ & 63;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = gg * 16 + 4 * (l >> 4) + i, col = 16 * j + (l & 15);
          if (j < 4) {
            if (j < ntile && col < E) s_logit[tok][col] = round_bf16(sum[u][i]);
          } else if (gate_tile && (l & 15) == 0) {
            s_logit[tok][64] = round_bf16(sum[u][i]);
          }
        }
      }
    }
  } else {
    for (int i = tid; i < TOK * E; i += ROUTE_THREADS) {
      const int tl = i / E, e = i - tl * E;
      const int64_t t = tb + tl;
      if (F32IO)
        s_logit[tl][e] = t < T ? static_cast<const float*>(logits_in)[t * E + e] : 0.0f;
      else
        s_logit[tl][e] = t < T ? bf16_to_f32(static_cast<const uint16_t*>(logits_in)[t * E + e]) : 0.0f;
    }
  }
  __syncthreads();

  if (logits_out != nullptr && logits_in == nullptr) {
    for (int i = tid; i < TOK * E; i += ROUTE_THREADS) {
      const int tl = i / E, e = i - tl * E;
      const int64_t t = tb + tl;
      if (t < T) logits_out[t * E + e] = (uint16_t)f32_to_bf16_rne(s_logit[tl][e]);
    }
    // The selection below overwrites tied rows' logits with their probabilities: every wave's
    // reads of the logits come first.
    __syncthreads();
  }
  if (gate_out != nullptr && wsg != nullptr && logits_in == nullptr && tid < TOK) {
    const int64_t t = tb + tid;
    if (t < T) gate_out[t] = (uint16_t)f32_to_bf16_rne(s_logit[tid][64]);
  }

  // Phase 3: SEL_LANES lanes per token (token tl0 + wave * 64 / SEL_LANES + lane / SEL_LANES).
  for (int tl0 = 0; tl0 < TOK; tl0 += ROUTE_THREADS / SEL_LANES) {
    const int tl = tl0 + wave * (64 / SEL_LANES) + lane / SEL_LANES;
    const int64_t t = tb + tl;
    if (tl < TOK && t < T) {  // uniform over the token's lanes
      int oi[KMAX];
      float ow[KMAX];
      const int sel = group_select<KT + 1>(s_logit[tl], bias != nullptr ? s_bias : nullptr, E,
                                           lane % SEL_LANES, oi, ow);
      const int s = lane % SEL_LANES;
      if (sel == SEL_DONE) {
        // Every lane of the group holds the answer; lane s < k writes pair s (index, weight and
        // histogram count), so the k outputs of a token leave in one store each.
        if (s < KT) {
          int my_i = oi[0];
          float my_w = ow[0];
#pragma unroll
          for (int r = 1; r < KT; ++r) {
            if (s == r) {
              my_i = oi[r];
              my_w = ow[r];
            }
          }
          idx_out[t * KT + s] = my_i;
          if (F32IO) static_cast<float*>(w_out)[t * KT + s] = my_w;
          else static_cast<uint16_t*>(w_out)[t * KT + s] = (uint16_t)f32_to_bf16_rne(my_w);
          atomicAdd(&s_hist[tl >> 6][my_i], 1);
        }
      } else if (s == 0) {
        s_ties[atomicAdd(&s_nties, 1)] = tl | (sel == SEL_REPLAY_PROBS ? 0x100 : 0);
      }
    }
  }
  __syncthreads();

  // Phase 4: tied tokens, one wave each.
  const int nties = s_nties;
  for (int q = wave; q < nties; q += ROUTE_THREADS / 64) {
    const int tl = s_ties[q] & 0xff;
    const bool probs = (s_ties[q] & 0x100) != 0;  // wave-uniform
    const int64_t t = tb + tl;
    int oi;
    float ow;
    if (probs) {
      select_token<KT>(lane < E ? s_logit[tl][lane] : 0.0f, false, lane, E, oi, ow, s_sv[wave], s_si[wave]);
    } else {
      const float z = lane < E ? s_logit[tl][lane] + s_bias[lane] : -INFINITY;
      route_token<KT>(z, lane, E, oi, ow, s_sv[wave], s_si[wave]);
    }
    if (lane < k) {
      idx_out[t * k + lane] = oi;
      if (F32IO) static_cast<float*>(w_out)[t * k + lane] = ow;
      else static_cast<uint16_t*>(w_out)[t * k + lane] = (uint16_t)f32_to_bf16_rne(ow);
      atomicAdd(&s_hist[tl >> 6][oi], 1);
    }
  }
  __syncthreads();
  // One histogram row per 64 tokens; rows wholly past T (the second half of a last 128-token
  // block) do not exist.
  if (hist != nullptr && tid < (TOK / 64) * 64 && (tid & 63) < E) {
    const int64_t row = (int64_t)blockIdx.x * (TOK / 64) + (tid >> 6);
    if (row * 64 < T) hist[row * E + (tid & 63)] = s_hist[tid >> 6][tid & 63];
  }
}

hipError_t launch_route(const uint16_t* x, const uint16_t* wr, const uint16_t* wsg,
                        const uint16_t* logits_in, const float* bias, uint16_t* logits_out,
                        int32_t* idx_out, uint16_t* w_out, uint16_t* gate_out, int32_t* hist,
                        int64_t T, int h, int E, int k, hipStream_t stream) {
  const int64_t nblk64 = (T + ROUTE_TOKENS - 1) / ROUTE_TOKENS;
  if (nblk64 == 0) return hipSuccess;
  // One block per CU at a time (the staged router weights fill most of its LDS). When 64-token
  // blocks would take more than one round, 128-token blocks take half as many: each stages the
  // weights once for twice the tokens (configuration 4, T = 32768: 71 -> 54 us).
  const bool wide = nblk64 > device_cus();
  const int64_t nblk = wide ? (T + 127) / 128 : nblk64;
  // Up to 16 tokens: the split-K logits (one workgroup either way).
  const bool splitk = logits_in == nullptr && T <= 16 && h % 512 == 0;
#define Q38_ROUTE(KT)                                                                                         \
  case KT:                                                                                                    \
    if (splitk)                                                                                               \
      hipLaunchKernelGGL((route_kernel<KT, false, 64, true>), dim3(1), dim3(ROUTE_THREADS), 0, stream, x, wr,  \
                         wsg, logits_in, bias, logits_out, idx_out, w_out, gate_out, hist, T, h, E, k);       \
    else if (wide)                                                                                            \
      hipLaunchKernelGGL((route_kernel<KT, false, 128>), dim3((unsigned)nblk), dim3(ROUTE_THREADS), 0, stream, \
                         x, wr, wsg, logits_in, bias, logits_out, idx_out, w_out, gate_out, hist, T, h, E, k); \
    else                                                                                                      \
      hipLaunchKernelGGL((route_kernel<KT, false, 64>), dim3((unsigned)nblk), dim3(ROUTE_THREADS), 0, stream, \
                         x, wr, wsg, logits_in, bias, logits_out, idx_out, w_out, gate_out, hist, T, h, E, k); \
    break;
  switch (k) {
    Q38_ROUTE(1) Q38_ROUTE(2) Q38_ROUTE(3) Q38_ROUTE(4) Q38_ROUTE(5) Q38_ROUTE(6) Q38_ROUTE(7) Q38_ROUTE(8)
    default: return hipErrorInvalidValue;
  }
#undef Q38_ROUTE
  return hipGetLastError();
}

hipError_t launch_route_from_f32_logits(const float* logits, const float* bias, int32_t* idx_out, float* w_out,
                                        int32_t* hist, int64_t T, int E, int k, hipStream_t stream) {
  const int64_t nblk = (T + ROUTE_TOKENS - 1) / ROUTE_TOKENS;
  if (nblk == 0) return hipSuccess;
#define Q38_ROUTE(KT)                                                                                        \
  case KT:                                                                                                   \
    hipLaunchKernelGGL((route_kernel<KT, true>), dim3((unsigned)nblk), dim3(ROUTE_THREADS), 0, stream, nullptr, \
                       nullptr, nullptr, logits, bias, nullptr, idx_out, w_out, nullptr, hist, T, 64, E, k);  \
    break;
  switch (k) {
    Q38_ROUTE(1) Q38_ROUTE(2) Q38_ROUTE(3) Q38_ROUTE(4) Q38_ROUTE(5) Q38_ROUTE(6) Q38_ROUTE(7) Q38_ROUTE(8)
    default: return hipErrorInvalidValue;
  }
#undef Q38_ROUTE
  return hipGetLastError();
}

}  // namespace q38
