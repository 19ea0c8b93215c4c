// Combine (R7 epilogue + R8) and the MoE block tail (modeling_qwen3_8_moe.py:831-833).
//
// For token t and its pairs p = t*k + j (valid when the routing index lies in [0, E)):
//   y_p      = bf16(Y[inv[p]] * w[p])           routing weight, inference.py:128-130
//   routed   = bf16(sum_j fp32(y_p))            fp32 k-sum, one rounding, inference.py:199
//   out[t]   = routed                                                 (no shared expert), or
//   out[t]   = bf16(routed + bf16(bf16(sigmoid(gate[t])) * S[t]))     modeling:831-833
// Y holds the down-projection rows in expert-sorted order (inv maps a pair to its row); S is the
// shared expert's output row of token t.
//
// HBM-bound: one wave per token, so the token's k routing entries (index, sorted row, weight) and
// its shared-gate logit are wave-uniform scalar loads; each lane owns 8 consecutive columns (16-byte
// loads/stores) of two 512-column chunks per pass, and all k gathered rows (plus the shared row) of
// both chunks are loaded before any is used, 2(k+1) 16-byte loads in flight per lane. Rows are read
// and the output written once, as streaming (non-temporal) accesses: whole 1 KiB runs per wave
// instruction, so nothing relies on the caches merging partial lines.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int COMBINE_WAVES = 4;  // tokens per 256-thread block

// bf16 element at a wave-uniform address, through a scalar load of its aligned dword (which never
// crosses a page boundary the element itself does not).
__device__ __forceinline__ uint32_t load_uniform_u16(const uint16_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t d = load_uniform(reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3));
  return (a & 2) ? (d >> 16) : (d & 0xffffu);
}

template <typename IdxT, int KT>
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv, const IdxT* __restrict__ idx,
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out, int64_t T, int h, int E) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * COMBINE_WAVES + wave;
  if (t >= T) return;
  // Routing entries of the token's pairs p = t*k + j; a pair whose index lies outside [0, E) is
  // dropped (its row is never read).
  int64_t ev[KT];
  int32_t row[KT];
  uint32_t wbits[KT];
  if (idx != nullptr) {
#pragma unroll
    for (int j = 0; j < KT; ++j) ev[j] = (int64_t)load_uniform(idx + t * KT + j);
  } else {
#pragma unroll
    for (int j = 0; j < KT; ++j) ev[j] = 0;
  }
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    row[j] = load_uniform(inv + t * KT + j);
    wbits[j] = load_uniform_u16(w + t * KT + j);
  }
  const uint16_t* yrow[KT];
  float wt[KT];
  bool ok[KT];
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    ok[j] = ev[j] >= 0 && ev[j] < E;
    yrow[j] = Y + (int64_t)row[j] * h;
    wt[j] = bf16_to_f32(wbits[j]);
  }
  const bool has_shared = shared != nullptr;
  const float g = has_shared ? round_bf16(sigmoid_f32(bf16_to_f32(load_uniform_u16(gate + t)))) : 0.0f;
  const uint16_t* srow = has_shared ? shared + t * h : nullptr;
  uint16_t* orow = out + t * h;

  for (int c0 = lane * 8; c0 < h; c0 += 1024) {
    const int c1 = c0 + 512;
    const bool two = c1 < h;
    u32x4_t v[2][KT], sv[2];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      if (ok[j]) {
        v[0][j] = ld16_stream(yrow[j] + c0);
        if (two) v[1][j] = ld16_stream(yrow[j] + c1);
      }
    }
    if (has_shared) {
      sv[0] = ld16_stream(srow + c0);
      if (two) sv[1] = ld16_stream(srow + c1);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (u == 1 && !two) break;
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        if (!ok[j]) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += round_bf16(bf16_to_f32(v[u][j][i] & 0xffffu) * wt[j]);
          acc[2 * i + 1] += round_bf16(bf16_to_f32(v[u][j][i] >> 16) * wt[j]);
        }
      }
      uint32_t o[4];
      if (has_shared) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float s0 = round_bf16(g * bf16_to_f32(sv[u][i] & 0xffffu));
          const float s1 = round_bf16(g * bf16_to_f32(sv[u][i] >> 16));
          const float r0 = round_bf16(acc[2 * i]) + s0;
          const float r1 = round_bf16(acc[2 * i + 1]) + s1;
          o[i] = f32_to_bf16_rne(r0) | (f32_to_bf16_rne(r1) << 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f32_to_bf16_rne(acc[2 * i]) | (f32_to_bf16_rne(acc[2 * i + 1]) << 16);
      }
      st16_stream(orow + (u == 0 ? c0 : c1), u32x4_t{o[0], o[1], o[2], o[3]});
    }
  }
}

template <typename IdxT>
static void launch_combine_t(dim3 grid, const uint16_t* Y, const int32_t* inv, const IdxT* idx, const uint16_t* w,
                             const uint16_t* shared, const uint16_t* gate, uint16_t* out, int64_t T, int h, int E,
                             int k, hipStream_t stream) {
#define Q38_COMBINE_K(KV)                                                                                   \
  case KV:                                                                                                  \
    hipLaunchKernelGGL((combine_kernel<IdxT, KV>), grid, dim3(256), 0, stream, Y, inv, idx, w, shared, gate, \
                       out, T, h, E);                                                                       \
    break;
  switch (k) {
    Q38_COMBINE_K(1) Q38_COMBINE_K(2) Q38_COMBINE_K(3) Q38_COMBINE_K(4)
    Q38_COMBINE_K(5) Q38_COMBINE_K(6) Q38_COMBINE_K(7) Q38_COMBINE_K(8)
  }
#undef Q38_COMBINE_K
}

hipError_t launch_combine(const uint16_t* Y, const int32_t* inv, const void* idx, bool idx64,
                          const uint16_t* w, const uint16_t* shared, const uint16_t* gate,
                          uint16_t* out, int64_t T, int h, int E, int k, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (k < 1 || k > 8) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((T + COMBINE_WAVES - 1) / COMBINE_WAVES));
  if (idx64)
    launch_combine_t(grid, Y, inv, (const int64_t*)idx, w, shared, gate, out, T, h, E, k, stream);
  else
    launch_combine_t(grid, Y, inv, (const int32_t*)idx, w, shared, gate, out, T, h, E, k, stream);
  return hipGetLastError();
}

}  // namespace q38
