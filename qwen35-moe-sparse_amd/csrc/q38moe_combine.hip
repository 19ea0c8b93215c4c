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
// HBM-bound: each thread owns 8 consecutive columns (16-byte loads/stores) of one token; the k
// gathered rows are whole 2*h-byte rows.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

template <typename IdxT>
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv, const IdxT* __restrict__ idx,
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out, int64_t T, int h, int E, int k) {
  const int cpt = h >> 3;  // 8-column chunks per token
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= T * cpt) return;
  const int64_t t = gid / cpt;
  const int c = (int)(gid - t * cpt) * 8;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int64_t pair = t * k + j;
    if (idx != nullptr) {
      const int64_t ev = (int64_t)idx[pair];
      if (ev < 0 || ev >= E) continue;
    }
    const int64_t row = inv[pair];
    const float wt = bf16_to_f32(w[pair]);
    const u32x4_t v = ld16(Y + row * h + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += round_bf16(bf16_to_f32(v[i] & 0xffffu) * wt);
      acc[2 * i + 1] += round_bf16(bf16_to_f32(v[i] >> 16) * wt);
    }
  }
  uint32_t o[4];
  if (shared != nullptr) {
    const float g = round_bf16(sigmoid_f32(bf16_to_f32(gate[t])));
    const u32x4_t sv = ld16(shared + t * h + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s0 = round_bf16(g * bf16_to_f32(sv[i] & 0xffffu));
      const float s1 = round_bf16(g * bf16_to_f32(sv[i] >> 16));
      const float r0 = round_bf16(acc[2 * i]) + s0;
      const float r1 = round_bf16(acc[2 * i + 1]) + s1;
      o[i] = f32_to_bf16_rne(r0) | (f32_to_bf16_rne(r1) << 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32_to_bf16_rne(acc[2 * i]) | (f32_to_bf16_rne(acc[2 * i + 1]) << 16);
  }
  st16(out + t * h + c, u32x4_t{o[0], o[1], o[2], o[3]});
}

hipError_t launch_combine(const uint16_t* Y, const int32_t* inv, const void* idx, bool idx64,
                          const uint16_t* w, const uint16_t* shared, const uint16_t* gate,
                          uint16_t* out, int64_t T, int h, int E, int k, hipStream_t stream) {
  const int64_t n = T * (h >> 3);
  if (n == 0) return hipSuccess;
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (idx64)
    hipLaunchKernelGGL(combine_kernel<int64_t>, dim3(grid), dim3(256), 0, stream, Y, inv,
                       (const int64_t*)idx, w, shared, gate, out, T, h, E, k);
  else
    hipLaunchKernelGGL(combine_kernel<int32_t>, dim3(grid), dim3(256), 0, stream, Y, inv,
                       (const int32_t*)idx, w, shared, gate, out, T, h, E, k);
  return hipGetLastError();
}

}  // namespace q38
