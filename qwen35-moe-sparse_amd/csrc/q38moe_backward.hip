// Experts backward pieces (the differentiable experts path of the reference,
// q38/inference.py:358-384, whose gradients scripts/check_q38_kernels.py:19-27 checks): the
// element-wise and reduction steps between the grouped GEMMs. The GEMMs themselves are the grouped
// kernels of q38moe_gemm.hip (MODE_GATHER for the gate/up pre-activations, MODE_DOWN with
// transposed weights for the two input-gradient products).
//
// Rounding follows torch's bf16 autograd of the reference ops: every product of two bf16 tensors is
// rounded to bf16, reductions accumulate in fp32 and round once.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// dw[p] = bf16(sum_c fp32(bf16(dout[t, c] * Y[inv[p], c]))) for the pairs p = t*k + j of token t (the
// gradient of routed = raw * top_k_weights, inference.py:381); pairs whose expert lies outside
// [0, E) get 0. One wave per token; lane l covers columns 8l + 512i.
template <typename IdxT>
__global__ __launch_bounds__(256) void pair_dots_kernel(const uint16_t* __restrict__ dout,
                                                        const uint16_t* __restrict__ Y,
                                                        const int32_t* __restrict__ inv,
                                                        const IdxT* __restrict__ idx,
                                                        uint16_t* __restrict__ dw, int64_t T, int h,
                                                        int E, int k) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;
  for (int j = 0; j < k; ++j) {
    const int64_t p = t * k + j;
    const int64_t e = idx != nullptr ? (int64_t)idx[p] : 0;
    float acc = 0.0f;
    if (e >= 0 && e < E) {  // wave-uniform
      const uint16_t* yr = Y + (int64_t)inv[p] * h;
      const uint16_t* dr = dout + t * h;
      for (int c = lane * 8; c < h; c += 512) {
        const u32x4_t a = ld16(dr + c), b = ld16(yr + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc += round_bf16(bf16_to_f32(a[i] & 0xffffu) * bf16_to_f32(b[i] & 0xffffu));
          acc += round_bf16(bf16_to_f32(a[i] >> 16) * bf16_to_f32(b[i] >> 16));
        }
      }
    }
    acc = wave_sum_f(acc);
    if (lane == 0) dw[p] = (uint16_t)f32_to_bf16_rne(acc);
  }
}

// dst[r] = bf16(src[perm[r] / k] * w[perm[r]]) (w == nullptr: the plain gathered row), rows r in
// expert-sorted order: the gradient of the routed raw rows (dout scaled by the routing weight,
// inference.py:381) or the gathered activation rows of the weight gradients. One wave per row.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                          const int32_t* __restrict__ perm,
                                                          const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ dst, int64_t P, int h,
                                                          int k) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  if (r >= P) return;
  const int64_t pair = perm[r];
  const uint16_t* sr = src + (pair / k) * h;
  uint16_t* dr = dst + r * h;
  const float s = w != nullptr ? bf16_to_f32(w[pair]) : 1.0f;
  for (int c = lane * 8; c < h; c += 512) {
    u32x4_t v = ld16(sr + c);
    if (w != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = pack_bf16x2(bf16_to_f32(v[i] & 0xffffu) * s, bf16_to_f32(v[i] >> 16) * s);
    }
    st16(dr + c, v);
  }
}

// SwiGLU backward per row r and column i < I, with g = GU[r, i], u = GU[r, I + i] the gate/up
// pre-activations and dh = dH[r, i] (forward: act = bf16(silu(g)), h = bf16(act * u)):
//   d_act = bf16(dh * u), d_u = bf16(dh * act),
//   d_g = bf16(d_act * sigmoid(g) * (1 + g * (1 - sigmoid(g))))   (torch's silu backward)
// written to dGU[r, i] and dGU[r, I + i] (the layout of gate_up_proj's rows). 8 columns per thread.
__global__ __launch_bounds__(256) void swiglu_backward_kernel(const uint16_t* __restrict__ dH,
                                                              const uint16_t* __restrict__ GU,
                                                              uint16_t* __restrict__ dGU, int64_t rows,
                                                              int I) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int per_row = I / 8;
  const int64_t r = gid / per_row;
  if (r >= rows) return;
  const int c = (int)(gid - r * per_row) * 8;
  const u32x4_t dh = ld16(dH + r * I + c);
  const u32x4_t gv = ld16(GU + r * 2 * I + c);
  const u32x4_t uv = ld16(GU + r * 2 * I + I + c);
  u32x4_t dg, du;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float d[2], g[2], u[2], og[2], ou[2];
    unpack_bf16x2(dh[i], d[0], d[1]);
    unpack_bf16x2(gv[i], g[0], g[1]);
    unpack_bf16x2(uv[i], u[0], u[1]);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const float sg = sigmoid_f32(g[h2]);
      const float act = round_bf16(g[h2] * sg);
      const float dact = round_bf16(d[h2] * u[h2]);
      ou[h2] = d[h2] * act;
      og[h2] = dact * (sg * (1.0f + g[h2] * (1.0f - sg)));
    }
    dg[i] = pack_bf16x2(og[0], og[1]);
    du[i] = pack_bf16x2(ou[0], ou[1]);
  }
  st16(dGU + r * 2 * I + c, dg);
  st16(dGU + r * 2 * I + I + c, du);
}

hipError_t launch_pair_dots(const uint16_t* dout, const uint16_t* Y, const int32_t* inv, const void* idx,
                            bool idx64, uint16_t* dw, int64_t T, int h, int E, int k, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const dim3 grid((unsigned)((T + 3) / 4));
  if (idx64)
    hipLaunchKernelGGL(pair_dots_kernel<int64_t>, grid, dim3(256), 0, stream, dout, Y, inv,
                       static_cast<const int64_t*>(idx), dw, T, h, E, k);
  else
    hipLaunchKernelGGL(pair_dots_kernel<int32_t>, grid, dim3(256), 0, stream, dout, Y, inv,
                       static_cast<const int32_t*>(idx), dw, T, h, E, k);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const uint16_t* src, const int32_t* perm, const uint16_t* w, uint16_t* dst,
                              int64_t P, int h, int k, hipStream_t stream) {
  if (P == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((P + 3) / 4)), dim3(256), 0, stream, src, perm, w, dst,
                     P, h, k);
  return hipGetLastError();
}

hipError_t launch_swiglu_backward(const uint16_t* dH, const uint16_t* GU, uint16_t* dGU, int64_t rows, int I,
                                  hipStream_t stream) {
  const int64_t n = rows * (I / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_backward_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dH, GU, dGU,
                     rows, I);
  return hipGetLastError();
}

}  // namespace q38
