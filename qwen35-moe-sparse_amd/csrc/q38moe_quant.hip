// Per-row e4m3 quantisation for the fp8 expert path (R14: the reference has no fp8; the format is
// this library's definition, following the fp8 configuration of the benchmark set: OCP e4m3
// values with one fp32 scale per token row or per weight output channel).
//
// For a row x[0..C) (bf16 in):
//   amax  = max |x|                      (NaN if the row holds a NaN)
//   inv   = amax > 0 ? 448 / amax : 0    (fp32, correctly rounded division)
//   q[c]  = e4m3_rne(clamp(x[c] * inv, -448, 448))
//   scale = amax / 448                   (dequantised value = q * scale)
// The same routine quantises expert weights (rows = output channels, at load time), the tokens
// entering the gate/up GEMM and the SwiGLU rows entering the down GEMM.
//
// HBM-bound: a wave quantises RPW rows (4 of 512 columns, 2 of 1024, else 1), so that every lane
// has four 16-byte loads (8 bf16 each) in flight whatever the row length; it stores 8-byte runs.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int QUANT_WAVES = 4;  // rows per 256-thread block

// Whole-wave maximum without LDS traffic (DPP within rows, then the gfx950 row-pair and half-wave
// swaps). NaN-propagating.
__device__ __forceinline__ float nan_max(float a, float b) {
  return (__builtin_isnan(a) || __builtin_isnan(b)) ? __builtin_nanf("") : fmaxf(a, b);
}
__device__ __forceinline__ float wave_amax(float v) {
  v = nan_max(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false)));
  v = nan_max(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false)));
  v = nan_max(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
  v = nan_max(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  v = nan_max(__int_as_float(r16[0]), __int_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return nan_max(__int_as_float(r32[0]), __int_as_float(r32[1]));
}

// Two fp32 values (already scaled) -> two e4m3 bytes in the low half (a first).
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
  a = __builtin_isnan(a) ? a : fminf(fmaxf(a, -448.0f), 448.0f);
  b = __builtin_isnan(b) ? b : fminf(fmaxf(b, -448.0f), 448.0f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

template <int NCH, int RPW>  // 16-byte chunks per lane and row (C = 512 * NCH; 0: any C), rows per wave
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x,
                                                         uint8_t* __restrict__ q,
                                                         float* __restrict__ scale, int64_t R,
                                                         int C) {
  constexpr int NV = NCH > 0 ? NCH : 8;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * QUANT_WAVES + wave) * RPW;
  if (r0 >= R) return;
  const int nch = NCH > 0 ? NCH : (C / 8 + 63) / 64;
  u32x4_t v[RPW][NV];
  float m[RPW];
#pragma unroll
  for (int u = 0; u < RPW; ++u) {
    m[u] = 0.0f;
    const bool row_in = r0 + u < R;  // wave-uniform
    const uint16_t* xr = x + (r0 + u) * C;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (NCH == 0 && j >= nch) break;
      const int c = 8 * (lane + 64 * j);
      v[u][j] = row_in && c < C ? ld16_stream(xr + c) : u32x4_t{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int u = 0; u < RPW; ++u) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (NCH == 0 && j >= nch) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a, b;
        unpack_bf16x2(v[u][j][i], a, b);
        m[u] = nan_max(m[u], nan_max(fabsf(a), fabsf(b)));
      }
    }
  }
#pragma unroll
  for (int u = 0; u < RPW; ++u) {
    if (r0 + u >= R) break;  // wave-uniform
    const float amax = wave_amax(m[u]);
    const float inv = amax > 0.0f ? 448.0f / amax : (__builtin_isnan(amax) ? amax : 0.0f);
    if (lane == 0) scale[r0 + u] = amax / 448.0f;
    uint8_t* qr = q + (r0 + u) * C;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (NCH == 0 && j >= nch) break;
      const int c = 8 * (lane + 64 * j);
      if (c < C) {
        uint32_t w[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float a0, b0, a1, b1;
          unpack_bf16x2(v[u][j][2 * i], a0, b0);
          unpack_bf16x2(v[u][j][2 * i + 1], a1, b1);
          w[i] = e4m3x2(a0 * inv, b0 * inv) | (e4m3x2(a1 * inv, b1 * inv) << 16);
        }
        *reinterpret_cast<uint2*>(qr + c) = make_uint2(w[0], w[1]);
      }
    }
  }
}

hipError_t launch_quant_rows(const uint16_t* x, uint8_t* q, float* scale, int64_t R, int C,
                             hipStream_t stream) {
  if (R == 0) return hipSuccess;
  if (C % 64 != 0 || C > 8 * 64 * 8) return hipErrorInvalidValue;
  auto grid = [&](int rpw) { return dim3((unsigned)((R + QUANT_WAVES * rpw - 1) / (QUANT_WAVES * rpw))); };
  switch (C) {
    case 512:
      hipLaunchKernelGGL((quant_rows_kernel<1, 4>), grid(4), dim3(256), 0, stream, x, q, scale, R, C);
      break;
    case 1024:
      hipLaunchKernelGGL((quant_rows_kernel<2, 2>), grid(2), dim3(256), 0, stream, x, q, scale, R, C);
      break;
    case 2048:
      hipLaunchKernelGGL((quant_rows_kernel<4, 1>), grid(1), dim3(256), 0, stream, x, q, scale, R, C);
      break;
    default:
      hipLaunchKernelGGL((quant_rows_kernel<0, 1>), grid(1), dim3(256), 0, stream, x, q, scale, R, C);
      break;
  }
  return hipGetLastError();
}

}  // namespace q38
