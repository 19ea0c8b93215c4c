// Shared device helpers for the Q38 MoE prefill kernels (gfx950 / CDNA4 only).
//
// Storage types: bf16 tensors travel as raw uint16_t bit patterns; every rounding point of the
// reference (round-to-nearest-even fp32 -> bf16, c10::BFloat16 semantics, NaN -> 0x7FC0) is made
// explicit with f32_to_bf16_rne so the kernels reproduce the reference rounding sequence.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
// Native 16-byte vector (HIP's uint4 is a union-based struct that defeats scalarisation of
// register arrays).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_to_f32(uint32_t v) { return __uint_as_float(v << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// Two floats -> two bf16 (a in the low half) with one v_cvt_pk_bf16_f32 (round to nearest even,
// as f32_to_bf16_rne for every non-NaN input; a NaN stays a NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ void unpack_bf16x2(uint32_t v, float& a, float& b) {
  a = __uint_as_float(v << 16);
  b = __uint_as_float(v & 0xffff0000u);
}

// SiLU / sigmoid evaluated in fp32 as x / (1 + exp(-x)) and 1 / (1 + exp(-x)).
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }
// Streaming (non-temporal) forms for data touched once: full cache lines per wave instruction
// only, since non-temporal writes are not merged in the L2.
__device__ __forceinline__ u32x4_t ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ void st16_stream(void* p, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(p));
}

// 32x32x16 bf16 MFMA: A fragment = row (lane % 32), k-chunk (lane / 32) of 8 elements;
// B fragment = column (lane % 32), same k-chunk; D[i] of lane l = row 8*(i/4) + 4*(l/32) + i%4,
// column l % 32.
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 32x32x64 e4m3 x e4m3 MFMA (gfx950 f8f6f4 form, both operands e4m3, no block scales): 32 bytes
// per lane; lane = row (lane % 32) as in the bf16 forms.
typedef int i32x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ i32x8_t cat8(u32x4_t lo, u32x4_t hi) {
  return __builtin_bit_cast(i32x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
__device__ __forceinline__ f32x16_t mfma32x32x64_fp8(i32x8_t a, i32x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// 16x16x32 bf16 MFMA: A fragment = row (lane % 16), k-chunk (lane / 16); D[i] of lane l = row
// 4*(l/16) + i, column l % 16.
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// Asynchronous 16-byte global -> LDS copy (gfx950 global_load_lds_dwordx4): lane l of the wave
// writes LDS bytes [lds_wave_base + 16*l, +16). lds_wave_base must be wave-uniform. Completion is
// tracked by vmcnt; wait with wait_vmcnt0() before a barrier that publishes the data.
__device__ __forceinline__ void load_lds16(const void* gsrc, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

// Same for 4 bytes per lane (global_load_lds_dword): lane l writes [lds_wave_base + 4*l, +4).
__device__ __forceinline__ void load_lds4(const void* gsrc, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_wave_base, 4, 0, 0);
}

// Load through the constant address space: for a wave-uniform address the compiler emits a scalar
// load (lgkmcnt), which keeps it out of the vmcnt queue that tracks the async LDS copies. Only
// for data no kernel writes while the reading kernel runs.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace q38
