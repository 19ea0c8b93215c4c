// Kernel launchers shared between the kernel translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

hipError_t launch_route(const uint16_t* x, const uint16_t* wr, const uint16_t* wsg,
                        const uint16_t* logits_in, const float* bias, uint16_t* logits_out,
                        int32_t* idx_out, uint16_t* w_out, uint16_t* gate_out, int32_t* hist,
                        int64_t T, int h, int E, int k, hipStream_t stream);

hipError_t launch_histogram(const void* idx, bool idx64, int32_t* hist, int64_t T, int E, int k,
                            hipStream_t stream);

hipError_t launch_permute(const void* idx, bool idx64, const int32_t* hist, int32_t* counts,
                          int32_t* starts, int32_t* perm, int4* tiles, int block_m,
                          int max_tiles, int64_t T, int E, int k, hipStream_t stream);

int gemm_block_m();

hipError_t launch_gate_up(const uint16_t* x, const int32_t* perm, const int4* tiles, int ntiles,
                          const uint16_t* w_gate, const uint16_t* w_up, int64_t estride,
                          uint16_t* H, int64_t M, int N, int K, int topk, hipStream_t stream);

hipError_t launch_down(const uint16_t* H, const int32_t* perm, const int4* tiles, int ntiles,
                       const uint16_t* w_down, int64_t estride, const uint16_t* rw, uint16_t* y,
                       int64_t M, int N, int K, hipStream_t stream);

hipError_t launch_combine(const uint16_t* y, const void* idx, bool idx64, const uint16_t* shared,
                          const uint16_t* gate, uint16_t* out, int64_t T, int h, int E, int k,
                          hipStream_t stream);

}  // namespace q38
