// Kernel launchers shared between the kernel translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace q38 {

// Compute units of the current device (the persistent kernels' grid), queried once per device.
inline int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

hipError_t launch_route(const uint16_t* x, const uint16_t* wr, const uint16_t* wsg,
                        const uint16_t* logits_in, const float* bias, uint16_t* logits_out,
                        int32_t* idx_out, uint16_t* w_out, uint16_t* gate_out, int32_t* hist,
                        int64_t T, int h, int E, int k, hipStream_t stream);

// Selection from fp32 logits (the fp32 path): fp32 renormalised weights out.
hipError_t launch_route_from_f32_logits(const float* logits, const float* bias, int32_t* idx_out, float* w_out,
                                        int32_t* hist, int64_t T, int E, int k, hipStream_t stream);

// fp32 path (q38moe_fp32.hip): gate/up + SwiGLU and plain GEMMs (down, dense router logits) on fp32
// MFMA over the same tile table (tiles != nullptr) or dense rows [0, M_dense) with the weights Ws
// (Ws_a/Ws_b), and the fp32 combine.
hipError_t launch_gate_up_f32(const float* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                              int max_mtiles, int64_t M_dense, int P, const float* w_gate_up, const float* ws_gate,
                              const float* ws_up, float* H, int N, int K, int E, int topk, hipStream_t stream);
hipError_t launch_plain_f32(const float* A, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles,
                            int64_t M_dense, const float* W, const float* Ws, float* C, int N, int K, int E,
                            hipStream_t stream);

// Router logits [T, E] and, with w_gate (and gate), the shared gate logit [T] as column E of one
// dense fp32 launch (gemm_f32_kernel), results as from separate launch_plain_f32 calls.
hipError_t launch_logits_f32(const float* x, const float* w_router, const float* w_gate, float* logits, float* gate,
                             int64_t T, int E, int K, hipStream_t stream);
hipError_t launch_combine_f32(const float* Y, const int32_t* inv, const void* idx, bool idx64, const float* w,
                              const float* shared, const float* gate, float* out, int64_t T, int h, int E, int k,
                              hipStream_t stream);

hipError_t launch_histogram(const void* idx, bool idx64, int32_t* hist, int64_t T, int E, int k,
                            hipStream_t stream);

hipError_t launch_permute(const void* idx, bool idx64, const int32_t* hist, int32_t* counts,
                          int32_t* starts, int32_t* perm, int32_t* inv, int4* tiles,
                          int32_t* tile_count, int block_m, int max_tiles, int shared_rows,
                          int64_t T, int E, int k, hipStream_t stream,
                          const float* row_scale_in = nullptr, float* row_scale_out = nullptr);

// Rows per grouped-GEMM tile.
int gemm_block_m();

// Grouped gate/up + SwiGLU. tiles != nullptr: routed (+ shared, group E) tiles from permute, at
// most max_mtiles, the used count in *ntiles_dev; rows [0, P) gather x via perm, rows >= P are
// shared-expert tokens r - P. tiles == nullptr: dense shared expert over M_dense rows.
hipError_t launch_gate_up(const uint16_t* x, const int32_t* perm, const int4* tiles,
                          const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                          const uint16_t* w_gate_up, const uint16_t* ws_gate,
                          const uint16_t* ws_up, uint16_t* H, int N, int K, int E, int topk,
                          hipStream_t stream);

// Grouped down projection: Y[r] = bf16(H[r] . W^T) for the same tiles (or dense rows).
hipError_t launch_down(const uint16_t* H, const int4* tiles, const int32_t* ntiles_dev,
                       int max_mtiles, int64_t M_dense, const uint16_t* w_down,
                       const uint16_t* ws_down, uint16_t* Y, int N, int K, int E,
                       hipStream_t stream);

// Four-wave bf16 grouped gate/up + SwiGLU (q38moe_gemm4w.hip): same arguments and results (up to fp32
// summation order) as launch_gate_up, which calls it when gemm4w_supported(N, K, x_rows); x_rows
// bounds every row of x read.
bool gemm4w_supported(int N, int K, int64_t x_rows);
hipError_t launch_gate_up_4w(const uint16_t* x, int64_t x_rows, const int32_t* perm, const int4* tiles,
                             const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                             const uint16_t* w_gate_up, const uint16_t* ws_gate, const uint16_t* ws_up, uint16_t* H,
                             int N, int K, int E, int topk, hipStream_t stream);
// The same kernel on e4m3 operands (K in elements; runs when gemm4w_supported(N, K / 2, x_rows)): same
// arguments and results (up to fp32 summation order) as launch_gate_up_fp8, which calls it.
hipError_t launch_gate_up_4w_fp8(const uint8_t* xq, int64_t x_rows, const int32_t* perm, const int4* tiles,
                                 const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                                 const float* a_scale, const uint8_t* wq_gate_up, const float* s_gate_up,
                                 const uint8_t* wq_sh_gate, const float* s_sh_gate, const uint8_t* wq_sh_up,
                                 const float* s_sh_up, uint16_t* H, int N, int K, int E, int topk,
                                 hipStream_t stream);

// Grouped gate/up + SwiGLU over routed tiles (no shared-expert rows) that also stores the bf16
// pre-activations GU [rows, 2N] = [bf16(g) | bf16(u)] next to H [rows, N].
hipError_t launch_gate_up_save(const uint16_t* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                               int max_mtiles, int P, const uint16_t* w_gate_up, uint16_t* H, uint16_t* GU, int N,
                               int K, int E, int topk, hipStream_t stream);

// Grouped down-form product with K-major weights: Y[r, n] = bf16(sum_k A[r, k] w_kn[e, k, n]) for
// the rows of each expert tile (tables without shared-expert rows), w_kn [E, K, N] bf16.
hipError_t launch_down_kn(const uint16_t* A, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles,
                          const uint16_t* w_kn, uint16_t* Y, int N, int K, int E, hipStream_t stream);

// The same two GEMMs (tile tables only, bf16) decomposed for few rows per expert: 16 weight rows x
// up to 64 activation rows per workgroup, K split over its waves (q38moe_gemm_small.hip), for K in
// {128, 256, 512, 1024, 2048} (small_gemm_supported); P = T * k routed rows, shared_rows after them.
bool small_gemm_supported(int K);
// e4m3 small tiles (q38moe_gemm_small.hip): K in {512, 1024, 2048}; scales as launch_gate_up_fp8 /
// launch_down_fp8 take them.
bool small_gemm_fp8_supported(int K);
hipError_t launch_gate_up_small_fp8(const uint8_t* xq, const float* a_scale, const int32_t* perm, const int4* tiles,
                                    const int32_t* ntiles_dev, int max_mtiles, int P, int shared_rows,
                                    const uint8_t* wq_gate_up, const float* s_gate_up, const uint8_t* wq_sh_gate,
                                    const float* s_sh_gate, const uint8_t* wq_sh_up, const float* s_sh_up,
                                    uint16_t* H, int N, int K, int E, int topk, hipStream_t stream);
hipError_t launch_down_small_fp8(const uint8_t* Hq, const float* a_scale, const int4* tiles, const int32_t* ntiles_dev,
                                 int max_mtiles, int P, int shared_rows, const uint8_t* wq_down, const float* s_down,
                                 const uint8_t* wq_sh_down, const float* s_sh_down, uint16_t* Y, int N, int K, int E,
                                 hipStream_t stream);
hipError_t launch_gate_up_small(const uint16_t* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                                int max_mtiles, int P, int shared_rows, const uint16_t* w_gate_up,
                                const uint16_t* ws_gate, const uint16_t* ws_up, uint16_t* H, int N, int K, int E,
                                int topk, hipStream_t stream);
hipError_t launch_down_small(const uint16_t* H, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles, int P,
                             int shared_rows, const uint16_t* w_down, const uint16_t* ws_down, uint16_t* Y, int N,
                             int K, int E, hipStream_t stream);

// Grouped GEMM with gathered activation rows and plain weight rows: C[r] = bf16(A[perm[r] / topk] .
// W[e]^T) for the routed rows of a tile table without shared-expert rows; W [E, N, K].
hipError_t launch_gather_gemm(const uint16_t* A, const int32_t* perm, const int4* tiles,
                              const int32_t* ntiles_dev, int max_mtiles, const uint16_t* W, uint16_t* C,
                              int N, int K, int E, int topk, hipStream_t stream);

// Experts backward element-wise steps (q38moe_backward.hip).
hipError_t launch_pair_dots(const uint16_t* dout, const uint16_t* Y, const int32_t* inv, const void* idx,
                            bool idx64, const uint16_t* w, uint16_t* dw, uint16_t* d_raw, int64_t T, int h, int E,
                            int k, hipStream_t stream);
hipError_t launch_gather_rows(const uint16_t* src, const int32_t* perm, const uint16_t* w, const int32_t* starts,
                              const int32_t* counts, uint16_t* dst, int64_t P, int h, int E, int k,
                              hipStream_t stream);
// dst[e] = src[e]^T, bf16 [E, R, C] -> [E, C, R]; R, C multiples of 64.
hipError_t launch_transpose_experts(const uint16_t* src, uint16_t* dst, int E, int R, int C, hipStream_t stream);
// dW[e] = G_e^T . X_e over each expert's sorted rows (X gathered through perm / k, or sorted rows
// when perm is NULL); G [P, M], dW [E, M, N] bf16.
hipError_t launch_expert_wgrad(const uint16_t* G, const uint16_t* X, const int32_t* perm, const int32_t* starts,
                               const int32_t* counts, uint16_t* dW, int64_t P, int E, int M, int N, int k,
                               hipStream_t stream);
hipError_t launch_swiglu_backward(const uint16_t* dH, const uint16_t* GU, uint16_t* dGU, int64_t rows, int I,
                                  hipStream_t stream);

// e4m3 forms (fp8 expert path): A rows and weights e4m3 (K elements per row), fp32 scales per
// GEMM row (a_scale, the sorted row space) and per weight row; outputs bf16 as above.
hipError_t launch_gate_up_fp8(const uint8_t* xq, const int32_t* perm, const int4* tiles,
                              const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                              const float* a_scale, const uint8_t* wq_gate_up, const float* s_gate_up,
                              const uint8_t* wq_sh_gate, const float* s_sh_gate,
                              const uint8_t* wq_sh_up, const float* s_sh_up, uint16_t* H, int N,
                              int K, int E, int topk, hipStream_t stream);
hipError_t launch_down_fp8(const uint8_t* Hq, const int4* tiles, const int32_t* ntiles_dev,
                           int max_mtiles, int64_t M_dense, const float* a_scale,
                           const uint8_t* wq_down, const float* s_down, const uint8_t* wq_sh_down,
                           const float* s_sh_down, uint16_t* Y, int N, int K, int E,
                           hipStream_t stream);

hipError_t launch_combine(const uint16_t* Y, const int32_t* inv, const void* idx, bool idx64,
                          const uint16_t* w, const uint16_t* shared, const uint16_t* gate,
                          uint16_t* out, int64_t T, int h, int E, int k, hipStream_t stream);

// Per-row e4m3 quantisation (fp8 expert path): q [R,C] e4m3 bytes, scale [R] fp32 (C % 64 == 0,
// C <= 4096).
hipError_t launch_quant_rows(const uint16_t* x, uint8_t* q, float* scale, int64_t R, int C,
                             hipStream_t stream);

}  // namespace q38
