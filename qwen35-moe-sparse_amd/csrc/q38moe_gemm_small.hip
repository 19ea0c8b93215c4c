// Grouped expert GEMMs on bf16 MFMA for few rows per expert (decode and short prefill chunks):
// the same products and roundings as grouped_gemm_kernel (q38moe_gemm.hip), decomposed for a
// weight-streaming regime instead of one persistent 256 x 256 tile per CU.
//
//   gate/up: H[r, n] = bf16(bf16(silu(bf16(a_r.Wg[n]))) * bf16(a_r.Wu[n]))   (inference.py:90-96)
//     a_r = x[perm[r] / k] for routed rows r < P, x[r - P] for shared-expert rows (group E)
//   down:    Y[r, c] = bf16(H[r].Wd[c])                                       (inference.py:122-127)
//
// With few rows per expert the GEMMs are bound by streaming each expert's weights once, and the
// persistent kernel's units (a 256-row tile x 256 weight rows) are too few and too long: each
// walks 512 KiB of weights through one CU. Here a workgroup owns 16 weight rows (gate/up: 8 gate
// and the matching 8 up rows; down: 16 rows) of one expert and up to 64 activation rows (a quarter
// of a tile-table tile). Its 4 waves split K (wave w takes the 32-element k-steps s = w, w+4, ...)
// and load all their weight fragments at once, straight into MFMA operand registers, so the whole
// weight block is in flight in one round trip. Activation rows follow in blocks of 16 (the next
// block's loads overlap the current block's reduction); each block is one chain of
// mfma_f32_16x16x32_bf16 per wave, the 4 partial sums meet in LDS and are added in wave order
// (fixed, so results repeat bit for bit), then rounded like the persistent kernel's epilogue.
#include <algorithm>

#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

namespace {

constexpr int SM_ROWS = 64;      // activation rows per workgroup
constexpr int SM_THREADS = 256;  // 4 waves

enum { SM_GATE_UP = 0, SM_DOWN = 1 };

struct SmParams {
  const uint16_t* A;
  const int32_t* perm;
  const int4* tiles;
  const int32_t* ntiles_dev;
  const uint16_t* W;
  const uint16_t* Ws_a;
  const uint16_t* Ws_b;
  uint16_t* C;
  int P;
  int N, K, E, topk;
};

// KJ = K / 128: k-steps of 32 per wave.
template <int MODE, int KJ>
__global__ __launch_bounds__(SM_THREADS) void gemm_small_kernel(SmParams p) {
  __shared__ __attribute__((aligned(16))) float red[2][4][16 * 16];  // [parity][wave][act row][w row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // blockIdx.x = weight block (fastest, so that workgroups dispatched together sweep one expert's
  // weights contiguously instead of the same offset of every expert, which would keep to a few HBM
  // channels), blockIdx.y = 4 * tile + 64-row quarter.
  const int mt = (int)(blockIdx.y >> 2);
  if (mt >= load_uniform(p.ntiles_dev)) return;
  const int32_t* ti = reinterpret_cast<const int32_t*>(p.tiles + mt);
  const int tile_rows = load_uniform(ti + 2);
  const int sub = (int)(blockIdx.y & 3) * SM_ROWS;
  if (sub >= tile_rows) return;
  const int group = load_uniform(ti), row0 = load_uniform(ti + 1) + sub, nrows = min(SM_ROWS, tile_rows - sub);
  const bool routed = group < p.E;
  const int K = p.K, N = p.N;
  const int lr = lane & 15, lq = lane >> 4;

  // Order of the loads: the gather indices of all activation rows of the sub-tile (they lead the
  // longest dependency chain), the whole weight block, then (once the indices are in) the first
  // activation block, so that weights and activations are in flight together. Rows past the
  // sub-tile repeat its first row (never stored).
  const int koff = 32 * wave + 8 * lq;
  const int nblk = (nrows + 15) >> 4;
  int gidx[SM_ROWS / 16];
#pragma unroll
  for (int b = 0; b < SM_ROWS / 16; ++b) {
    const int r = 16 * b + lr;
    const int grow = row0 + (r < nrows ? r : 0);
    gidx[b] = MODE == SM_GATE_UP && routed ? p.perm[grow] : grow;
  }
  // This lane's weight row (MFMA A operand row lr) at k offsets 32 (4 j + wave) + 8 lq.
  const uint16_t* wrow;
  int n0;
  if (MODE == SM_GATE_UP) {
    n0 = (int)blockIdx.x * 8;
    const bool up = lr >= 8;
    const int64_t col = n0 + (lr & 7);
    wrow = routed ? p.W + (int64_t)group * 2 * N * K + (up ? (int64_t)N * K : 0) + col * K
                  : (up ? p.Ws_b : p.Ws_a) + col * K;
  } else {
    n0 = (int)blockIdx.x * 16;
    const int64_t col = n0 + lr;
    wrow = (routed ? p.W + (int64_t)group * N * K : p.Ws_a) + col * K;
  }
  u32x4_t wf[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) wf[j] = ld16(wrow + koff + 128 * j);

  const uint16_t* arow[SM_ROWS / 16];
#pragma unroll
  for (int b = 0; b < SM_ROWS / 16; ++b) {
    int64_t a = gidx[b];
    if (MODE == SM_GATE_UP) a = routed ? (int64_t)(gidx[b] / p.topk) : a - p.P;
    arow[b] = p.A + a * K + koff;
  }
  u32x4_t af[KJ];
  auto load_act = [&](const uint16_t* a) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) af[j] = ld16(a + 128 * j);
  };
  load_act(arow[0]);

  for (int b = 0; b < nblk; ++b) {
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < KJ; ++j) acc = mfma16x16x32(wf[j], af[j], acc);
    // D[i] of lane l: weight row 4 (l / 16) + i, activation row l % 16.
    float* part = red[b & 1][wave];
    *reinterpret_cast<f32x4_t*>(part + lr * 16 + 4 * lq) = acc;
    if (b + 1 < nblk) load_act(arow[b + 1]);
    __syncthreads();
    const float* rp = &red[b & 1][0][0];
    if (MODE == SM_GATE_UP) {
      // 16 activation rows x 8 columns; thread t < 128: row t / 8, column t % 8 (gate in weight
      // rows 0..7, up in 8..15). Rounding sequence and SiLU form of the persistent kernel.
      if (tid < 128) {
        const int ar = tid >> 3, c = tid & 7;
        const int r = 16 * b + ar;
        if (r < nrows) {
          float g = rp[ar * 16 + c], u = rp[ar * 16 + 8 + c];
#pragma unroll
          for (int w = 1; w < 4; ++w) {
            g += rp[w * 256 + ar * 16 + c];
            u += rp[w * 256 + ar * 16 + 8 + c];
          }
          float gb, ub, sb, dummy;
          unpack_bf16x2(pack_bf16x2(g, u), gb, ub);
          unpack_bf16x2(pack_bf16x2(gb * __builtin_amdgcn_rcpf(1.0f + __expf(-gb)), 0.0f), sb, dummy);
          float hv, dummy2;
          unpack_bf16x2(pack_bf16x2(sb * ub, 0.0f), hv, dummy2);
          p.C[(int64_t)(row0 + r) * N + n0 + c] = (uint16_t)(__float_as_uint(hv) >> 16);
        }
      }
    } else {
      // 16 activation rows x 16 columns, one per thread.
      const int ar = tid >> 4, c = tid & 15;
      const int r = 16 * b + ar;
      if (r < nrows) {
        float y = rp[ar * 16 + c];
#pragma unroll
        for (int w = 1; w < 4; ++w) y += rp[w * 256 + ar * 16 + c];
        float yb, dummy;
        unpack_bf16x2(pack_bf16x2(y, 0.0f), yb, dummy);
        p.C[(int64_t)(row0 + r) * N + n0 + c] = (uint16_t)(__float_as_uint(yb) >> 16);
      }
    }
  }
}

// The same decomposition for the e4m3 expert path (configuration 4's definition: include/q38moe.h,
// q38moe_block_forward_fp8): e4m3 activation rows with one fp32 scale per sorted row, e4m3 weight
// rows with one fp32 scale per output channel. Each wave takes the 128-byte k-steps s = w, w + 4, ...
// of K (one mfma_f32_16x16x128_f8f6f4 each, lane l: row l % 16, bytes 32 (l / 16) .. + 32 of the
// step), the four partial sums meet in LDS and are added in wave order, and the sum is dequantised
// as the persistent fp8 kernel does (sum * (weight scale * row scale)) before the same roundings.
struct Sm8Params {
  const uint8_t* A;
  const float* a_scale;  // per sorted row (gate/up: the token's scale; down: the H row's)
  const int32_t* perm;
  const int4* tiles;
  const int32_t* ntiles_dev;
  const uint8_t* W;
  const float* sW;       // per output channel of W
  const uint8_t* Ws_a;   // shared expert: gate (gate/up) or down
  const float* sWs_a;
  const uint8_t* Ws_b;   // shared expert: up (gate/up)
  const float* sWs_b;
  uint16_t* C;
  int P;
  int N, K, E, topk;
};

__device__ __forceinline__ f32x4_t mfma16x16x128_fp8(i32x8_t a, i32x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// KJ = K / 512: 128-byte k-steps per wave.
template <int MODE, int KJ>
__global__ __launch_bounds__(SM_THREADS) void gemm_small_fp8_kernel(Sm8Params p) {
  __shared__ __attribute__((aligned(16))) float red[2][4][16 * 16];  // [parity][wave][act row][w row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mt = (int)(blockIdx.y >> 2);
  if (mt >= load_uniform(p.ntiles_dev)) return;
  const int32_t* ti = reinterpret_cast<const int32_t*>(p.tiles + mt);
  const int tile_rows = load_uniform(ti + 2);
  const int sub = (int)(blockIdx.y & 3) * SM_ROWS;
  if (sub >= tile_rows) return;
  const int group = load_uniform(ti), row0 = load_uniform(ti + 1) + sub, nrows = min(SM_ROWS, tile_rows - sub);
  const bool routed = group < p.E;
  const int K = p.K, N = p.N;
  const int lr = lane & 15, lq = lane >> 4;

  const int koff = 128 * wave + 32 * lq;  // bytes
  const int nblk = (nrows + 15) >> 4;
  int gidx[SM_ROWS / 16];
#pragma unroll
  for (int b = 0; b < SM_ROWS / 16; ++b) {
    const int r = 16 * b + lr;
    const int grow = row0 + (r < nrows ? r : 0);
    gidx[b] = MODE == SM_GATE_UP && routed ? p.perm[grow] : grow;
  }
  const uint8_t* wrow;
  int n0;
  if (MODE == SM_GATE_UP) {
    n0 = (int)blockIdx.x * 8;
    const bool up = lr >= 8;
    const int64_t col = n0 + (lr & 7);
    wrow = routed ? p.W + (int64_t)group * 2 * N * K + (up ? (int64_t)N * K : 0) + col * K
                  : (up ? p.Ws_b : p.Ws_a) + col * K;
  } else {
    n0 = (int)blockIdx.x * 16;
    const int64_t col = n0 + lr;
    wrow = (routed ? p.W + (int64_t)group * N * K : p.Ws_a) + col * K;
  }
  i32x8_t wf[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) wf[j] = cat8(ld16(wrow + koff + 512 * j), ld16(wrow + koff + 512 * j + 16));

  const uint8_t* arow[SM_ROWS / 16];
#pragma unroll
  for (int b = 0; b < SM_ROWS / 16; ++b) {
    int64_t a = gidx[b];
    if (MODE == SM_GATE_UP) a = routed ? (int64_t)(gidx[b] / p.topk) : a - p.P;
    arow[b] = p.A + a * K + koff;
  }
  i32x8_t af[KJ];
  auto load_act = [&](const uint8_t* a) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) af[j] = cat8(ld16(a + 512 * j), ld16(a + 512 * j + 16));
  };
  load_act(arow[0]);

  for (int b = 0; b < nblk; ++b) {
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < KJ; ++j) acc = mfma16x16x128_fp8(wf[j], af[j], acc);
    float* part = red[b & 1][wave];
    *reinterpret_cast<f32x4_t*>(part + lr * 16 + 4 * lq) = acc;
    if (b + 1 < nblk) load_act(arow[b + 1]);
    __syncthreads();
    const float* rp = &red[b & 1][0][0];
    if (MODE == SM_GATE_UP) {
      if (tid < 128) {
        const int ar = tid >> 3, c = tid & 7;
        const int r = 16 * b + ar;
        if (r < nrows) {
          float g = rp[ar * 16 + c], u = rp[ar * 16 + 8 + c];
#pragma unroll
          for (int w = 1; w < 4; ++w) {
            g += rp[w * 256 + ar * 16 + c];
            u += rp[w * 256 + ar * 16 + 8 + c];
          }
          const float sa = p.a_scale[row0 + r];
          const float swg = routed ? p.sW[(int64_t)group * 2 * N + n0 + c] : p.sWs_a[n0 + c];
          const float swu = routed ? p.sW[(int64_t)group * 2 * N + N + n0 + c] : p.sWs_b[n0 + c];
          g = g * (swg * sa);
          u = u * (swu * sa);
          float gb, ub, sb, dummy;
          unpack_bf16x2(pack_bf16x2(g, u), gb, ub);
          unpack_bf16x2(pack_bf16x2(gb * __builtin_amdgcn_rcpf(1.0f + __expf(-gb)), 0.0f), sb, dummy);
          float hv, dummy2;
          unpack_bf16x2(pack_bf16x2(sb * ub, 0.0f), hv, dummy2);
          p.C[(int64_t)(row0 + r) * N + n0 + c] = (uint16_t)(__float_as_uint(hv) >> 16);
        }
      }
    } else {
      const int ar = tid >> 4, c = tid & 15;
      const int r = 16 * b + ar;
      if (r < nrows) {
        float y = rp[ar * 16 + c];
#pragma unroll
        for (int w = 1; w < 4; ++w) y += rp[w * 256 + ar * 16 + c];
        const float sa = p.a_scale[row0 + r];
        const float sw = routed ? p.sW[(int64_t)group * N + n0 + c] : p.sWs_a[n0 + c];
        y = y * (sw * sa);
        float yb, dummy;
        unpack_bf16x2(pack_bf16x2(y, 0.0f), yb, dummy);
        p.C[(int64_t)(row0 + r) * N + n0 + c] = (uint16_t)(__float_as_uint(yb) >> 16);
      }
    }
  }
}

// Tiles a tile table can hold: each expert with c rows has ceil(c / 256) <= c / 256 + 1 tiles, so at
// most ceil(P / 256) + min(E, P) routed tiles, plus ceil(shared / 256).
int tile_bound(int max_mtiles, int P, int E, int shared_rows) {
  const int bm = gemm_block_m();
  const int64_t b = ((int64_t)P + bm - 1) / bm + std::min<int64_t>(E, P) + ((int64_t)shared_rows + bm - 1) / bm;
  return (int)std::min<int64_t>(b, max_mtiles);
}

template <int MODE>
hipError_t launch_small(const SmParams& p, int mtiles, int ncols_per_wg, hipStream_t stream) {
  const dim3 grid((unsigned)(p.N / ncols_per_wg), 4 * (unsigned)mtiles);
  switch (p.K) {
    case 128: hipLaunchKernelGGL((gemm_small_kernel<MODE, 1>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((gemm_small_kernel<MODE, 2>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 512: hipLaunchKernelGGL((gemm_small_kernel<MODE, 4>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 1024: hipLaunchKernelGGL((gemm_small_kernel<MODE, 8>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 2048: hipLaunchKernelGGL((gemm_small_kernel<MODE, 16>), grid, dim3(SM_THREADS), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_small_fp8(const Sm8Params& p, int mtiles, int ncols_per_wg, hipStream_t stream) {
  const dim3 grid((unsigned)(p.N / ncols_per_wg), 4 * (unsigned)mtiles);
  switch (p.K) {
    case 512: hipLaunchKernelGGL((gemm_small_fp8_kernel<MODE, 1>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 1024: hipLaunchKernelGGL((gemm_small_fp8_kernel<MODE, 2>), grid, dim3(SM_THREADS), 0, stream, p); break;
    case 2048: hipLaunchKernelGGL((gemm_small_fp8_kernel<MODE, 4>), grid, dim3(SM_THREADS), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool small_gemm_supported(int K) { return K == 128 || K == 256 || K == 512 || K == 1024 || K == 2048; }

hipError_t launch_gate_up_small(const uint16_t* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                                int max_mtiles, int P, int shared_rows, const uint16_t* w_gate_up,
                                const uint16_t* ws_gate, const uint16_t* ws_up, uint16_t* H, int N, int K, int E,
                                int topk, hipStream_t stream) {
  if (gemm_block_m() != 4 * SM_ROWS || !small_gemm_supported(K) || N % 8 != 0) return hipErrorInvalidValue;
  const int mtiles = tile_bound(max_mtiles, P, E, shared_rows);
  if (mtiles == 0) return hipSuccess;
  return launch_small<SM_GATE_UP>(SmParams{x, perm, tiles, ntiles_dev, w_gate_up, ws_gate, ws_up, H, P, N, K, E, topk},
                                  mtiles, 8, stream);
}

hipError_t launch_down_small(const uint16_t* H, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles, int P,
                             int shared_rows, const uint16_t* w_down, const uint16_t* ws_down, uint16_t* Y, int N,
                             int K, int E, hipStream_t stream) {
  if (gemm_block_m() != 4 * SM_ROWS || !small_gemm_supported(K) || N % 16 != 0) return hipErrorInvalidValue;
  const int mtiles = tile_bound(max_mtiles, P, E, shared_rows);
  if (mtiles == 0) return hipSuccess;
  return launch_small<SM_DOWN>(SmParams{H, nullptr, tiles, ntiles_dev, w_down, ws_down, nullptr, Y, P, N, K, E, 1},
                               mtiles, 16, stream);
}

}  // namespace q38

namespace q38 {

bool small_gemm_fp8_supported(int K) { return K == 512 || K == 1024 || K == 2048; }

hipError_t launch_gate_up_small_fp8(const uint8_t* xq, const float* a_scale, const int32_t* perm, const int4* tiles,
                                    const int32_t* ntiles_dev, int max_mtiles, int P, int shared_rows,
                                    const uint8_t* wq_gate_up, const float* s_gate_up, const uint8_t* wq_sh_gate,
                                    const float* s_sh_gate, const uint8_t* wq_sh_up, const float* s_sh_up,
                                    uint16_t* H, int N, int K, int E, int topk, hipStream_t stream) {
  if (gemm_block_m() != 4 * SM_ROWS || !small_gemm_fp8_supported(K) || N % 8 != 0) return hipErrorInvalidValue;
  const int mtiles = tile_bound(max_mtiles, P, E, shared_rows);
  if (mtiles == 0) return hipSuccess;
  return launch_small_fp8<SM_GATE_UP>(Sm8Params{xq, a_scale, perm, tiles, ntiles_dev, wq_gate_up, s_gate_up, wq_sh_gate,
                                                s_sh_gate, wq_sh_up, s_sh_up, H, P, N, K, E, topk},
                                      mtiles, 8, stream);
}

hipError_t launch_down_small_fp8(const uint8_t* Hq, const float* a_scale, const int4* tiles, const int32_t* ntiles_dev,
                                 int max_mtiles, int P, int shared_rows, const uint8_t* wq_down, const float* s_down,
                                 const uint8_t* wq_sh_down, const float* s_sh_down, uint16_t* Y, int N, int K, int E,
                                 hipStream_t stream) {
  if (gemm_block_m() != 4 * SM_ROWS || !small_gemm_fp8_supported(K) || N % 16 != 0) return hipErrorInvalidValue;
  const int mtiles = tile_bound(max_mtiles, P, E, shared_rows);
  if (mtiles == 0) return hipSuccess;
  return launch_small_fp8<SM_DOWN>(Sm8Params{Hq, a_scale, nullptr, tiles, ntiles_dev, wq_down, s_down, wq_sh_down,
                                             s_sh_down, nullptr, nullptr, Y, P, N, K, E, 1},
                                   mtiles, 16, stream);
}

}  // namespace q38
