// fp32 expert path (configuration 1 and fp32 models): the reference runs fp32 models with true
// fp32 products and no intermediate roundings (its Triton experts use input_precision="ieee" for
// fp32, q38/inference.py:54-57, 172; the eager module computes in the parameters' dtype,
// modeling_qwen3_8_moe.py:769-793). The MFMA here is v_mfma_f32_32x32x2_f32: fp32 operands, fp32
// products and accumulation, so only the summation order differs from the CPU.
//
//   gate/up (F32_GATE_UP): H[r, n] = silu(g) * u, g = a_r . Wg[n], u = a_r . Wu[n]   (inference.py:90-96)
//     a_r = x[perm[r] / k] for routed rows r < P, x[r - P] for shared-expert rows (group E)
//   plain   (F32_PLAIN):   C[r, c] = a_r . W[c]  (down projection, inference.py:122-127; the dense
//     router logits x . W_router^T, modeling:807, with rows = tokens)
//   combine:               out[t] = sum_j Y[inv[t*k+j]] * w[t*k+j] (+ sigmoid(gate[t]) * S[t])
//
// GEMM tiling: a workgroup of 4 waves computes 64 rows x 64 output columns of one tile of the
// grouped GEMMs' tile table (each 256-row table tile is four 64-row sub-tiles) or of a dense row
// range; K runs in 32-wide fp32 slices staged through LDS (row stride 36 floats: the 16-byte
// fragment reads of 16 lanes cover all 64 banks once), double buffered with register staging. Wave
// w owns rows 32 (w / 2) and output columns 32 (w % 2); one 32x32x2 MFMA takes k-values i and 16 + i
// of the slice in its two lane halves, so a lane's operand for 16 MFMAs is one contiguous run of
// 16 floats (four 16-byte LDS reads).
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

namespace {

constexpr int F32_BM = 64;        // rows per workgroup
constexpr int F32_BN = 64;        // output columns per workgroup
constexpr int F32_BK = 32;        // K slice (fp32 elements)
constexpr int F32_LD = 36;        // LDS row stride (floats)
constexpr int F32_THREADS = 256;

enum { F32_GATE_UP = 0, F32_PLAIN = 1 };

struct F32Params {
  const float* A;            // activation rows: x [T,K] (gate/up, router) or H rows (down)
  const int32_t* perm;       // routed gate/up rows: sorted row -> pair (token = pair / topk)
  const int4* tiles;         // {group, row0, rows, -} (nullptr: dense rows [0, M))
  const int32_t* ntiles_dev; // used entries of tiles
  int64_t M;                 // dense: rows
  const float* W;            // routed weights: gate/up [E, 2N, K], down [E, N, K]; dense [N, K]
  const float* Ws_a;         // shared expert: gate [N,K] (gate/up) or down [N,K]
  const float* Ws_b;         // shared expert: up [N,K]
  float* C;                  // output rows [*, N]
  int P;                     // first shared-expert row of the row space
  int N, K, E, topk;
  float* C2;                 // dense plain only: one extra output column (weight row Ws_b), C2[row]
};

__device__ __forceinline__ f32x16_t mfma32x32x2_f32(float w, float a, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(w, a, c, 0, 0, 0);
}

// silu(g) * u in fp32: g / (1 + exp(-g)) with an accurate exp and IEEE division.
__device__ __forceinline__ float swiglu_f32(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int MODE>
__global__ __launch_bounds__(F32_THREADS) void gemm_f32_kernel(F32Params p) {
  constexpr int WROWS = MODE == F32_GATE_UP ? 2 * F32_BN : F32_BN;  // weight rows per tile
  __shared__ __attribute__((aligned(16))) float sa[2][F32_BM * F32_LD];
  __shared__ __attribute__((aligned(16))) float sw[2][WROWS * F32_LD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;

  // This workgroup's rows: sub-tile (blockIdx.x & 3) of table tile blockIdx.x >> 2, or a dense range.
  int group, row0, nrows;
  if (p.tiles != nullptr) {
    const int mt = (int)(blockIdx.x >> 2);
    if (mt >= load_uniform(p.ntiles_dev)) return;
    const int4 ti = p.tiles[mt];
    const int sub = (int)(blockIdx.x & 3) * F32_BM;
    if (sub >= ti.z) return;
    group = ti.x;
    row0 = ti.y + sub;
    nrows = min(F32_BM, ti.z - sub);
  } else {
    group = p.E;  // dense: the "shared" weights Ws_a (and Ws_b)
    row0 = (int)blockIdx.x * F32_BM;
    if ((int64_t)row0 >= p.M) return;
    nrows = (int)min((int64_t)F32_BM, p.M - row0);
  }
  const int col0 = (int)blockIdx.y * F32_BN;
  const bool routed = group < p.E;
  const int K = p.K, N = p.N;

  // Global sources of this thread's staging loads: activation rows (2 float4 per thread per
  // slice: 64 rows x 8 float4) and weight rows (WROWS x 8 float4). Rows past the tile read the
  // tile's first row; weight rows past N read row 0; their products are never stored.
  const float* asrc[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = (tid >> 3) + 32 * q;
    int grow = row0 + (r < nrows ? r : 0);
    int64_t arow;
    if (p.tiles != nullptr && MODE == F32_GATE_UP)
      arow = routed ? (int64_t)(p.perm[grow] / p.topk) : (int64_t)(grow - p.P);
    else
      arow = grow;
    asrc[q] = p.A + arow * K + 4 * (tid & 7);
  }
  constexpr int WQ = WROWS / 32;  // float4 loads per thread per slice for the weights
  const float* wsrc[WQ];
#pragma unroll
  for (int q = 0; q < WQ; ++q) {
    const int r = (tid >> 3) + 32 * q;
    int col;
    const float* base;
    if (MODE == F32_GATE_UP) {
      const bool up = r >= F32_BN;
      col = col0 + (r & (F32_BN - 1));
      base = routed ? p.W + (int64_t)group * 2 * N * K + (up ? (int64_t)N * K : 0) : (up ? p.Ws_b : p.Ws_a);
    } else {
      col = col0 + r;
      base = routed ? p.W + (int64_t)group * N * K : p.Ws_a;
      if (!routed && p.C2 != nullptr && col == N) {  // the extra column: weight row Ws_b
        base = p.Ws_b;
        col = 0;
      }
    }
    wsrc[q] = base + (int64_t)(col < N ? col : 0) * K + 4 * (tid & 7);
  }

  f32x16_t acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;

  f32x4_t ra[2], rw[WQ];
  auto load_slice = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) ra[q] = *reinterpret_cast<const f32x4_t*>(asrc[q] + k0);
#pragma unroll
    for (int q = 0; q < WQ; ++q) rw[q] = *reinterpret_cast<const f32x4_t*>(wsrc[q] + k0);
  };
  auto store_slice = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      *reinterpret_cast<f32x4_t*>(&sa[buf][((tid >> 3) + 32 * q) * F32_LD + 4 * (tid & 7)]) = ra[q];
#pragma unroll
    for (int q = 0; q < WQ; ++q)
      *reinterpret_cast<f32x4_t*>(&sw[buf][((tid >> 3) + 32 * q) * F32_LD + 4 * (tid & 7)]) = rw[q];
  };

  const int nk = K / F32_BK;
  load_slice(0);
  store_slice(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_slice((kt + 1) * F32_BK);
    // Fragments: activation row 32 wm + lr, weight rows (gate/up: gate 32 wn + lr and up 64 + ...),
    // floats [16 lh, 16 lh + 16) of the slice.
    const float* arow = &sa[buf][(32 * wm + lr) * F32_LD + 16 * lh];
    f32x4_t af[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) af[q] = *reinterpret_cast<const f32x4_t*>(arow + 4 * q);
#pragma unroll
    for (int j = 0; j < (MODE == F32_GATE_UP ? 2 : 1); ++j) {
      const float* wrow = &sw[buf][(F32_BN * j + 32 * wn + lr) * F32_LD + 16 * lh];
      f32x4_t wf[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) wf[q] = *reinterpret_cast<const f32x4_t*>(wrow + 4 * q);
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[j] = mfma32x32x2_f32(wf[i >> 2][i & 3], af[i >> 2][i & 3], acc[j]);
    }
    if (kt + 1 < nk) {
      store_slice(buf ^ 1);
      __syncthreads();
    }
  }

  // Lane lr holds activation row 32 wm + lr; register i holds output column
  // 8 (i / 4) + 4 lh + i % 4 of the wave's 32 columns.
  const int r = 32 * wm + lr;
  if (r >= nrows) return;
  float* crow = p.C + (int64_t)(row0 + r) * N;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const int c = col0 + 32 * wn + 8 * g4 + 4 * lh;
    f32x4_t v;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = MODE == F32_GATE_UP ? swiglu_f32(acc[0][4 * g4 + i], acc[1][4 * g4 + i]) : acc[0][4 * g4 + i];
    // 16-byte stores only where the row stride keeps them aligned (N % 4 == 0; c is a multiple of
    // 4); narrow or odd widths (router logits with E % 4 != 0) store element by element.
    if ((N & 3) == 0 && c + 3 < N) {
      *reinterpret_cast<f32x4_t*>(crow + c) = v;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (c + i < N) crow[c + i] = v[i];
        if (MODE == F32_PLAIN && p.C2 != nullptr && c + i == N) p.C2[row0 + r] = v[i];
      }
    }
  }
}

template <typename IdxT, int KT>
__global__ __launch_bounds__(256) void combine_f32_kernel(const float* __restrict__ Y, const int32_t* __restrict__ inv,
                                                          const IdxT* __restrict__ idx, const float* __restrict__ w,
                                                          const float* __restrict__ shared,
                                                          const float* __restrict__ gate, float* __restrict__ out,
                                                          int64_t T, int h, int E) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;
  const float* yrow[KT];
  float wt[KT];
  bool ok[KT];
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    const int64_t e = idx != nullptr ? (int64_t)load_uniform(idx + t * KT + j) : 0;
    ok[j] = e >= 0 && e < E;
    yrow[j] = Y + (int64_t)load_uniform(inv + t * KT + j) * h;
    wt[j] = load_uniform(w + t * KT + j);
  }
  const float g = shared != nullptr ? 1.0f / (1.0f + expf(-load_uniform(gate + t))) : 0.0f;
  for (int c = 4 * lane; c < h; c += 256) {
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      if (!ok[j]) continue;
      const f32x4_t y = *reinterpret_cast<const f32x4_t*>(yrow[j] + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float yw = y[i] * wt[j];  // the weighted pair row, then the k-sum (inference.py:128-130, 199)
        acc[i] = acc[i] + yw;
      }
    }
    if (shared != nullptr) {
      const f32x4_t s = *reinterpret_cast<const f32x4_t*>(shared + t * h + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gs = g * s[i];  // modeling:831-833
        acc[i] = acc[i] + gs;
      }
    }
    *reinterpret_cast<f32x4_t*>(out + t * h + c) = acc;
  }
}

}  // namespace

// Launch helpers. tiles != nullptr: grouped over the tile table (max_mtiles entries of 256-row
// tiles); else dense over M_dense rows with the weights Ws_a (/ Ws_b).
hipError_t launch_gate_up_f32(const float* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                              int max_mtiles, int64_t M_dense, int P, const float* w_gate_up, const float* ws_gate,
                              const float* ws_up, float* H, int N, int K, int E, int topk, hipStream_t stream) {
  if (gemm_block_m() != 4 * F32_BM) return hipErrorInvalidValue;
  F32Params p{x, perm, tiles, ntiles_dev, M_dense, w_gate_up, ws_gate, ws_up, H, P, N, K, E, topk};
  const int64_t rb = tiles != nullptr ? 4 * (int64_t)max_mtiles : (M_dense + F32_BM - 1) / F32_BM;
  if (rb == 0) return hipSuccess;
  hipLaunchKernelGGL(gemm_f32_kernel<F32_GATE_UP>, dim3((unsigned)rb, (unsigned)((N + F32_BN - 1) / F32_BN)),
                     dim3(F32_THREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_plain_f32(const float* A, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles,
                            int64_t M_dense, const float* W, const float* Ws, float* C, int N, int K, int E,
                            hipStream_t stream) {
  if (gemm_block_m() != 4 * F32_BM) return hipErrorInvalidValue;
  F32Params p{A, nullptr, tiles, ntiles_dev, M_dense, W, Ws, nullptr, C, 0, N, K, E, 1};
  const int64_t rb = tiles != nullptr ? 4 * (int64_t)max_mtiles : (M_dense + F32_BM - 1) / F32_BM;
  if (rb == 0) return hipSuccess;
  hipLaunchKernelGGL(gemm_f32_kernel<F32_PLAIN>, dim3((unsigned)rb, (unsigned)((N + F32_BN - 1) / F32_BN)),
                     dim3(F32_THREADS), 0, stream, p);
  return hipGetLastError();
}

// Router logits [T, E] = x . w_router^T and, with w_gate, the shared-expert gate logit [T] =
// x . w_gate as column E of the same launch (modeling:807, 831): the same fp32 products and
// summation order as separate dense GEMMs, in one launch.
hipError_t launch_logits_f32(const float* x, const float* w_router, const float* w_gate, float* logits, float* gate,
                             int64_t T, int E, int K, hipStream_t stream) {
  if (gemm_block_m() != 4 * F32_BM) return hipErrorInvalidValue;
  if ((w_gate == nullptr) != (gate == nullptr)) return hipErrorInvalidValue;
  F32Params p{x, nullptr, nullptr, nullptr, T, nullptr, w_router, w_gate, logits, 0, E, K, 0, 1, gate};
  const int64_t rb = (T + F32_BM - 1) / F32_BM;
  if (rb == 0) return hipSuccess;
  const int ncols = E + (gate != nullptr ? 1 : 0);
  hipLaunchKernelGGL(gemm_f32_kernel<F32_PLAIN>, dim3((unsigned)rb, (unsigned)((ncols + F32_BN - 1) / F32_BN)),
                     dim3(F32_THREADS), 0, stream, p);
  return hipGetLastError();
}

template <typename IdxT>
static void launch_combine_f32_t(dim3 grid, const float* Y, const int32_t* inv, const IdxT* idx, const float* w,
                                 const float* shared, const float* gate, float* out, int64_t T, int h, int E, int k,
                                 hipStream_t stream) {
#define Q38_COMBINE_F32(KV)                                                                                      \
  case KV:                                                                                                       \
    hipLaunchKernelGGL((combine_f32_kernel<IdxT, KV>), grid, dim3(256), 0, stream, Y, inv, idx, w, shared, gate, \
                       out, T, h, E);                                                                            \
    break;
  switch (k) {
    Q38_COMBINE_F32(1) Q38_COMBINE_F32(2) Q38_COMBINE_F32(3) Q38_COMBINE_F32(4)
    Q38_COMBINE_F32(5) Q38_COMBINE_F32(6) Q38_COMBINE_F32(7) Q38_COMBINE_F32(8)
  }
#undef Q38_COMBINE_F32
}

hipError_t launch_combine_f32(const float* Y, const int32_t* inv, const void* idx, bool idx64, const float* w,
                              const float* shared, const float* gate, float* out, int64_t T, int h, int E, int k,
                              hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (k < 1 || k > 8 || h % 4 != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((T + 3) / 4));
  if (idx64)
    launch_combine_f32_t(grid, Y, inv, (const int64_t*)idx, w, shared, gate, out, T, h, E, k, stream);
  else
    launch_combine_f32_t(grid, Y, inv, (const int32_t*)idx, w, shared, gate, out, T, h, E, k, stream);
  return hipGetLastError();
}

}  // namespace q38
