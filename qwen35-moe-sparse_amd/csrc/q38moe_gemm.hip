// Grouped expert GEMMs on bf16 MFMA (R5-R7, R9).
//
//   gate/up (MODE_GATE_UP): H[r, n] = bf16(bf16(silu(bf16(A[r].Wg[n]))) * bf16(A[r].Wu[n]))
//     A[r] = x[perm[r] / k] for routed experts (the token gather of inference.py:74, 83-84), or
//     x[r] for the shared expert (dense, one group). Reference rounding: inference.py:90-96.
//   down (MODE_DOWN): routed: y[perm[r], c] = bf16(bf16(H[r].Wd[c]) * w[perm[r]])
//     (inference.py:122-130, pair-order store); shared: out[r, c] = bf16(Hs[r].Wd[c]).
//
// Weights are [N, K] row-major (K contiguous), the layout of experts.gate_up_proj[e] /
// experts.down_proj[e] and of nn.Linear weights, so both MFMA operands are K-contiguous.
// One workgroup (4 waves, 2x2) computes a 128-row x 128-weight-row tile; K advances in 64-wide
// slices staged through double-buffered LDS (XOR-swizzled 16-byte chunks: conflict-free
// fragment reads). Each wave owns a 64x64 accumulator block of four 32x32x16 MFMA tiles. For
// gate/up the 128 weight rows of a tile are 64 gate rows and the matching 64 up rows, arranged
// so each wave holds gate and up accumulators of the same output columns and applies SwiGLU in
// registers.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int GEMM_BM = 128;
constexpr int GEMM_BNB = 128;
constexpr int GEMM_BK = 64;

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

struct GemmParams {
  const uint16_t* A;    // activations, K contiguous
  const int32_t* perm;  // routed: sorted row -> pair; nullptr for the dense shared expert
  const int4* tiles;    // routed tile table {expert, row0, rows, -}; nullptr = dense
  const uint16_t* Bg;   // gate (or down) weights of expert 0
  const uint16_t* Bu;   // up weights of expert 0 (gate/up only)
  int64_t b_estride;    // elements between consecutive experts' weights
  uint16_t* C;          // output
  const uint16_t* rw;   // routing weight per pair (routed down), else nullptr
  int64_t M;            // rows of the dense problem
  int N;                // output columns
  int K;
  int topk;
};

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][GEMM_BM * GEMM_BK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][GEMM_BNB * GEMM_BK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int e, row0, nrows;
  if (p.tiles != nullptr) {
    const int4 ti = p.tiles[blockIdx.x];
    e = ti.x;
    row0 = ti.y;
    nrows = ti.z;
  } else {
    e = 0;
    row0 = blockIdx.x * GEMM_BM;
    nrows = (int)min((int64_t)GEMM_BM, p.M - (int64_t)row0);
  }
  if (nrows <= 0) return;
  constexpr int BN_OUT = MODE == MODE_GATE_UP ? GEMM_BNB / 2 : GEMM_BNB;
  const int n0 = blockIdx.y * BN_OUT;
  const int K = p.K, N = p.N;

  // Global -> LDS slots: 16-byte chunk c = tid + 256*i, tile row (tid >> 3) + 32*i, chunk tid & 7.
  const int kc = tid & 7;
  // Rows past the tile's valid rows (and weight rows past N) read a clamped in-bounds row; their
  // accumulators only reach output rows/columns that are never stored.
  const uint16_t* a_src[4];
  const uint16_t* b_src[4];
  int lds_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    const bool a_ok = r < nrows;
    int64_t arow;
    if (MODE == MODE_GATE_UP && p.perm != nullptr)
      arow = (int64_t)(p.perm[row0 + (a_ok ? r : 0)] / p.topk);
    else
      arow = (int64_t)row0 + (a_ok ? r : 0);
    a_src[i] = p.A + arow * K + kc * 8;
    int col;
    const uint16_t* base;
    if (MODE == MODE_GATE_UP) {
      const int half = r >> 6, within = r & 63;
      col = n0 + 32 * half + (within & 31);
      base = (within >= 32 ? p.Bu : p.Bg) + (int64_t)e * p.b_estride;
    } else {
      col = n0 + r;
      base = p.Bg + (int64_t)e * p.b_estride;
    }
    b_src[i] = base + (int64_t)(col < N ? col : 0) * K + kc * 8;
    lds_off[i] = r * GEMM_BK + ((kc ^ (r & 7)) << 3);
  }

  f32x16_t acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;

  u32x4_t ra[4], rb[4];

  const int lr = lane & 31, lh = lane >> 5;
  const int nk = K / GEMM_BK;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ra[i] = ld16(a_src[i]);
    rb[i] = ld16(b_src[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    st16(&As[0][lds_off[i]], ra[i]);
    st16(&Bs[0][lds_off[i]], rb[i]);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      const int ko = (kt + 1) * GEMM_BK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ra[i] = ld16(a_src[i] + ko);
        rb[i] = ld16(b_src[i] + ko);
      }
    }
#pragma unroll
    for (int kk = 0; kk < GEMM_BK / 16; ++kk) {
      const int c = 2 * kk + lh;
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int r = 64 * wm + 32 * mi + lr;
        af[mi] = ld16(&As[buf][r * GEMM_BK + ((c ^ (r & 7)) << 3)]);
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int r = 64 * wn + 32 * ni + lr;
        bf[ni] = ld16(&Bs[buf][r * GEMM_BK + ((c ^ (r & 7)) << 3)]);
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32x32x16(af[mi], bf[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st16(&As[buf ^ 1][lds_off[i]], ra[i]);
        st16(&Bs[buf ^ 1][lds_off[i]], rb[i]);
      }
    }
    __syncthreads();
  }

  if (MODE == MODE_GATE_UP) {
    const int col = n0 + 32 * wn + lr;
    if (col < N) {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = 64 * wm + 32 * mi + 8 * (i >> 2) + 4 * lh + (i & 3);
          if (r < nrows) {
            const float g = round_bf16(acc[mi][0][i]);
            const float u = round_bf16(acc[mi][1][i]);
            const float s = round_bf16(silu_f32(g));
            p.C[(int64_t)(row0 + r) * N + col] = (uint16_t)f32_to_bf16_rne(s * u);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 64 * wm + 32 * mi + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (r < nrows) {
          int64_t orow = (int64_t)row0 + r;
          float scale = 1.0f;
          if (p.perm != nullptr) {
            const int pair = p.perm[row0 + r];
            orow = pair;
            scale = bf16_to_f32(p.rw[pair]);
          }
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            const int col = n0 + 64 * wn + 32 * ni + lr;
            if (col < N) {
              float v = round_bf16(acc[mi][ni][i]);
              if (p.perm != nullptr) v = v * scale;
              p.C[orow * N + col] = (uint16_t)f32_to_bf16_rne(v);
            }
          }
        }
      }
    }
  }
}

int gemm_block_m() { return GEMM_BM; }

hipError_t launch_gate_up(const uint16_t* x, const int32_t* perm, const int4* tiles, int ntiles,
                          const uint16_t* w_gate, const uint16_t* w_up, int64_t estride,
                          uint16_t* H, int64_t M, int N, int K, int topk, hipStream_t stream) {
  GemmParams p;
  p.A = x;
  p.perm = perm;
  p.tiles = tiles;
  p.Bg = w_gate;
  p.Bu = w_up;
  p.b_estride = estride;
  p.C = H;
  p.rw = nullptr;
  p.M = M;
  p.N = N;
  p.K = K;
  p.topk = topk;
  const int64_t mt = tiles != nullptr ? ntiles : (M + GEMM_BM - 1) / GEMM_BM;
  const int nt = (N + GEMM_BNB / 2 - 1) / (GEMM_BNB / 2);
  if (mt == 0 || nt == 0) return hipSuccess;
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_GATE_UP>, dim3((unsigned)mt, (unsigned)nt),
                     dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_down(const uint16_t* H, const int32_t* perm, const int4* tiles, int ntiles,
                       const uint16_t* w_down, int64_t estride, const uint16_t* rw, uint16_t* y,
                       int64_t M, int N, int K, hipStream_t stream) {
  GemmParams p;
  p.A = H;
  p.perm = perm;
  p.tiles = tiles;
  p.Bg = w_down;
  p.Bu = nullptr;
  p.b_estride = estride;
  p.C = y;
  p.rw = rw;
  p.M = M;
  p.N = N;
  p.K = K;
  p.topk = 1;
  const int64_t mt = tiles != nullptr ? ntiles : (M + GEMM_BM - 1) / GEMM_BM;
  const int nt = (N + GEMM_BNB - 1) / GEMM_BNB;
  if (mt == 0 || nt == 0) return hipSuccess;
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_DOWN>, dim3((unsigned)mt, (unsigned)nt), dim3(256),
                     0, stream, p);
  return hipGetLastError();
}

}  // namespace q38
