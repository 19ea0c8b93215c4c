// Experts backward pieces (the differentiable experts path of the reference,
// q38/inference.py:358-384, whose gradients scripts/check_q38_kernels.py:19-27 checks): the
// element-wise and reduction steps between the grouped GEMMs. The GEMMs themselves are the grouped
// kernels of q38moe_gemm.hip (MODE_GATHER for the gate/up pre-activations, MODE_DOWN with
// transposed weights for the two input-gradient products).
//
// Rounding follows torch's bf16 autograd of the reference ops: every product of two bf16 tensors is
// rounded to bf16, reductions accumulate in fp32 and round once.
#include <type_traits>

#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int WG_T = 256;  // weight-gradient output tile: G columns (X columns: WD_TN)

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// dw[p] = bf16(sum_c fp32(bf16(dout[t, c] * Y[inv[p], c]))) for the pairs p = t*k + j of token t (the
// gradient of routed = raw * top_k_weights, inference.py:381); pairs whose expert lies outside
// [0, E) get 0. With w and d_raw given, the same pass also writes the routed raw rows' gradient in
// sorted order, d_raw[inv[p]] = bf16(dout[t] * w[p]) (what gather_rows_kernel computes), reading
// each dout row once for both. One wave per token; lane l covers columns 8l + 512i.
template <typename IdxT, int KT>
__global__ __launch_bounds__(256) void pair_dots_kernel(const uint16_t* __restrict__ dout,
                                                        const uint16_t* __restrict__ Y,
                                                        const int32_t* __restrict__ inv,
                                                        const IdxT* __restrict__ idx,
                                                        const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ dw,
                                                        uint16_t* __restrict__ d_raw, int64_t T, int h,
                                                        int E) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;
  // The token's KT pairs: every Y row load of a column chunk is issued before any is used.
  bool ok[KT];
  int64_t row[KT];
  float s[KT], acc[KT];
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    const int64_t p = t * KT + j;
    const int e = __builtin_amdgcn_readfirstlane((int)idx[p]);
    ok[j] = e >= 0 && e < E;  // wave-uniform
    row[j] = ok[j] ? (int64_t)__builtin_amdgcn_readfirstlane(inv[p]) : 0;
    s[j] = d_raw != nullptr ? bf16_to_f32(w[p]) : 0.0f;
    acc[j] = 0.0f;
  }
  const uint16_t* dr = dout + t * h;
  for (int c = lane * 8; c < h; c += 512) {
    const u32x4_t a = ld16(dr + c);
    u32x4_t b[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) b[j] = ok[j] ? ld16(Y + row[j] * h + c) : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      if (!ok[j]) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[j] += round_bf16(bf16_to_f32(a[i] & 0xffffu) * bf16_to_f32(b[j][i] & 0xffffu));
        acc[j] += round_bf16(bf16_to_f32(a[i] >> 16) * bf16_to_f32(b[j][i] >> 16));
      }
      if (d_raw != nullptr) {
        u32x4_t v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = pack_bf16x2(bf16_to_f32(a[i] & 0xffffu) * s[j], bf16_to_f32(a[i] >> 16) * s[j]);
        st16(d_raw + row[j] * h + c, v);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    const float r = wave_sum_f(acc[j]);
    if (lane == 0) dw[t * KT + j] = (uint16_t)f32_to_bf16_rne(r);
  }
}

// dst[r] = bf16(src[perm[r] / k] * w[perm[r]]) (w == nullptr: the plain gathered row), rows r in
// expert-sorted order: the gradient of the routed raw rows (dout scaled by the routing weight,
// inference.py:381). Only the rows r < starts[E-1] + counts[E-1] that the permutation filled (pairs
// routed outside [0, E) hold no row); one wave per row.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                          const int32_t* __restrict__ perm,
                                                          const uint16_t* __restrict__ w,
                                                          const int32_t* __restrict__ starts,
                                                          const int32_t* __restrict__ counts,
                                                          uint16_t* __restrict__ dst, int64_t P, int h,
                                                          int E, int k) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  const int64_t filled = (int64_t)starts[E - 1] + counts[E - 1];
  if (r >= P || r >= filled) return;
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

// Expert weight gradients dW[e][m][n] = sum over the rows r of expert e (sorted order, r in
// [starts[e], starts[e] + counts[e])) of G[r][m] * X[src(r)][n], rounded once to bf16; src(r) =
// perm[r] / k (X = the tokens, gathered) or r (X already in sorted order). With G = [d_g | d_u] and
// X = x this is gate_up_proj's gradient [E, 2I, h]; with G = the routed output rows' gradient and
// X = H it is down_proj's [E, h, I] (torch's bf16 mm: fp32 accumulation, one rounding). The
// reduction runs over rows, the strided dimension of both operands.
//
// 32-row slices of G[:, m0 .. m0+255] and X[:, n0 .. n0+255] are copied global -> LDS by
// global_load_lds_dwordx4 into a WD_NS-slot ring (WD_NS - 1 slices in flight, no register
// staging; gathered X rows through an LDS ring of row indices) and the MFMA fragments are read
// straight from the row-major slices with the gfx950 transposing LDS read ds_read_b64_tr_b16:
// within each 16-lane group, component j of lane i is element i % 4 of the 8 bytes that lane
// 4j + i/4 addresses, so lanes addressing rows k0 + s/4, columns c0 + 4 (s % 4) receive rows
// k0 .. k0+3 of column c0 + i; two such reads are one 8-row fragment. Slices are row-major, 512
// bytes per row (256 columns), 16-byte chunk c of row r at chunk c ^ 4 (r % 4): the 32 lanes of a
// half-wave read 4 rows x 64 bytes and cover the 64 banks once. Rows past the
// expert's count are copied from its last row (in bounds) and zeroed in the fragments of the last
// slice; columns past
// M or N are copied from column 0 and never stored. One 512-thread block per 256 (G) x 256 (X)
// tile, one block per CU; each of the 8 waves multiplies 64 x 128 (2 x 4 blocks of
// mfma_f32_32x32x16_bf16, X as the A operand). Against 128 x 256 tiles in two 4-wave blocks per CU
// (the same per-wave work), a slice copies a third fewer bytes per FLOP, which the copies' LDS
// writes had made the limit (gate_up_proj's gradient 137 -> 123 us, down_proj's 63 -> 58 us at
// configuration 2).
constexpr int WD_BK = 32;   // rows per slice
constexpr int WD_NS = 3;    // ring slots (96 KB + the index rings' 6 KB: one block per CU)
constexpr int WD_TN = 256;  // X columns per tile (G columns: WG_T = 256)

__device__ __forceinline__ uint32_t wd_lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
// global_load_lds_dwordx4 from inline asm (M0 = the wave's LDS base; lane l lands at +16 l). The
// compiler does not see these loads: their completion is ordered by the explicit vmcnt waits below.
__device__ __forceinline__ void wd_dma16(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(gsrc)
               : "memory", "m0");
}
__device__ __forceinline__ void wd_dma4(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(gsrc)
               : "memory", "m0");
}
typedef short i16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 wd_read_tr(const uint8_t* lds) {
  const i16x4_t v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(uintptr_t)(
          (const __attribute__((address_space(3))) uint8_t*)lds));
  return __builtin_bit_cast(uint2, v);
}
// Byte offset of (row, col) in a slice of PITCH-byte rows: 16-byte chunk c of row r at c ^ 4 (r % 4).
template <int PITCH>
__device__ __forceinline__ int wd_off(int row, int col) {
  return row * PITCH + 16 * ((col >> 3) ^ (4 * (row & 3))) + 2 * (col & 7);
}

// GX: X rows gathered, X[perm[r] / k] (X = the tokens [T, N]). Each wave copies the 32 row
// indices of slice t into its own LDS ring (global_load_lds_dword, issued two steps before slice
// t's data copies, which read them), so the pipeline holds no compiler-visible loads: every step
// issues the same 5 asynchronous copies per wave (4 data + 1 index) and waits with one constant.
template <bool GX>
__global__ __launch_bounds__(512) void expert_wgrad_dma_kernel(const uint16_t* G, const uint16_t* X,
                                                               const int32_t* perm,
                                                               const int32_t* __restrict__ starts,
                                                               const int32_t* __restrict__ counts,
                                                               uint16_t* __restrict__ dW, int64_t P, int M,
                                                               int N, int k, int tm, int tn) {
  static_assert(!GX || WD_NS == 3, "the index lead below is written for a 3-slot ring");
  __shared__ __align__(16) uint8_t ring_g[WD_NS][WD_BK * 2 * WG_T];   // [slot][row][256 columns]
  __shared__ __align__(16) uint8_t ring_x[WD_NS][WD_BK * 2 * WD_TN];  // [slot][row][256 columns]
  __shared__ __align__(16) int32_t ring_i[GX ? 8 : 1][GX ? 3 : 1][64];  // [wave][slot][row (+32 copies)]
  const int nb = gridDim.x, b = blockIdx.x;
  const int L = (nb & 7) == 0 ? (b & 7) * (nb >> 3) + (b >> 3) : b;
  const int e = L / (tm * tn), rem = L - e * tm * tn;
  const int m0 = (rem / tn) * WG_T, n0 = (rem % tn) * WD_TN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t r0 = P > 0 ? starts[e] : 0;
  const int cnt = P > 0 ? (int)max((int64_t)0, min((int64_t)counts[e], P - r0)) : 0;
  const int nsl = (cnt + WD_BK - 1) / WD_BK;
  // Wave (wm, wn) owns G columns 64 wm .. +63 and X columns 128 wn .. +127 of the tile.
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
  f32x16_t acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;

  if (nsl > 0) {
    // Copies: wave w fills slice rows 4w .. 4w+3 of both operands, each in 2 instructions of 2
    // 512-byte rows (lane l: row 4w + 2q + l/32, position l % 32); position p of row r holds
    // chunk p ^ 4 (r % 4).
    // perm[r] / k as a multiply-high by ceil(2^32 / k) (exact for pair indices below 2^29).
    const uint32_t kmagic = k > 1 ? (uint32_t)((0x100000000ull + (uint32_t)k - 1) / (uint32_t)k) : 0u;
    auto issue_idx = [&](int sl) {  // slice sl's 32 row indices (lanes 32-63 repeat them)
      const int64_t r = r0 + min(sl * WD_BK + (lane & 31), cnt - 1);
      wd_dma4(perm + r, wd_lds_addr(&ring_i[wave][sl % 3][0]));
    };
    auto issue = [&](int sl, const int (&xrow)[4]) {
      const int slot = sl % WD_NS;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int row = 4 * wave + 2 * q + (lane >> 5);
        const int col = m0 + 8 * ((lane & 31) ^ (4 * (row & 3)));
        const int64_t grow = r0 + min(sl * WD_BK + row, cnt - 1);
        wd_dma16(G + grow * M + (col < M ? col : 0), wd_lds_addr(&ring_g[slot][(4 * wave + 2 * q) * 2 * WG_T]));
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int row = 4 * wave + 2 * q + (lane >> 5);
        const int col = n0 + 8 * ((lane & 31) ^ (4 * (row & 3)));
        const int64_t grow = GX ? (int64_t)xrow[q] : r0 + min(sl * WD_BK + row, cnt - 1);
        wd_dma16(X + grow * N + (col < N ? col : 0), wd_lds_addr(&ring_x[slot][(4 * wave + 2 * q) * 2 * WD_TN]));
      }
    };
    // This wave's X source rows of slice sl (rows 8 wave + 2q + lane / 32): from memory for the
    // first two slices (nothing is in flight yet), then from the index ring.
    auto xrows_direct = [&](int sl, int (&xr)[4]) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t pr = (uint32_t)perm[r0 + min(sl * WD_BK + 4 * wave + 2 * q + (lane >> 5), cnt - 1)];
        xr[q] = (int)(k > 1 ? __umulhi(pr, kmagic) : pr);
      }
    };
    auto xrows_ring = [&](int sl, int (&xr)[4]) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t pr = (uint32_t)ring_i[wave][sl % 3][4 * wave + 2 * q + (lane >> 5)];
        xr[q] = (int)(k > 1 ? __umulhi(pr, kmagic) : pr);
      }
    };
    int xr[4] = {0, 0, 0, 0};
    // Prologue: the copies of steps -2 and -1 (data of slices 0 and 1, indices of slices 2 and 3).
#pragma unroll
    for (int sl = 0; sl < WD_NS - 1; ++sl) {
      if (GX) xrows_direct(sl, xr);
      issue(sl, xr);
      if (GX) issue_idx(sl + WD_NS - 1);
    }
    const int g = lane >> 4, gi = lane & 15;
    for (int s = 0; s < nsl; ++s) {
      // This wave's copies issued up to step s-2 (data of slice s, and with GX the indices of
      // slice s+2) are done when at most those of step s-1 are outstanding; the barrier makes that
      // true of every wave and orders the LDS reads of slice s-1 (drained by the lgkmcnt wait)
      // before its slot is refilled with slice s+NS-1.
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((GX ? 5 : 4) * (WD_NS - 2)) : "memory");
      if (GX) xrows_ring(s + WD_NS - 1, xr);
      issue(s + WD_NS - 1, xr);
      if (GX) issue_idx(s + 2 * (WD_NS - 1));
      const uint8_t* sg = ring_g[s % WD_NS];
      const uint8_t* sx = ring_x[s % WD_NS];
      const int left = cnt - s * WD_BK;  // rows of this slice that exist (mask when < 32)
#pragma unroll
      for (int u = 0; u < WD_BK / 16; ++u) {
        u32x4_t gf[2], xf[4];
        const int row = 16 * u + 8 * (g >> 1) + (gi >> 2), colo = 16 * (g & 1) + 4 * (gi & 3);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int cg = 64 * wm + 32 * i + colo;
          const uint2 g0 = wd_read_tr(sg + wd_off<2 * WG_T>(row, cg));
          const uint2 g1 = wd_read_tr(sg + wd_off<2 * WG_T>(row + 4, cg));
          gf[i] = (u32x4_t){g0.x, g0.y, g1.x, g1.y};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int cx = 128 * wn + 32 * i + colo;
          const uint2 x0 = wd_read_tr(sx + wd_off<2 * WD_TN>(row, cx));
          const uint2 x1 = wd_read_tr(sx + wd_off<2 * WD_TN>(row + 4, cx));
          xf[i] = (u32x4_t){x0.x, x0.y, x1.x, x1.y};
        }
        if (left < WD_BK) {  // last, partial slice: rows k >= left are copies of the last row
          const int kb = 16 * u + 8 * lh;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t keep = (kb + 2 * d < left ? 0xffffu : 0u) | (kb + 2 * d + 1 < left ? 0xffff0000u : 0u);
#pragma unroll
            for (int i = 0; i < 2; ++i) gf[i][d] &= keep;
#pragma unroll
            for (int i = 0; i < 4; ++i) xf[i][d] &= keep;
          }
        }
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int mi = 0; mi < 2; ++mi) acc[ni][mi] = mfma32x32x16(xf[ni], gf[mi], acc[ni][mi]);
      }
    }
    // The copies of the NS - 1 slices past the end are still in flight: complete them before the
    // block's LDS can be released.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  // acc[ni][mi][i] of lane l: column n = 128 wn + 32 ni + 8 (i/4) + 4 (l/32) + i%4, row m = 64 wm + 32 mi + l%32.
  uint16_t* const out = dW + (int64_t)e * M * N;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int m = m0 + 64 * wm + 32 * mi + lr;
    if (m >= M) continue;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = n0 + 128 * wn + 32 * ni + 8 * gq + 4 * lh;
        if (n < N)
          *reinterpret_cast<uint2*>(out + (int64_t)m * N + n) =
              make_uint2(pack_bf16x2(acc[ni][mi][4 * gq], acc[ni][mi][4 * gq + 1]),
                         pack_bf16x2(acc[ni][mi][4 * gq + 2], acc[ni][mi][4 * gq + 3]));
      }
  }
}

// 8 x 8 transpose of 16-bit elements held as 8 rows of 16 bytes: b[j] = column j of a.
__device__ __forceinline__ void transpose8x8(const u32x4_t (&a)[8], u32x4_t (&b)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = a[2 * q][j >> 1], hi = a[2 * q + 1][j >> 1];
      b[j][q] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
}

// dst[e] = src[e]^T for bf16 matrices [E, R, C] -> [E, C, R] (the expert weights as the K-major
// operand of the input-gradient products). One wave per 64 x 64 tile: lane l moves the 8 x 8 block
// at source rows 8 (l % 8), columns 8 (l / 8) through registers (8 16-byte loads, transpose8x8,
// 8 16-byte stores), so every load instruction covers 8 source rows x 128 contiguous bytes and
// every store 8 destination rows x 128 bytes: whole lines both ways, no LDS.
__global__ __launch_bounds__(256) void transpose_experts_kernel(const uint16_t* __restrict__ src,
                                                                uint16_t* __restrict__ dst, int E, int R,
                                                                int C) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int tr = R / 64, tc = C / 64;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= (int64_t)E * tr * tc) return;
  const int e = (int)(tile / (tr * tc));
  const int rem = (int)(tile - (int64_t)e * tr * tc);
  const int r0 = (rem / tc) * 64 + 8 * (lane & 7), c0 = (rem % tc) * 64 + 8 * (lane >> 3);
  const uint16_t* s = src + (int64_t)e * R * C + (int64_t)r0 * C + c0;
  uint16_t* d = dst + (int64_t)e * R * C + (int64_t)c0 * R + r0;
  u32x4_t a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = ld16(s + (int64_t)i * C);
  transpose8x8(a, b);
#pragma unroll
  for (int j = 0; j < 8; ++j) st16(d + (int64_t)j * R, b[j]);
}

hipError_t launch_transpose_experts(const uint16_t* src, uint16_t* dst, int E, int R, int C, hipStream_t stream) {
  const int64_t tiles = (int64_t)E * (R / 64) * (C / 64);
  if (tiles == 0) return hipSuccess;
  hipLaunchKernelGGL(transpose_experts_kernel, dim3((unsigned)((tiles + 3) / 4)), dim3(256), 0, stream, src, dst, E,
                     R, C);
  return hipGetLastError();
}

template <typename IdxT>
static hipError_t launch_pair_dots_t(const uint16_t* dout, const uint16_t* Y, const int32_t* inv, const IdxT* idx,
                                     const uint16_t* w, uint16_t* dw, uint16_t* d_raw, int64_t T, int h, int E, int k,
                                     hipStream_t stream) {
  const dim3 grid((unsigned)((T + 3) / 4));
#define Q38_PD(KT)                                                                                              \
  case KT:                                                                                                      \
    hipLaunchKernelGGL((pair_dots_kernel<IdxT, KT>), grid, dim3(256), 0, stream, dout, Y, inv, idx, w, dw, d_raw, \
                       T, h, E);                                                                                \
    break;
  switch (k) {
    Q38_PD(1) Q38_PD(2) Q38_PD(3) Q38_PD(4) Q38_PD(5) Q38_PD(6) Q38_PD(7) Q38_PD(8)
    default: return hipErrorInvalidValue;
  }
#undef Q38_PD
  return hipGetLastError();
}

hipError_t launch_pair_dots(const uint16_t* dout, const uint16_t* Y, const int32_t* inv, const void* idx,
                            bool idx64, const uint16_t* w, uint16_t* dw, uint16_t* d_raw, int64_t T, int h, int E,
                            int k, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (idx64)
    return launch_pair_dots_t(dout, Y, inv, static_cast<const int64_t*>(idx), w, dw, d_raw, T, h, E, k, stream);
  return launch_pair_dots_t(dout, Y, inv, static_cast<const int32_t*>(idx), w, dw, d_raw, T, h, E, k, stream);
}

hipError_t launch_gather_rows(const uint16_t* src, const int32_t* perm, const uint16_t* w, const int32_t* starts,
                              const int32_t* counts, uint16_t* dst, int64_t P, int h, int E, int k,
                              hipStream_t stream) {
  if (P == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((P + 3) / 4)), dim3(256), 0, stream, src, perm, w, starts,
                     counts, dst, P, h, E, k);
  return hipGetLastError();
}

hipError_t launch_expert_wgrad(const uint16_t* G, const uint16_t* X, const int32_t* perm, const int32_t* starts,
                               const int32_t* counts, uint16_t* dW, int64_t P, int E, int M, int N, int k,
                               hipStream_t stream) {
  const int tm = (M + WG_T - 1) / WG_T, tn = (N + WG_T - 1) / WG_T;
  const int64_t nb = (int64_t)E * tm * tn;
  if (nb == 0) return hipSuccess;
  const int tnd = (N + WD_TN - 1) / WD_TN;
  const dim3 grid((unsigned)((int64_t)E * tm * tnd));
  if (perm == nullptr)
    hipLaunchKernelGGL(expert_wgrad_dma_kernel<false>, grid, dim3(512), 0, stream, G, X, perm, starts, counts, dW, P,
                       M, N, k, tm, tnd);
  else
    hipLaunchKernelGGL(expert_wgrad_dma_kernel<true>, grid, dim3(512), 0, stream, G, X, perm, starts, counts, dW, P,
                       M, N, k, tm, tnd);
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
