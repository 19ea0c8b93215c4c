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

constexpr int WG_T = 128;              // weight-gradient output tile (rows and columns)
constexpr int WG_K = 64;               // sorted rows per LDS slice
constexpr int WG_PITCH = 2 * WG_K;     // bytes per staged column: 64 bf16 in 8 16-byte chunks

// LDS byte offset of 16-byte row chunk q (0..7) of staged column c. Columns 2p and 2p+1 share a
// 256-byte line of 16 chunk slots; slot (8 (c & 1) + q) ^ key(p), key(p) = ((p >> 2) ^ (p & 7)) & 15.
// The LDS serves a 16-byte access 16 lanes per pass over its 64 banks (16 slots of 16 bytes), and
// both access patterns fill all 16 slots per pass: the transpose writes (16 lanes = 16 column
// blocks 8cb + j, one chunk: key runs over 16 values with cb) and the fragment reads (16 lanes = 16
// consecutive columns, one chunk: c & 1 and the low 3 key bits run over 2 x 8 values).
__device__ __forceinline__ int wg_slot(int c, int q) {
  const int p = c >> 1;
  return p * 256 + 16 * (((c & 1) * 8 + q) ^ (((p >> 2) ^ (p & 7)) & 15));
}

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
// X = H it is down_proj's [E, h, I] (torch's bf16 mm: fp32 accumulation, one rounding). The sorted
// form runs expert_wgrad_dma_kernel (below); this kernel is the gathered form.
//
// The reduction runs over rows, which are the strided dimension of both operands, so each 64-row
// slice is transposed on its way into LDS: a thread loads an 8 x 8 block (8 rows, 16 bytes each),
// transposes it in registers and writes 8 column-major 16-byte runs, after which the MFMA
// fragments (8 consecutive rows of one column) are single 16-byte LDS reads, without bank
// conflicts on either side (wg_slot). One 256-thread block
// per 128 x 128 output tile: waves 0-1 stage G, waves 2-3 stage X, every wave multiplies a 64 x 64
// quarter (2 x 2 blocks of mfma_f32_32x32x16_bf16, X as the A operand so that a lane's
// accumulators are 4 consecutive output columns).
// Two LDS stages and two register stages (below).
// Blocks are numbered so that the tiles of one expert run on one XCD (workgroups go to the 8 XCDs
// round robin) and share its L2.
__device__ __forceinline__ void transpose8x8(const u32x4_t (&a)[8], u32x4_t (&b)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = a[2 * q][j >> 1], hi = a[2 * q + 1][j >> 1];
      b[j][q] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
}

// G, X and perm are not declared __restrict__: loads from restrict read-only arguments count as
// unclobbered and may be moved across the workgroup barriers, which undoes the slice pipeline.
__global__ __launch_bounds__(256) void expert_wgrad_kernel(const uint16_t* G, const uint16_t* X,
                                                           const int32_t* perm,
                                                           const int32_t* __restrict__ starts,
                                                           const int32_t* __restrict__ counts,
                                                           uint16_t* __restrict__ dW, int64_t P, int M,
                                                           int N, int k, int tm, int tn) {
  __shared__ __align__(16) uint8_t lds[2][2][WG_T * WG_PITCH];  // [stage][G, X][column][row]
  const int nb = gridDim.x, b = blockIdx.x;
  const int L = (nb & 7) == 0 ? (b & 7) * (nb >> 3) + (b >> 3) : b;
  const int e = L / (tm * tn), rem = L - e * tm * tn;
  const int m0 = (rem / tn) * WG_T, n0 = (rem % tn) * WG_T;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Rows of expert e, kept inside the P sorted rows (P = 0: no rows, counts never read).
  const int64_t r0 = P > 0 ? starts[e] : 0;
  const int cnt = P > 0 ? (int)max((int64_t)0, min((int64_t)counts[e], P - r0)) : 0;
  const int nsl = (cnt + WG_K - 1) / WG_K;

  const int st = tid & 127, cb = st & 15, rb = st >> 4;
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lh = lane >> 5;
  f32x16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;
  auto compute = [&](int buf) {
    // Fragment of column 64w + 32i + lr, k-chunk 2s + lh.
#pragma unroll
    for (int s = 0; s < WG_K / 16; ++s) {
      u32x4_t gf[2], xf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        gf[i] = *reinterpret_cast<const u32x4_t*>(lds[buf][0] + wg_slot(64 * wm + 32 * i + lr, 2 * s + lh));
        xf[i] = *reinterpret_cast<const u32x4_t*>(lds[buf][1] + wg_slot(64 * wn + 32 * i + lr, 2 * s + lh));
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) acc[ni][mi] = mfma32x32x16(xf[ni], gf[mi], acc[ni][mi]);
    }
  };

  // Staging role (a compile-time constant inside `run`, so that neither role branches around the
  // other's loads): an 8-row x 8-column block of G (waves 0-1) or X (waves 2-3) per thread.
  //
  // Every global load is issued unconditionally from a clamped in-bounds address (rows past the
  // expert's count read its last row, columns past the edge column 0) and its result is always
  // consumed: the zero mask is applied at the transpose. With a fixed number of loads per slice,
  // the compiler's vmcnt waits count only the loads that are needed (a load under a branch makes
  // it wait for all of them).
  //
  // Pipeline: while slice s is multiplied from LDS, slice s+1 (loaded during the previous slice)
  // waits in registers for its transpose into the other LDS stage, slice s+2's loads are in flight
  // and slice s+3's gathered row indices are being fetched: a load has two slices of MFMA work to
  // arrive in. Register sets alternate between even and odd slices; slices past the last one are
  // masked to zero (the last two steps write such a slice into the stage that is no longer read).
  // perm[r] / k as a multiply-high by ceil(2^32 / k): exact for every pair index below 2^29
  // (the error term p * (ceil(2^32/k) * k - 2^32) / (k 2^32) stays below 1/k), and pair indices
  // are below 2^25 here (P * 64 < 2^31).
  const uint32_t kmagic = k > 1 ? (uint32_t)((0x100000000ull + (uint32_t)k - 1) / (uint32_t)k) : 0u;
  auto run = [&](auto role) {
    constexpr bool XR = decltype(role)::value;
    const int col = (XR ? n0 : m0) + 8 * cb;
    const bool col_ok = col < (XR ? N : M);
    const int col_ld = col_ok ? col : 0;
    const uint16_t* const base = XR ? X : G;
    const int ld = XR ? N : M;
    auto rows_of = [&](int sl, int (&src)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rr = min(sl * WG_K + 8 * rb + i, cnt - 1);
        if (XR) {
          const uint32_t pr = (uint32_t)perm[r0 + rr];
          src[i] = (int)(k > 1 ? __umulhi(pr, kmagic) : pr);
        } else {
          src[i] = (int)r0 + rr;
        }
      }
    };
    auto load = [&](const int (&src)[8], u32x4_t (&v)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = ld16(base + (int64_t)src[i] * ld + col_ld);
    };
    auto store = [&](int buf, int sl, const u32x4_t (&v)[8]) {
      u32x4_t w[8], t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        w[i] = col_ok && sl * WG_K + 8 * rb + i < cnt ? v[i] : (u32x4_t){0u, 0u, 0u, 0u};
      transpose8x8(w, t);
      // Columns 8cb + j, row chunk rb.
      uint8_t* dst = lds[buf][XR ? 1 : 0];
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4_t*>(dst + wg_slot(8 * cb + j, rb)) = t[j];
    };
    u32x4_t va[8], vb[8];
    int pa[8], pb[8];
    auto step = [&](int s, u32x4_t (&r1)[8], u32x4_t (&r2)[8], int (&p1)[8], int (&p2)[8]) {
      rows_of(s + 3, p2);
      load(p1, r2);
      compute(s & 1);
      store((s + 1) & 1, s + 1, r1);
      __syncthreads();
    };
    if (nsl == 0) return;
    // The prologue leaves the same loads outstanding, in the same order, as the loop's back edge
    // (slice 2's row indices, then slice 1's data), and the loop always runs whole pairs of steps
    // (an odd count multiplies one zero slice more), so the waits at the loop head stay partial.
    rows_of(0, pa);
    rows_of(1, pb);
    load(pa, va);
    rows_of(2, pa);
    load(pb, vb);
    store(0, 0, va);
    __syncthreads();
    for (int s = 0; s < nsl; s += 2) {
      step(s, vb, va, pa, pb);
      step(s + 1, va, vb, pb, pa);
    }
  };
  if (wave >= 2) run(std::true_type{});
  else run(std::false_type{});

  // acc[ni][mi][i] of lane l: column n = 64wn + 32ni + 8(i/4) + 4(l/32) + i%4, row m = 64wm + 32mi + l%32.
  uint16_t* const out = dW + (int64_t)e * M * N;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int m = m0 + 64 * wm + 32 * mi + lr;
    if (m >= M) continue;
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = n0 + 64 * wn + 32 * ni + 8 * gq + 4 * lh;
        if (n < N)
          *reinterpret_cast<uint2*>(out + (int64_t)m * N + n) =
              make_uint2(pack_bf16x2(acc[ni][mi][4 * gq], acc[ni][mi][4 * gq + 1]),
                         pack_bf16x2(acc[ni][mi][4 * gq + 2], acc[ni][mi][4 * gq + 3]));
      }
  }
}

// Sorted-row form of the weight gradients with asynchronous staging: both operands' rows are in
// sorted order (X = H, or the tokens already gathered into sorted order), so 32-row slices of
// G[:, m0 .. m0+127] and X[:, n0 .. n0+127] are copied global -> LDS by global_load_lds_dwordx4 into
// a WD_NS-slot ring (WD_NS - 1 slices in flight, no register staging) and the MFMA fragments are read
// straight from the row-major slices with the gfx950 transposing LDS read ds_read_b64_tr_b16:
// within each 16-lane group, component j of lane i is element i % 4 of the 8 bytes that lane
// 4j + i/4 addresses, so lanes addressing rows k0 + s/4, columns c0 + 4 (s % 4) receive rows
// k0 .. k0+3 of column c0 + i; two such reads are one 8-row fragment. Slices are row-major, 256
// or 512 bytes per row (128 or 256 columns), 16-byte chunk c of row r at chunk c ^ 4 (r % 4): the
// 32 lanes of a half-wave read 4 rows x 64 bytes and cover the 64 banks once. Rows past the expert's count are
// copied from its last row (in bounds) and zeroed in the fragments of the last slice; columns past
// M or N are copied from column 0 and never stored. One 256-thread block per 128 (G) x 256 (X)
// tile; each wave multiplies 64 x 128 (2 x 4 blocks of mfma_f32_32x32x16_bf16, X as the A operand).
constexpr int WD_BK = 32;   // rows per slice
constexpr int WD_NS = 3;    // ring slots (72 KB: two blocks per CU)
constexpr int WD_TN = 256;  // X columns per tile (G columns: WG_T = 128)

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

__global__ __launch_bounds__(256) void expert_wgrad_dma_kernel(const uint16_t* G, const uint16_t* X,
                                                               const int32_t* __restrict__ starts,
                                                               const int32_t* __restrict__ counts,
                                                               uint16_t* __restrict__ dW, int64_t P, int M,
                                                               int N, int tm, int tn) {
  __shared__ __align__(16) uint8_t ring_g[WD_NS][WD_BK * 2 * WG_T];   // [slot][row][128 columns]
  __shared__ __align__(16) uint8_t ring_x[WD_NS][WD_BK * 2 * WD_TN];  // [slot][row][256 columns]
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
    // Copies: wave w fills slice rows 8w .. 8w+7 of both operands: G in 2 instructions of 4
    // 256-byte rows (lane l: row 4q + l/16, position l % 16), X in 4 instructions of 2 512-byte
    // rows (lane l: row 2q + l/32, position l % 32); position p of row r holds chunk p ^ 4 (r % 4).
    auto issue = [&](int sl) {
      const int slot = sl % WD_NS;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int row = 8 * wave + 4 * q + (lane >> 4);
        const int col = m0 + 8 * ((lane & 15) ^ (4 * (row & 3)));
        const int64_t grow = r0 + min(sl * WD_BK + row, cnt - 1);
        wd_dma16(G + grow * M + (col < M ? col : 0), wd_lds_addr(&ring_g[slot][(8 * wave + 4 * q) * 2 * WG_T]));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = 8 * wave + 2 * q + (lane >> 5);
        const int col = n0 + 8 * ((lane & 31) ^ (4 * (row & 3)));
        const int64_t grow = r0 + min(sl * WD_BK + row, cnt - 1);
        wd_dma16(X + grow * N + (col < N ? col : 0), wd_lds_addr(&ring_x[slot][(8 * wave + 2 * q) * 2 * WD_TN]));
      }
    };
#pragma unroll
    for (int sl = 0; sl < WD_NS - 1; ++sl) issue(sl);
    const int g = lane >> 4, gi = lane & 15;
    for (int s = 0; s < nsl; ++s) {
      // This wave's copies of slice s are done when at most those of slices s+1 .. s+NS-2 (6
      // each) are outstanding; the barrier makes that true of every wave and orders the LDS reads
      // of slice s-1 (drained by the lgkmcnt wait) before its slot is refilled with slice s+NS-1.
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(6 * (WD_NS - 2)) : "memory");
      issue(s + WD_NS - 1);
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
  if (perm == nullptr) {
    const int tnd = (N + WD_TN - 1) / WD_TN;
    hipLaunchKernelGGL(expert_wgrad_dma_kernel, dim3((unsigned)((int64_t)E * tm * tnd)), dim3(256), 0, stream, G, X,
                       starts, counts, dW, P, M, N, tm, tnd);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(expert_wgrad_kernel, dim3((unsigned)nb), dim3(256), 0, stream, G, X, perm, starts, counts, dW, P,
                     M, N, k, tm, tn);
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
