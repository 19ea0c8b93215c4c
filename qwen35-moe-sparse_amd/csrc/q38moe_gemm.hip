// Grouped expert GEMMs on bf16 MFMA (R5-R7, R9): routed experts and the shared expert in one launch.
//
//   gate/up (MODE_GATE_UP): H[r, n] = bf16(bf16(silu(bf16(a_r.Wg[n]))) * bf16(a_r.Wu[n]))
//     a_r = x[perm[r] / k] for routed rows r < P (the token gather of inference.py:74, 83-84) and
//     a_r = x[r - P] for shared-expert rows. Reference rounding: inference.py:90-96.
//   down (MODE_DOWN):      Y[r, c] = bf16(H[r].Wd[c])  (inference.py:122-127; the routing weight
//     is applied by the combine with the reference's rounding, inference.py:128-130).
// Rows live in one space: [0, P) routed pairs in expert-sorted order, [P, P+T) shared-expert
// tokens; outputs are stored row-contiguous in that order (no scatter).
//
// Weights are [N, K] row-major (experts.gate_up_proj[e], experts.down_proj[e], nn.Linear), so
// both MFMA operands are K-contiguous. Tile: 256 activation rows x 128 weight rows, K in 32-wide
// slices. 4 waves (2x2), each 128 x 64 = 4x2 tiles of 32x32x16 MFMA with the weight fragment as
// the first operand, so lane = activation row and each lane holds runs of 4 consecutive output
// columns. For gate/up, a wave's 64 weight rows are [32 gate | 32 up] of the same 32 output
// columns, so SwiGLU runs in registers. 128 accumulator registers and 72 KiB of LDS per workgroup
// let two workgroups share a CU, so one's prologue/epilogue overlaps the other's MFMA loop.
//
// K-slices are copied global -> LDS asynchronously (global_load_lds_dwordx4) two slices ahead
// into a 3-deep ring; slices are XOR-swizzled (16-byte chunk c of row r at slot
// c ^ ((r >> 2) & 3): conflict-free fragment reads). The epilogue stages 32-row slabs in LDS and
// stores whole 16-byte row chunks. Tiles are spread over the 8 XCDs in contiguous runs
// (workgroup b runs on XCD b % 8 and takes logical tile (b % 8) * per + b / 8), so an expert's
// weights and gathered rows stay in one XCD's L2.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int BM = 256;  // activation rows per tile
constexpr int BN = 128;  // weight rows per tile
constexpr int BK = 32;   // K slice
constexpr int NTHREADS = 256;
constexpr int NSTAGE = 3;                    // LDS ring of K-slices
constexpr int STAGE_ELEMS = (BM + BN) * BK;  // bf16 elements per slice
constexpr int NCOPY = (BM + BN) / 16 / 4;    // async copies per wave per slice (16 rows each)
constexpr int EPI_PITCH = 72;                // epilogue slab row pitch (elements): 64 + 8 pad

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

struct GemmParams {
  const uint16_t* A;          // activations: x [T,h] (gate/up) or H rows (down)
  const int32_t* perm;        // gate/up routed rows: sorted row -> pair (token = pair / topk)
  const int4* tiles;          // {group (E = shared expert), row0, rows, -}; nullptr = dense
  const int32_t* ntiles_dev;  // number of valid entries in tiles (device)
  int ntiles_host;            // dense launch: number of row tiles
  int64_t M;                  // dense launch: rows
  const uint16_t* W;          // routed weights: gate/up [E, 2N, K], down [E, N, K]
  const uint16_t* Ws_a;       // shared expert: gate [N, K] (gate/up) or down [N, K]
  const uint16_t* Ws_b;       // shared expert: up [N, K] (gate/up)
  uint16_t* C;                // output rows [*, N]
  int P;                      // first shared-expert row of the row space
  int N, K, E, topk;
  int ntiles_n;               // weight-row tiles per row tile
};

__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ ((r >> 2) & 3)) << 3); }

template <int MODE>
__global__ __launch_bounds__(NTHREADS, 2) void grouped_gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t ring[NSTAGE * STAGE_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;

  // XCD-aware logical tile.
  const int used_m = p.tiles != nullptr ? *p.ntiles_dev : p.ntiles_host;
  const int used = used_m * p.ntiles_n;
  const int per = (used + 7) >> 3;
  const int jb = (int)(blockIdx.x >> 3);
  if (jb >= per) return;
  const int logical = (int)(blockIdx.x & 7) * per + jb;
  if (logical >= used) return;
  const int mt = logical / p.ntiles_n;
  constexpr int BN_OUT = MODE == MODE_GATE_UP ? BN / 2 : BN;
  const int n0 = (logical - mt * p.ntiles_n) * BN_OUT;

  int grp, row0, nrows;
  if (p.tiles != nullptr) {
    const int4 ti = p.tiles[mt];
    grp = ti.x;
    row0 = ti.y;
    nrows = ti.z;
  } else {
    grp = p.E;
    row0 = mt * BM;
    nrows = (int)min((int64_t)BM, p.M - (int64_t)row0);
  }
  if (nrows <= 0) return;
  const int K = p.K, N = p.N;
  const bool shared_grp = grp >= p.E;

  // Async copy sources. Copy instruction j = NCOPY*wave + q fills 16 rows (1 KiB) of the slice:
  // j < 16 -> activation rows 16j.., else weight rows 16(j-16)... Lane l lands in slot l: row
  // r0 + l/4, position l%4, i.e. 16-byte chunk (l%4) ^ ((row >> 2) & 3). Rows past the tile (or
  // weight rows past N) read a clamped in-bounds row; their results only reach outputs that are
  // never stored.
  const uint16_t* src[NCOPY];
  int prow[NCOPY];
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) {  // gather indices first: one load latency, not NCOPY
    const int j = NCOPY * wave + q;
    const int r = 16 * j + (lane >> 2);
    const int rr = row0 + (r < nrows ? r : 0);
    prow[q] = (j < 16 && MODE == MODE_GATE_UP && !shared_grp) ? p.perm[rr] : rr;
  }
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) {
    const int j = NCOPY * wave + q;
    if (j < 16) {
      const int r = 16 * j + (lane >> 2);
      const int c = (lane & 3) ^ ((r >> 2) & 3);
      int64_t arow = prow[q];
      if (MODE == MODE_GATE_UP) arow = shared_grp ? (int64_t)(prow[q] - p.P) : (int64_t)(prow[q] / p.topk);
      src[q] = p.A + arow * K + c * 8;
    } else {
      const int r = 16 * (j - 16) + (lane >> 2);
      const int c = (lane & 3) ^ ((r >> 2) & 3);
      const uint16_t* base;
      int col;
      if (MODE == MODE_GATE_UP) {
        // Weight rows of wave column w: [32 gate | 32 up] for output columns n0 + 32w + 0..31.
        const int half = r >> 6, within = r & 63;
        const bool up = within >= 32;
        col = n0 + 32 * half + (within & 31);
        if (shared_grp) base = up ? p.Ws_b : p.Ws_a;
        else base = p.W + (int64_t)grp * 2 * N * K + (up ? (int64_t)N * K : 0);
      } else {
        col = n0 + r;
        base = shared_grp ? p.Ws_a : p.W + (int64_t)grp * N * K;
      }
      src[q] = base + (int64_t)(col < N ? col : 0) * K + c * 8;
    }
  }
  const int dst0 = NCOPY * wave * 16 * BK;  // element offset of this wave's first copy

  f32x16_t acc[2][4];
#pragma unroll
  for (int ni = 0; ni < 2; ++ni)
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[ni][mi][i] = 0.0f;

  const int nk = K / BK;
#define Q38_ISSUE(KT)                                                                 \
  do {                                                                                \
    uint16_t* st_ = ring + ((KT) % NSTAGE) * STAGE_ELEMS + dst0;                      \
    const int ko_ = (KT) * BK;                                                        \
    _Pragma("unroll") for (int q_ = 0; q_ < NCOPY; ++q_)                              \
      load_lds16(src[q_] + ko_, st_ + q_ * 16 * BK);                                  \
  } while (0)

  // Step kt: wait for this wave's copies of slice kt, barrier (publishes slice kt, retires the
  // slot of slice kt-1; raw s_barrier, as __syncthreads() would also drain the copy still in
  // flight), copy slice kt+2 into that slot, multiply slice kt.
  Q38_ISSUE(0);
  if (nk > 1) Q38_ISSUE(1);
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (kt + 2 < nk) Q38_ISSUE(kt + 2);
    const uint16_t* as_ = ring + (kt % NSTAGE) * STAGE_ELEMS;
    const uint16_t* bs_ = as_ + BM * BK;
    u32x4_t wf[2][2], af[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = 2 * kk + lh;
#pragma unroll
      for (int t = 0; t < 2; ++t) wf[kk][t] = ld16(bs_ + swz(64 * wn + 32 * t + lr, c));
#pragma unroll
      for (int t = 0; t < 4; ++t) af[kk][t] = ld16(as_ + swz(128 * wm + 32 * t + lr, c));
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) acc[ni][mi] = mfma32x32x16(wf[kk][ni], af[kk][mi], acc[ni][mi]);
  }
#undef Q38_ISSUE
  __syncthreads();

  // Epilogue: per 32-row slab (mi), lanes write runs of 4 columns to a wave-private LDS slab,
  // then the wave stores whole 16-byte row chunks.
  constexpr int NW = MODE == MODE_GATE_UP ? 32 : 64;  // output columns per wave
  constexpr int NT_OUT = NW / 32;                      // 32-column output tiles per wave
  constexpr int CPR = NW / 8;                          // 16-byte chunks per slab row
  constexpr int RPI = 64 / CPR;                        // slab rows per store instruction
  uint16_t* slab = ring + wave * (32 * EPI_PITCH);
  const int col_wave = n0 + NW * wn;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int nt = 0; nt < NT_OUT; ++nt) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t packed[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          uint32_t v2 = 0;
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {
            const int i = 4 * q + 2 * h2 + e2;
            float v;
            if (MODE == MODE_GATE_UP) {
              const float g = round_bf16(acc[0][mi][i]);
              const float u = round_bf16(acc[1][mi][i]);
              v = round_bf16(g * __builtin_amdgcn_rcpf(1.0f + __expf(-g))) * u;
            } else {
              v = acc[nt][mi][i];
            }
            v2 |= f32_to_bf16_rne(v) << (16 * e2);
          }
          packed[h2] = v2;
        }
        const int col = 32 * nt + 8 * q + 4 * lh;
        *reinterpret_cast<uint2*>(slab + lr * EPI_PITCH + col) = make_uint2(packed[0], packed[1]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < 32 / RPI; ++s) {
      const int rl = s * RPI + lane / CPR;
      const int cc = (lane % CPR) * 8;
      const int r = 128 * wm + 32 * mi + rl;
      const u32x4_t v = ld16(slab + rl * EPI_PITCH + cc);
      if (r < nrows && col_wave + cc < N) st16(p.C + (int64_t)(row0 + r) * N + col_wave + cc, v);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

int gemm_block_m() { return BM; }

static unsigned grid_for(int max_mtiles, int ntiles_n) {
  const int64_t g = (int64_t)max_mtiles * ntiles_n;
  return (unsigned)((g + 7) / 8 * 8);
}

hipError_t launch_gate_up(const uint16_t* x, const int32_t* perm, const int4* tiles,
                          const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                          const uint16_t* w_gate_up, const uint16_t* ws_gate,
                          const uint16_t* ws_up, uint16_t* H, int N, int K, int E, int topk,
                          hipStream_t stream) {
  GemmParams p;
  p.A = x;
  p.perm = perm;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.ntiles_host = tiles != nullptr ? 0 : (int)((M_dense + BM - 1) / BM);
  p.M = M_dense;
  p.W = w_gate_up;
  p.Ws_a = ws_gate;
  p.Ws_b = ws_up;
  p.C = H;
  p.P = P;
  p.N = N;
  p.K = K;
  p.E = E;
  p.topk = topk;
  p.ntiles_n = (N + BN / 2 - 1) / (BN / 2);
  const int mt = tiles != nullptr ? max_mtiles : p.ntiles_host;
  if (mt == 0) return hipSuccess;
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_GATE_UP>, dim3(grid_for(mt, p.ntiles_n)),
                     dim3(NTHREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_down(const uint16_t* H, const int4* tiles, const int32_t* ntiles_dev,
                       int max_mtiles, int64_t M_dense, const uint16_t* w_down,
                       const uint16_t* ws_down, uint16_t* Y, int N, int K, int E,
                       hipStream_t stream) {
  GemmParams p;
  p.A = H;
  p.perm = nullptr;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.ntiles_host = tiles != nullptr ? 0 : (int)((M_dense + BM - 1) / BM);
  p.M = M_dense;
  p.W = w_down;
  p.Ws_a = ws_down;
  p.Ws_b = nullptr;
  p.C = Y;
  p.P = 0;
  p.N = N;
  p.K = K;
  p.E = E;
  p.topk = 1;
  p.ntiles_n = (N + BN - 1) / BN;
  const int mt = tiles != nullptr ? max_mtiles : p.ntiles_host;
  if (mt == 0) return hipSuccess;
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE_DOWN>, dim3(grid_for(mt, p.ntiles_n)), dim3(NTHREADS),
                     0, stream, p);
  return hipGetLastError();
}

}  // namespace q38
