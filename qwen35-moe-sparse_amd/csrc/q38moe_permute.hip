// Token->expert permutation (R3-R4): per-block histogram, expert prefix sums and a stable
// counting-sort scatter (perm and its inverse), plus the padded tile table of the grouped GEMMs.
//
// Reference semantics (q38/inference.py:163-171, 39-50, 174-183): perm is
// torch.sort(ids, stable=True).indices over the flattened pair ids (pair p = t*k + j),
// starts/counts are the expert boundaries in sorted order. Here the sort is a counting sort:
// perm[starts[e] + r] = the r-th pair (ascending p) routed to e. Every block of 64 tokens derives
// its base offsets from the per-block histograms, so the scatter needs no atomics and the order is
// deterministic.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int PERM_TOKENS = 64;  // tokens per histogram block (matches the router's blocks)
constexpr int PERM_KMAX = 8;

template <typename IdxT>
__global__ __launch_bounds__(256) void hist_kernel(const IdxT* __restrict__ idx, int64_t T, int E,
                                                   int k, int32_t* __restrict__ hist) {
  __shared__ int s_h[64];
  const int tid = threadIdx.x;
  if (tid < 64) s_h[tid] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * PERM_TOKENS;
  const int64_t t1 = min(t0 + PERM_TOKENS, T);
  const int np = (int)((t1 - t0) * k);
  for (int i = tid; i < np; i += 256) {
    const int64_t e = (int64_t)idx[t0 * k + i];
    if (e >= 0 && e < E) atomicAdd(&s_h[(int)e], 1);
  }
  __syncthreads();
  if (tid < E) hist[(int64_t)blockIdx.x * E + tid] = s_h[tid];
}

template <typename IdxT>
__global__ __launch_bounds__(256) void permute_kernel(
    const IdxT* __restrict__ idx, const int32_t* __restrict__ hist, int64_t T, int E, int k,
    int nblk, int32_t* __restrict__ counts, int32_t* __restrict__ starts,
    int32_t* __restrict__ perm, int32_t* __restrict__ inv, int4* __restrict__ tiles,
    int32_t* __restrict__ tile_count, int block_m, int max_tiles, int shared_rows,
    const float* __restrict__ row_scale_in, float* __restrict__ row_scale_out) {
  constexpr int NCHUNK = PERM_TOKENS * PERM_KMAX / 64;  // 64-pair chunks per block (<= 8)
  __shared__ int s_tot[4][64];
  __shared__ int s_bef[4][64];
  __shared__ int s_start[64];
  __shared__ int s_total[64];
  __shared__ int s_tile0[64];
  __shared__ int s_ntile[64];
  __shared__ int s_ccnt[NCHUNK][64];  // pairs per expert in each chunk, then the chunk's offsets
  const int tid = threadIdx.x, e = tid & 63, part = tid >> 6;
  const int lane = e, wave = part;
  const int b = blockIdx.x;
  for (int i = tid; i < NCHUNK * 64; i += 256) (&s_ccnt[0][0])[i] = 0;

  // This block's pairs p0 + i, i = 64 c + lane for chunks c = wave, wave + 4: loaded first, so that
  // their round trip overlaps the histogram scan's (they do not depend on it).
  const int64_t t0 = (int64_t)b * PERM_TOKENS;
  const int64_t t1 = min(t0 + PERM_TOKENS, T);
  const int np = (int)((t1 - t0) * k);
  const int64_t p0 = t0 * k;
  const int nchunk = (np + 63) / 64;
  int64_t vload[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = 64 * (wave + 4 * j) + lane;
    vload[j] = i < np ? (int64_t)idx[p0 + i] : (int64_t)-1;
  }

  // Expert totals over all blocks and the counts of the blocks before this one. Thread `tid`
  // sums column e over rows part, part + 4, ...; up to 64 independent loads are in flight per
  // step (a wave's load is one contiguous 256-byte row), so the 256 rows of the benchmark's
  // 16384 tokens take one round trip to L2.
  int tot = 0, bef = 0;
  if (e < E) {
    int bb = part;
    for (; bb + 252 < nblk; bb += 256) {
      int c[64];
#pragma unroll
      for (int u = 0; u < 64; ++u) c[u] = hist[(int64_t)(bb + 4 * u) * E + e];
#pragma unroll
      for (int u = 0; u < 64; ++u) {
        tot += c[u];
        if (bb + 4 * u < b) bef += c[u];
      }
    }
    for (; bb + 60 < nblk; bb += 64) {
      int c[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) c[u] = hist[(int64_t)(bb + 4 * u) * E + e];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        tot += c[u];
        if (bb + 4 * u < b) bef += c[u];
      }
    }
    for (; bb < nblk; bb += 4) {
      const int c = hist[(int64_t)bb * E + e];
      tot += c;
      if (bb < b) bef += c;
    }
  }
  s_tot[part][e] = tot;
  s_bef[part][e] = bef;

  // This block's pairs in chunks of 64 (pair p0 + 64c + lane), chunk c on wave c % 4. A pair's
  // rank among the earlier pairs of its chunk with the same expert is a popcount of the lanes
  // below it in the mask of equal ids, built from one ballot per id bit (ids 0..63, 64 = dropped:
  // out of range or past the block's pairs, like transformers' grouped_mm, moe.py:405-420).
  int cv[2], crank[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = wave + 4 * j;
    cv[j] = 64;
    crank[j] = 0;
    if (c < nchunk) {  // wave-uniform
      const int64_t v = vload[j];  // -1 past the block's pairs
      if (v >= 0 && v < E) cv[j] = (int)v;
      uint64_t same = ~0ull;
#pragma unroll
      for (int bit = 0; bit < 7; ++bit) {
        const bool on = (cv[j] >> bit) & 1;
        const uint64_t m = ballot64(on);
        same &= on ? m : ~m;
      }
      crank[j] = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
      if (cv[j] < 64 && crank[j] == 0) s_ccnt[c][cv[j]] = __popcll(same);
    }
  }
  __syncthreads();

  if (tid < 64) {
    const int t = s_tot[0][tid] + s_tot[1][tid] + s_tot[2][tid] + s_tot[3][tid];
    const int bf = s_bef[0][tid] + s_bef[1][tid] + s_bef[2][tid] + s_bef[3][tid];
    int incl = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int nb = __shfl_up(incl, o);
      if (tid >= o) incl += nb;
    }
    const int st = incl - t;
    s_start[tid] = st;
    s_total[tid] = t;
    // Offset of each chunk's first pair of expert tid: this block's base (the stable counting
    // sort's position), plus the pairs of the block's earlier chunks.
    int off = st + bf;
    for (int c = 0; c < nchunk; ++c) {
      const int n = s_ccnt[c][tid];
      s_ccnt[c][tid] = off;
      off += n;
    }
    // Full tiles per expert and their prefix (the blk_cum of inference.py:176 splits into these
    // and one partial tile per expert with a remainder).
    const int nt = (tid < E) ? t / block_m : 0;
    int tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int nb = __shfl_up(tincl, o);
      if (tid >= o) tincl += nb;
    }
    s_ntile[tid] = nt;
    s_tile0[tid] = tincl - nt;
    if (b == 0 && tid < E) {
      counts[tid] = t;
      starts[tid] = st;
    }
  }
  __syncthreads();

  // Scatter: perm[off] = pair, inv[pair] = off. perm holds T*k entries; the bound only matters
  // for a hist inconsistent with idx.
  const int64_t cap = T * k;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = wave + 4 * j;
    if (c < nchunk && cv[j] < 64) {
      const int off = s_ccnt[c][cv[j]] + crank[j];
      const int64_t pair = p0 + 64 * c + lane;
      if (off < cap) {
        perm[off] = (int32_t)pair;
        if (inv != nullptr) inv[pair] = off;
        // fp8 path: the token's quantisation scale follows its row into sorted order.
        if (row_scale_out != nullptr) row_scale_out[off] = row_scale_in[pair / k];
      }
    }
  }

  // fp8 path: shared-expert rows P + t take token t's scale.
  if (row_scale_out != nullptr && tid < t1 - t0 && t0 + tid < shared_rows)
    row_scale_out[cap + t0 + tid] = row_scale_in[t0 + tid];

  if (tiles != nullptr) {
    // Tile table, in the order the persistent grouped GEMM walks it: every full tile (block_m
    // rows) by expert, then the shared-expert rows [P, P + shared_rows) (group id E), then one
    // partial tile per group with a remainder, by falling row count (ties: lower group first),
    // then unused entries {-1, 0, 0, 0}. Cost falls along the list, so round-robin assignment
    // balances the workgroups. Every block knows every group's totals, so the table is built in
    // parallel: block b writes the entries of groups b, b + grid, ... (group E = the shared rows),
    // block 0 the count and the unused entries.
    const int routed_full = s_tile0[63] + s_ntile[63];
    const int shared_full = shared_rows / block_m;
    const int full = routed_full + shared_full;
    const int64_t P = T * k;
    // Remainder (partial-tile rows) of group `tid`, for the ranks below.
    const int h = tid;
    const int rem_h = h < E ? s_total[h] % block_m : (h == E ? shared_rows % block_m : 0);
    const int npartial = __syncthreads_count(h <= E && rem_h > 0);
    for (int g = b; g <= E; g += (int)gridDim.x) {  // block-uniform
      const int rem = g < E ? s_total[g] % block_m : shared_rows % block_m;
      // Rank of group g's partial tile among all partial tiles.
      const int rank = __syncthreads_count(h <= E && rem_h > 0 && (rem_h > rem || (rem_h == rem && h < g)));
      if (tid == 0 && rem > 0) {
        const int row_start = g < E ? s_start[g] + s_ntile[g] * block_m : (int)P + shared_full * block_m;
        tiles[full + rank] = make_int4(g, row_start, rem, 0);
      }
      if (g < E) {
        for (int j = tid; j < s_ntile[g]; j += 256)
          tiles[s_tile0[g] + j] = make_int4(g, s_start[g] + j * block_m, block_m, 0);
      } else {
        for (int j = tid; j < shared_full; j += 256)
          tiles[routed_full + j] = make_int4(E, (int)P + j * block_m, block_m, 0);
      }
    }
    if (b == 0) {
      if (tid == 0 && tile_count != nullptr) *tile_count = full + npartial;
      for (int i = full + npartial + tid; i < max_tiles; i += 256) tiles[i] = make_int4(-1, 0, 0, 0);
    }
  }
}

hipError_t launch_histogram(const void* idx, bool idx64, int32_t* hist, int64_t T, int E, int k,
                            hipStream_t stream) {
  const int64_t nblk = (T + PERM_TOKENS - 1) / PERM_TOKENS;
  if (nblk == 0) return hipSuccess;
  if (idx64)
    hipLaunchKernelGGL(hist_kernel<int64_t>, dim3((unsigned)nblk), dim3(256), 0, stream,
                       (const int64_t*)idx, T, E, k, hist);
  else
    hipLaunchKernelGGL(hist_kernel<int32_t>, dim3((unsigned)nblk), dim3(256), 0, stream,
                       (const int32_t*)idx, T, E, k, hist);
  return hipGetLastError();
}

hipError_t launch_permute(const void* idx, bool idx64, const int32_t* hist, int32_t* counts,
                          int32_t* starts, int32_t* perm, int32_t* inv, int4* tiles,
                          int32_t* tile_count, int block_m, int max_tiles, int shared_rows,
                          int64_t T, int E, int k, hipStream_t stream, const float* row_scale_in,
                          float* row_scale_out) {
  // At least one block, so T == 0 still writes zero counts and an empty tile table; with a tile
  // table at least E + 1 blocks, one per group's entries (blocks past the pairs' own only write
  // those): fewer would walk several groups each, one after another (at T <= 64, a single block
  // wrote all 65 groups' entries in about 25 us).
  const int64_t nblk = (T + PERM_TOKENS - 1) / PERM_TOKENS;
  int64_t g = nblk > 0 ? nblk : 1;
  if (tiles != nullptr && g < E + 1) g = E + 1;
  const unsigned grid = (unsigned)g;
  if (idx64)
    hipLaunchKernelGGL(permute_kernel<int64_t>, dim3(grid), dim3(256), 0, stream,
                       (const int64_t*)idx, hist, T, E, k, (int)nblk, counts, starts, perm, inv,
                       tiles, tile_count, block_m, max_tiles, shared_rows, row_scale_in, row_scale_out);
  else
    hipLaunchKernelGGL(permute_kernel<int32_t>, dim3(grid), dim3(256), 0, stream,
                       (const int32_t*)idx, hist, T, E, k, (int)nblk, counts, starts, perm, inv,
                       tiles, tile_count, block_m, max_tiles, shared_rows, row_scale_in, row_scale_out);
  return hipGetLastError();
}

}  // namespace q38
