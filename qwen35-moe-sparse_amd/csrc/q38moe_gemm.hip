// Grouped expert GEMMs on bf16 MFMA (R5-R7, R9): routed experts and the shared expert in one launch.
//
//   gate/up (MODE_GATE_UP): H[r, n] = bf16(bf16(silu(bf16(a_r.Wg[n]))) * bf16(a_r.Wu[n]))
//     a_r = x[perm[r] / k] for routed rows r < P (the token gather of inference.py:74, 83-84) and
//     a_r = x[r - P] for shared-expert rows. Reference rounding: inference.py:90-96.
//   down (MODE_DOWN):      Y[r, c] = bf16(H[r].Wd[c])  (inference.py:122-127; the routing weight
//     is applied by the combine with the reference's rounding, inference.py:128-130).
//   gathered (MODE_GATHER): C[r, c] = bf16(a_r.W[c]) with a_r gathered as for gate/up and the weight
//     rows plain, as for down: the experts backward's recomputation of the gate/up pre-activations
//     (W = gate_up_proj[e], 2I output columns).
// Rows live in one space: [0, P) routed pairs in expert-sorted order, [P, P+T) shared-expert
// tokens; outputs are stored row-contiguous in that order (no scatter).
//
// Weights are [N, K] row-major (experts.gate_up_proj[e], experts.down_proj[e], nn.Linear), so
// both MFMA operands are K-contiguous. One down instantiation (WKN) takes them K-major, [K, N]: the
// experts backward multiplies by gate_up_proj[e] and down_proj[e] themselves (dx rows, dH), and
// reads them as stored through the transposing LDS read instead of transposing them first. A tile
// is 256 activation rows x 256 weight rows; K runs in 32-wide slices. One 512-thread workgroup per
// CU (8 waves, two per SIMD); wave w owns activation rows 64*(w/2).. and weight rows 128*(w%2)..,
// i.e. 2x4 blocks of mfma_f32_32x32x16_bf16 with the weight fragment as the first operand, so
// lane = activation row and each lane holds runs of 4 consecutive output columns. For gate/up a wave's 128 weight rows are [64 gate | 64 up] of the
// same 64 output columns, so SwiGLU runs in registers. Waves whose 64 rows are all past the
// tile's row count skip their MFMAs; rows are paired across SIMDs (waves 0-3 hold rows 0-127), so
// a tile of <= 128 rows costs half a full one.
//
// The kernel is persistent: workgroup b walks tiles slot(b), slot(b) + G, ... (G = grid size; for
// down, half of the workgroups walk theirs backwards) of a list the permutation orders full tiles
// first and partial tiles by falling row count. Its async
// copy streams (global_load_lds_dwordx4 into LDS rings: activation rows 3 slices ahead in a
// 4-slot ring, copied by waves 0-3; weight rows 2 slices ahead in a 3-slot ring, waves 4-7) run
// on across tile boundaries, so the next tile's first slices load during this tile's epilogue. The
// next tile's tile entry and row gather indices are fetched one tile ahead. Slots are spread over
// the 8 XCDs in contiguous runs (workgroup b runs on XCD b % 8 and takes slot (b % 8) * G/8 + b/8),
// so tiles that share an expert's weights or gathered rows run in one XCD's L2 at the same time.
//
// Slices are XOR-swizzled (16-byte chunk c of row r at slot c ^ ((r >> 2) & 3): conflict-free
// fragment reads). The epilogue transposes each wave's output through a private LDS staging area so
// that every store instruction writes whole 128-byte lines.
#include <cstdlib>
#include <cstring>

#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {

constexpr int BM = 256;        // activation rows per tile
constexpr int BW = 256;        // weight rows per tile
constexpr int BK = 32;         // K slice
constexpr int NTHREADS = 512;  // 8 waves: 0-3 copy activation rows, 4-7 weight rows
constexpr int NA = 4;          // activation ring slots: copies run 3 slices ahead
constexpr int NW = 3;          // weight ring slots: copies run 2 slices ahead
constexpr int SLOT_ELEMS = 256 * BK;  // one ring slot: 256 rows of one K slice (16 KiB)
constexpr int NCOPY = 4;       // async copies per lane per slice (16 rows each, 64 rows per wave)

// Destination of the epilogue stores of lanes outside the output (rows past a partial tile,
// columns past N): garbage, never read. External linkage on purpose: stores into a file-local
// array nobody reads are dead code to the optimizer, and the slice waits count every one.
__device__ __attribute__((aligned(16))) u32x4_t q38moe_gemm_store_sink[8 * 64];

enum { MODE_GATE_UP = 0, MODE_DOWN = 1, MODE_GATHER = 2 };

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
  uint16_t* GU;               // gate/up with SAVE_GU: the bf16 pre-activations [g | u], rows [*, 2N]
  int P;                      // first shared-expert row of the row space
  int N, K, E, topk;
  int ntiles_n;               // output-column tiles per row tile
  // e4m3 operands only (FP8 instantiations): K counts 16-bit units (two e4m3 values each), so
  // the copy machinery moves the same 64 bytes per row and slice. Dequantisation scales:
  const float* a_scale;       // per GEMM row (the sorted row space)
  const float* w_scale;       // routed weights: gate/up [E, 2N], down [E, N]
  const float* ws_scale_a;    // shared expert: gate [N] (gate/up) or down [N]
  const float* ws_scale_b;    // shared expert: up [N] (gate/up)
};

__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ ((r >> 2) & 3)) << 3); }

// A weight fragment of mfma_f32_32x32x16_bf16 from a ring slot: output row n0 + lane % 32, the 8
// K elements of 16-byte chunk kc + lane / 32 (kc = 0: the slice's first 16, 2: its second 16).
// Row-major weight slots ([256 rows][32 K], swizzled as swz) are read directly. K-major slots (WKN:
// [32 K rows][256 columns], 512 bytes per K row, 16-byte chunk c of K row r at c ^ 4 (r % 4)) are
// read with the gfx950 transposing LDS read ds_read_b64_tr_b16: within each 16-lane group, component
// j of lane i is element i % 4 of the 8 bytes that lane 4j + i / 4 addresses, so lane s addressing
// K row k0 + s / 4, columns c0 + 4 (s % 4) .. + 3 receives K rows k0 .. k0 + 3 of column c0 + s;
// two such reads (k0 and k0 + 4) are the fragment. A half-wave's reads cover 4 K rows x 64 bytes,
// which the swizzle spreads over all 64 banks.
typedef short q38_i16x4_t __attribute__((ext_vector_type(4)));
template <bool WKN>
__device__ __forceinline__ u32x4_t w_frag(const uint16_t* slot, int n0, int kc, int lane) {
  if constexpr (!WKN) {
    return ld16(slot + swz(n0 + (lane & 31), kc + (lane >> 5)));
  } else {
    const int s = lane & 15;
    const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
    const int k0 = 8 * (kc + (lane >> 5)) + (s >> 2);
    const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)slot;
    auto off = [&](int kr) { return kr * 512 + 16 * ((col >> 3) ^ (4 * (kr & 3))) + 2 * (col & 7); };
    const q38_i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) q38_i16x4_t*)(uintptr_t)(base + off(k0)));
    const q38_i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) q38_i16x4_t*)(uintptr_t)(base + off(k0 + 4)));
    const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
    return u32x4_t{a.x, a.y, b.x, b.y};
  }
}

// Tile-table entry as scalar loads (x2 + x1: there is no 3-dword scalar load, and a 3-dword vector
// load would join the copy queue).
__device__ __forceinline__ int4 tile_entry(const GemmParams& p, int mt) {
  if (p.tiles != nullptr) {
    const uint64_t xy = load_uniform(reinterpret_cast<const uint64_t*>(p.tiles + mt));
    const int z = load_uniform(reinterpret_cast<const int*>(p.tiles + mt) + 2);
    return make_int4((int)(uint32_t)xy, (int)(uint32_t)(xy >> 32), z, 0);
  }
  const int row0 = mt * BM;
  return make_int4(p.E, row0, (int)min((int64_t)BM, p.M - (int64_t)row0), 0);
}

// Entry of a table that must hold expert groups only (the K-major down and the saving gate/up,
// whose callers permute without shared rows): a shared-expert tile found there runs as an empty
// tile of expert 0 from row 0, so every read stays in bounds and nothing is stored.
template <bool EXPERTS_ONLY>
__device__ __forceinline__ int4 tile_entry_of(const GemmParams& p, int mt) {
  const int4 t = tile_entry(p, mt);
  return EXPERTS_ONLY && t.x >= p.E ? make_int4(0, 0, 0, 0) : t;
}

// True when the activation rows of tile `ti` are gathered through perm (routed gate/up rows).
template <int MODE>
__device__ __forceinline__ bool gathered(const GemmParams& p, int4 ti) {
  return (MODE == MODE_GATE_UP || MODE == MODE_GATHER) && ti.x < p.E;
}

// Row index behind each of this lane's activation copies (only activation-copying waves use it):
// the pair of a routed gate/up row, else the row itself. Rows past the tile read row 0 of the
// tile; their products only reach outputs that are never stored.
__device__ __forceinline__ void plain_rows(int4 ti, int wave, int lane, int (&rows)[NCOPY]) {
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) {
    const int r = 64 * wave + 16 * q + (lane >> 2);
    rows[q] = ti.y + (r < ti.z ? r : 0);
  }
}

template <int MODE>
__device__ __forceinline__ void gather_rows(const GemmParams& p, int4 ti, int wave, int lane,
                                            int (&rows)[NCOPY]) {
  plain_rows(ti, wave, lane, rows);
  if (gathered<MODE>(p, ti)) {
#pragma unroll
    for (int q = 0; q < NCOPY; ++q) rows[q] = p.perm[rows[q]];
  }
}

// Global source of each of this lane's copies for tile `ti`, output-column tile `nt`. Copy q of
// wave w fills slice rows 64w + 16q + lane/4 (rows < 256: activations, else weights); lane l
// lands in 16-byte slot l % 4 of its row, which holds chunk (l % 4) ^ ((row >> 2) & 3).
// WKN (down only): the weights are [E, K, N] (each expert's matrix stored K-major, as the
// experts' backward multiplies by gate_up_proj and down_proj themselves). A weight slot then holds
// the slice's 32 K rows of the tile's 256 output columns, 512 bytes per K row: copy q of weight
// wave w fills K row 8 (w - 4) + 2q + lane/32, 16-byte slot lane % 32, which holds column chunk
// (lane % 32) ^ 4 (K row % 4). The slice's K offset is then a multiple of N (see Q38_ISSUE).
template <int MODE, bool WKN = false>
__device__ __forceinline__ void copy_sources(const GemmParams& p, int4 ti, int nt, int wave,
                                             int lane, const int (&rows)[NCOPY],
                                             const uint16_t* (&src)[NCOPY]) {
  const int K = p.K, N = p.N;
  const bool shared_grp = ti.x >= p.E;
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) {
    const int r = 64 * wave + 16 * q + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    if (WKN && wave >= 4) {
      const int kr = 8 * (wave - 4) + 2 * q + (lane >> 5);
      const int col = nt * BW + 8 * ((lane & 31) ^ (4 * (kr & 3)));
      // Tile tables of this form hold experts only; another group reads expert 0 (in bounds).
      src[q] = p.W + (int64_t)(ti.x < p.E ? ti.x : 0) * K * N + (int64_t)kr * N + (col < N ? col : 0);
    } else if (wave < 4) {
      int64_t arow = rows[q];
      if (MODE != MODE_DOWN) arow = shared_grp ? (int64_t)(rows[q] - p.P) : (int64_t)(rows[q] / p.topk);
      src[q] = p.A + arow * K + c * 8;
    } else {
      const int rb = r - BM;
      const uint16_t* base;
      int col;
      if (MODE == MODE_GATE_UP) {
        // Weight rows 128 * half + [0, 64): gate, + [64, 128): up, of output columns
        // nt * 128 + 64 * half + [0, 64).
        const int half = rb >> 7, within = rb & 127;
        const bool up = within >= 64;
        col = nt * 128 + 64 * half + (within & 63);
        if (shared_grp) base = up ? p.Ws_b : p.Ws_a;
        else base = p.W + (int64_t)ti.x * 2 * N * K + (up ? (int64_t)N * K : 0);
      } else {
        col = nt * BW + rb;
        base = shared_grp ? p.Ws_a : p.W + (int64_t)ti.x * N * K;
      }
      src[q] = base + (int64_t)(col < N ? col : 0) * K + c * 8;
    }
  }
}

// Dequantisation scale of weight row rb (0..BW-1) of tile `ti`, output-column tile `nt`: the same
// row mapping as copy_sources (fp8 only).
template <int MODE>
__device__ __forceinline__ const float* weight_scale_src(const GemmParams& p, int4 ti, int nt, int rb) {
  const int N = p.N;
  const bool shared_grp = ti.x >= p.E;
  if (MODE == MODE_GATE_UP) {
    const int half = rb >> 7, within = rb & 127;
    const bool up = within >= 64;
    int col = nt * 128 + 64 * half + (within & 63);
    col = col < N ? col : 0;
    if (shared_grp) return (up ? p.ws_scale_b : p.ws_scale_a) + col;
    return p.w_scale + (int64_t)ti.x * 2 * N + (up ? N : 0) + col;
  }
  int col = nt * BW + rb;
  col = col < N ? col : 0;
  return shared_grp ? p.ws_scale_a + col : p.w_scale + (int64_t)ti.x * N + col;
}

// Async global -> LDS copies issued from inline asm: lane l copies 16 (or 4) bytes from gsrc to
// LDS [lds_wave_base + 16*l] (or + 4*l); M0 holds the wave's LDS base. The compiler's wait
// analysis mistakes the copy's address register for a destination (its builtin form is followed
// by vmcnt(0) wherever the register allocator reuses that register) and, for the 4-byte form,
// treats it as a write to any LDS address; from asm the copies are invisible to it. Their
// completion is ordered by the explicit vmcnt waits of the slice pipeline (vector memory loads
// complete in order); a compiler-generated wait for one of its own loads can only count them as
// further outstanding operations, i.e. wait longer. The s_nop covers the M0-write hazard.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ void dma16(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(gsrc)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* gsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(gsrc)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) + s_barrier for a compile-time N.
// Every wait also drains this wave's LDS reads: the bf16 main loop reads the second half of
// slice j while it multiplies the first, so those reads may still be in flight here, and the
// copies issued after the barrier refill the slot they read. The drain is a separate builtin wait,
// so that the compiler's own wait insertion knows no LDS read or scalar load is pending after it
// (lgkmcnt counts both, and while a scalar load may be pending it can only wait for zero).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier_imm() {
  wait_lgkm0();
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// s_waitcnt vmcnt(n) + s_barrier for a wave-uniform n in [0, 48] (vmcnt takes an immediate): a
// multi-level branch tree, used only off the steady state (drain after the last tile, K shorter
// than a ring).
__device__ __forceinline__ void wait_vmcnt_barrier(int n) {
  wait_lgkm0();
#define Q38_W(N) case N: asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_barrier" ::: "memory"); break;
  switch (n) {
    Q38_W(1) Q38_W(2) Q38_W(3) Q38_W(4) Q38_W(5) Q38_W(6) Q38_W(7) Q38_W(8) Q38_W(9) Q38_W(10)
    Q38_W(11) Q38_W(12) Q38_W(13) Q38_W(14) Q38_W(15) Q38_W(16) Q38_W(17) Q38_W(18) Q38_W(19)
    Q38_W(20) Q38_W(21) Q38_W(22) Q38_W(23) Q38_W(24) Q38_W(25) Q38_W(26) Q38_W(27) Q38_W(28)
    Q38_W(29) Q38_W(30) Q38_W(31) Q38_W(32) Q38_W(33) Q38_W(34) Q38_W(35) Q38_W(36) Q38_W(37)
    Q38_W(38) Q38_W(39) Q38_W(40) Q38_W(41) Q38_W(42) Q38_W(43) Q38_W(44) Q38_W(45) Q38_W(46)
    Q38_W(47) Q38_W(48)
    default: asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory"); break;
  }
#undef Q38_W
}

// SAVE_GU (bf16 gate/up only): the epilogue also stores the rounded pre-activations bf16(g) and
// bf16(u) of every row to GU [rows, 2N] ([g | u], the operand of the SwiGLU backward), the values it
// computes H from, so a training forward keeps them instead of recomputing them in the backward.
template <int MODE, bool ASYNC_ROWS, bool FP8, bool WKN = false, bool SAVE_GU = false>
__global__ __launch_bounds__(NTHREADS, 1) void grouped_gemm_kernel(GemmParams p) {
  static_assert(!WKN || (MODE == MODE_DOWN && !FP8), "K-major weights: bf16 down only");
  static_assert(!SAVE_GU || (MODE == MODE_GATE_UP && !FP8), "saved pre-activations: bf16 gate/up only");
  // 16-byte stores per wave and tile: 2 per 32x32 output block, 2 x 2 (gate/up, and as many again
  // for each of g and u with SAVE_GU) or 2 x 4 blocks.
  constexpr int EPI_STORES = MODE == MODE_GATE_UP ? (SAVE_GU ? 24 : 8) : 16;
  constexpr int NT_OUT = MODE == MODE_GATE_UP ? 2 : 4;  // 32-column output blocks per wave
  __shared__ __attribute__((aligned(16))) uint16_t ring_a[NA * SLOT_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t ring_w[NW * SLOT_ELEMS];
  // Gather indices of the next tile (perm[row0 + r], r < 256), copied asynchronously; activation
  // wave w copies and reads entries [64w, 64w + 64) only.
  __shared__ __attribute__((aligned(16))) int32_t next_rows[BM];
  // Epilogue staging, private to each wave: 32 output rows x 64 columns (bf16, 128 bytes per row).
  __shared__ __attribute__((aligned(16))) uint16_t epi_stage[8 * 32 * 64];
  // fp8: dequantisation scales of the tile's 256 activation rows and 256 weight rows, double
  // buffered by tile parity (copied one tile ahead, like the gather indices).
  __shared__ __attribute__((aligned(16))) float sc_a[FP8 ? 2 : 1][FP8 ? BM : 1];
  __shared__ __attribute__((aligned(16))) float sc_w[FP8 ? 2 : 1][FP8 ? BW : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches, SGPR M0
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const bool is_a = wave < 4;

  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  const int slot = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
  const int used_m = p.tiles != nullptr ? load_uniform(p.ntiles_dev) : p.ntiles_host;
  const int used = used_m * p.ntiles_n;
  int L = slot;
  if (L >= used) return;
  // Down: every other group of ntiles_n consecutive slots (one row tile's column tiles; each XCD
  // holds a contiguous run of slots, so every XCD has both kinds) walks its units last to first.
  // The same units per workgroup, in another order: the XCD's epilogues, which write 128 KiB of
  // Y each, no longer fall at the same moments across all of its CUs (down 77-78 -> 73-74 us at
  // configuration 2; gate/up, whose outputs are a quarter the size, gains nothing from it).
  const bool reverse = MODE == MODE_DOWN && ((slot / p.ntiles_n) & 1) != 0;
  const int step = reverse ? -G : G;
  if (reverse) L = slot + ((used - 1 - slot) / G) * G;
  const int nk = p.K / BK;
  // This wave's copy distance and ring: activation rows (gathered, farther away in the memory
  // hierarchy) run NA - 1 = 3 slices ahead, weight rows (shared by the concurrent tiles of an
  // expert, mostly L2 hits) NW - 1 = 2. Each wave waits only for its own copies (vmcnt counts per
  // wave), so the two streams do not hold each other up.
  const int ring_n = is_a ? NA : NW;
  const int dist = min(ring_n - 1, nk);  // <= nk: copies run at most one tile ahead
  const bool steady = dist == ring_n - 1;
  // ASYNC_ROWS (K >= 2 (NA - 1) + 1 slices): the next tile's gather indices are copied to LDS
  // before this tile's slice-0 wait, behind the copies of slices 0 .. d-1 (d = NA - 1), so the
  // in-order wait of slice d completes them; they are read after the wait of slice nk - d - 1 >= d.
  // Otherwise they are plain loads there (which the compiler waits for, draining the copies in
  // flight): a separate instantiation, so the main one carries no such load.
  constexpr bool async_rows = ASYNC_ROWS;

  // K-slice order rotated per expert: slice j of a unit of expert e is K slice (j + 2e) mod nk (the
  // sum over K is order-free up to fp32 rounding); shared-expert units rotate by row tile. Rows are
  // 2 KiB (or 512 B) apart, so without it the 512 row segments of a slice sit at one offset modulo
  // the row pitch in every unit, and the units running together on an XCD would all hit the same
  // few L2 channels at each step. The units of one expert (adjacent in the tile list, run together
  // on one XCD) keep one order, so their copies of the same weight rows and, for the output-column
  // tiles of a row tile, of the same gathered activation rows meet in that XCD's L2.
  auto rot_of = [&](int4 t_, int u) { return (t_.x < p.E ? 2 * t_.x : 2 * (u / p.ntiles_n)) % nk; };
  int4 ti = tile_entry_of<WKN || SAVE_GU>(p, L / p.ntiles_n);
  int rot = rot_of(ti, L);
  int Ln = L + step;
  int4 tin = (Ln >= 0 && Ln < used) ? tile_entry_of<WKN || SAVE_GU>(p, Ln / p.ntiles_n) : make_int4(0, 0, 0, 0);
  int rows[NCOPY], rows_n[NCOPY];
  const uint16_t* src[NCOPY];
  const uint16_t* src_n[NCOPY];
  gather_rows<MODE>(p, ti, wave, lane, rows);
  // fp8: the first tile's dequantisation scales (the wait below completes them).
#define Q38_SCALES(BUF, TI, NT)                                                               \
  do {                                                                                     \
    if (is_a) {                                                                            \
      const int r_ = 64 * wave + lane;                                                     \
      dma4(p.a_scale + (TI).y + (r_ < (TI).z ? r_ : 0), lds_addr(&sc_a[BUF][64 * wave]));  \
    } else {                                                                               \
      dma4(weight_scale_src<MODE>(p, TI, NT, 64 * (wave - 4) + lane),                      \
           lds_addr(&sc_w[BUF][64 * (wave - 4)]));                                         \
    }                                                                                      \
  } while (0)
  if (FP8) Q38_SCALES(0, ti, L % p.ntiles_n);
  // Retire these loads on every path (waves >= 4 never read them); a load left pending in the
  // compiler's bookkeeping makes it wait for all copies wherever its register is reused.
  wait_vmcnt0();
  copy_sources<MODE, WKN>(p, ti, L % p.ntiles_n, wave, lane, rows, src);
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) {
    rows_n[q] = 0;
    src_n[q] = src[q];
  }

  // This wave's 64 rows of a slot: activation rows 64w.. of ring_a, weight rows 64(w-4).. of ring_w.
  const uint32_t my_ring = is_a ? lds_addr(ring_a) + 2 * 64 * wave * BK : lds_addr(ring_w) + 2 * 64 * (wave - 4) * BK;
  // Elements between consecutive K positions of this wave's copy sources: 1, or N for the K-major
  // weights of WKN (their slice offset moves down K rows).
  const int kstride = WKN && !is_a ? p.N : 1;
#define Q38_ISSUE(SLOT, SRC, KS, ROT)                                                    \
  do {                                                                                   \
    const uint32_t st_ = my_ring + (uint32_t)(SLOT) * (2 * SLOT_ELEMS);                  \
    const int ko_ = ((KS) + (ROT) < nk ? (KS) + (ROT) : (KS) + (ROT) - nk) * BK;         \
    _Pragma("unroll") for (int q_ = 0; q_ < NCOPY; ++q_)                                 \
      dma16((SRC)[q_] + (int64_t)ko_ * kstride, st_ + q_ * (2 * 16 * BK));               \
  } while (0)

  uint16_t* const sink = reinterpret_cast<uint16_t*>(q38moe_gemm_store_sink + 64 * wave + lane);
  for (int d = 0; d < dist; ++d) Q38_ISSUE(d, src, d, rot);
  int fill = dist;  // ring slot of the next copy: (slice + dist) % ring_n
  int ra = 0, rw = 0;  // ring_a / ring_w slots of the slice being multiplied

  f32x16_t acc[4][2];
  u32x4_t wy[4], ay[2];  // bf16: the current slice's second-half fragments (see Q38_COMPUTE)
  int stores_prev = 0;  // epilogue stores this wave issued at the previous tile's end
  int tpar = 0;         // fp8: scale buffer of the current tile
  for (;;) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][mi][i] = 0.0f;
    const bool has_next = Ln >= 0 && Ln < used;
    const int Lnn = Ln + step;
    int4 tinn = make_int4(0, 0, 0, 0);
    const bool active = 64 * wm < ti.z;
    const bool next_async = has_next && async_rows && gathered<MODE>(p, tin);

    // One tile ahead: the next tile's gather indices; two ahead: its successor's entry.
    if (has_next) {
      if (next_async && is_a) {
        const int r = 64 * wave + lane;
        dma4(p.perm + tin.y + (r < tin.z ? r : 0), lds_addr(next_rows + 64 * wave));
      }
      if (Lnn >= 0 && Lnn < used) tinn = tile_entry_of<WKN || SAVE_GU>(p, Lnn / p.ntiles_n);
    }

    // Step: wait until at most N of this wave's vector-memory operations are outstanding, which
    // completes its copies of the current slice (loads complete in order; N counts what was
    // issued after them: 4 per later slice already copied, plus, during the first `dist` steps,
    // the previous tile's epilogue stores, which follow those copies in the queue; the next
    // tile's gather-index copy is one more, not counted: a longer wait), then barrier: publishes
    // the slice and retires the slots of the previous one, which the next copies refill. Raw
    // s_barrier: __syncthreads() would also drain the copies in flight.
#define Q38_STORES_AFTER(KT) ((KT) < dist ? stores_prev : 0)
#define Q38_WAIT_BARRIER(N) wait_vmcnt_barrier(N)
  // Steady state (dist == ring_n - 1): the count is a compile-time constant of the wave's role,
  // plus EPI_STORES while the previous epilogue's stores follow the slice.
#define Q38_WAIT_STEADY(STORES)                                                              \
  do {                                                                                     \
    if (is_a) {                                                                            \
      if (STORES) wait_vmcnt_barrier_imm<4 * (NA - 2) + EPI_STORES>();                     \
      else wait_vmcnt_barrier_imm<4 * (NA - 2)>();                                         \
    } else {                                                                               \
      if (STORES) wait_vmcnt_barrier_imm<4 * (NW - 2) + EPI_STORES>();                     \
      else wait_vmcnt_barrier_imm<4 * (NW - 2)>();                                         \
    }                                                                                      \
  } while (0)
#define Q38_NEXT_SOURCES()                                                                 \
  do {                                                                                     \
    if (is_a && next_async) {                                                              \
      _Pragma("unroll") for (int q = 0; q < NCOPY; ++q)                                    \
        rows_n[q] = next_rows[(64 * wave + 16 * q + (lane >> 2)) & (BM - 1)];              \
    } else if (!is_a || async_rows || !gathered<MODE>(p, tin)) {                           \
      plain_rows(tin, wave, lane, rows_n);                                                 \
    } else {                                                                               \
      gather_rows<MODE>(p, tin, wave, lane, rows_n);                                       \
    }                                                                                      \
    copy_sources<MODE, WKN>(p, tin, Ln % p.ntiles_n, wave, lane, rows_n, src_n);           \
  } while (0)
#define Q38_COMPUTE()                                                                      \
  do {                                                                                     \
    if (active && FP8) {                                                                   \
      /* e4m3: one 32x32x64 MFMA per block and slice; lane half lh takes the slice's */    \
      /* 16-byte chunks 2lh, 2lh+1 of its row in both operands (any k order shared by */   \
      /* both operands gives the same dot product). */                                     \
      const uint16_t* as_ = ring_a + ra * SLOT_ELEMS;                                      \
      const uint16_t* bs_ = ring_w + rw * SLOT_ELEMS;                                      \
      i32x8_t wf8[4], af8[2];                                                              \
      _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
        wf8[t] = cat8(ld16(bs_ + swz(128 * wn + 32 * t + lr, 2 * lh)),                     \
                      ld16(bs_ + swz(128 * wn + 32 * t + lr, 2 * lh + 1)));                \
      _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                     \
        af8[mi] = cat8(ld16(as_ + swz(64 * wm + 32 * mi + lr, 2 * lh)),                    \
                       ld16(as_ + swz(64 * wm + 32 * mi + lr, 2 * lh + 1)));               \
      _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
        _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                   \
          acc[t][mi] = mfma32x32x64_fp8(wf8[t], af8[mi], acc[t][mi]);                      \
    } else if (active) {                                                                   \
      /* bf16, software-pipelined by half slices (16 k each): the reads of this slice's */ \
      /* first half run under the MFMAs of the previous slice's second half (held in    */ \
      /* wy/ay since the previous step), and the reads of the second half under the     */ \
      /* MFMAs of the first, so the matrix pipe is not left waiting on LDS after the     */ \
      /* barrier. The tile's last second half is multiplied after the slice loop.       */ \
      const uint16_t* as_ = ring_a + ra * SLOT_ELEMS;                                      \
      const uint16_t* bs_ = ring_w + rw * SLOT_ELEMS;                                      \
      u32x4_t wx[4], ax[2];                                                                \
      _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
        wx[t] = w_frag<WKN>(bs_, 128 * wn + 32 * t, 0, lane);                              \
      _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                     \
        ax[mi] = ld16(as_ + swz(64 * wm + 32 * mi + lr, lh));                              \
      /* keeps these reads ahead of the MFMAs below (not sunk past the branch) */          \
      asm volatile("" ::: "memory");                                                       \
      if (kt > 0) {                                                                        \
        _Pragma("unroll") for (int t = 0; t < 4; ++t)                                      \
          _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                 \
            acc[t][mi] = mfma32x32x16(wy[t], ay[mi], acc[t][mi]);                          \
      }                                                                                    \
      _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
        wy[t] = w_frag<WKN>(bs_, 128 * wn + 32 * t, 2, lane);                              \
      _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                     \
        ay[mi] = ld16(as_ + swz(64 * wm + 32 * mi + lr, 2 + lh));                          \
      _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
        _Pragma("unroll") for (int mi = 0; mi < 2; ++mi)                                   \
          acc[t][mi] = mfma32x32x16(wx[t], ax[mi], acc[t][mi]);                            \
      /* Issue order of the second half's reads and the first half's MFMAs: one read after */ \
      /* each of the first six MFMAs, so the eight waves' LDS reads spread over the matrix */  \
      /* pipe's work instead of arriving together (bit-identical; the configuration-2 block */ \
      /* 0.2713-0.2723 -> 0.2685-0.2691 ms, same box, three interleaved runs). */          \
      /* (K-major weights: ten reads, two transposing reads per weight fragment, two after  */ \
      /* each of the first five MFMAs.) */                                                  \
      _Pragma("unroll") for (int i_ = 0; i_ < (WKN ? 5 : 6); ++i_) {                       \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* one MFMA */                  \
        __builtin_amdgcn_sched_group_barrier(0x100, WKN ? 2 : 1, 0); /* LDS reads */       \
      }                                                                                    \
      __builtin_amdgcn_sched_group_barrier(0x008, 10, 0);                                  \
    }                                                                                      \
    ra = ra + 1 == NA ? 0 : ra + 1;                                                        \
    rw = rw + 1 == NW ? 0 : rw + 1;                                                        \
    fill = fill + 1 == ring_n ? 0 : fill + 1;                                              \
  } while (0)

    // fp8: the next tile's scales go to the other buffer once the step-0 barrier has retired the
    // previous tile's epilogue reads of it.
#define Q38_NEXT_SCALES()                                                                  \
  do {                                                                                     \
    if (FP8 && kt == 0 && has_next) Q38_SCALES(tpar ^ 1, tin, Ln % p.ntiles_n);            \
  } while (0)
    // Phase 1: this wave's copy at step kt is this tile's slice kt + dist.
    const int p1 = nk - dist;
    const int head = min(dist, p1);
    int kt = 0;
    for (; kt < head; ++kt) {  // kt < dist: the previous epilogue's stores follow the slice
      if (steady) Q38_WAIT_STEADY(stores_prev != 0);
      else Q38_WAIT_BARRIER(4 * (dist - 1) + stores_prev);
      Q38_NEXT_SCALES();
      Q38_ISSUE(fill, src, kt + dist, rot);
      Q38_COMPUTE();
    }
    // Only reached with p1 > dist, i.e. steady: the count is the role's constant.
    for (; kt < p1; ++kt) {
      Q38_WAIT_STEADY(false);
      Q38_ISSUE(fill, src, kt + dist, rot);
      Q38_COMPUTE();
    }
    // Phase 2 (this wave's last `dist` steps): the copies run on into the next tile, or the
    // stream drains after the last tile.
    if (has_next) Q38_NEXT_SOURCES();
    for (; kt < nk; ++kt) {
      if (steady && has_next) Q38_WAIT_STEADY(kt < dist && stores_prev != 0);
      else Q38_WAIT_BARRIER(4 * (has_next ? dist - 1 : nk - 1 - kt) + Q38_STORES_AFTER(kt));
      Q38_NEXT_SCALES();
      if (has_next) Q38_ISSUE(fill, src_n, kt + dist - nk, rot_of(tin, Ln));
      Q38_COMPUTE();
    }
    // The last slice's second half.
    if (active && !FP8) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) acc[t][mi] = mfma32x32x16(wy[t], ay[mi], acc[t][mi]);
    }
#undef Q38_WAIT_BARRIER
#undef Q38_NEXT_SCALES
#undef Q38_WAIT_STEADY
#undef Q38_STORES_AFTER
#undef Q38_NEXT_SOURCES
#undef Q38_COMPUTE

    // Epilogue. In a 32x32 block lane l holds row l % 32 and 4-column runs at 8*gq + 4*(l / 32);
    // each pair of blocks (32 rows x 64 columns) goes through this wave's LDS staging area (16-byte
    // chunk c of row r at slot c ^ ((r >> 1) & 7): two-way bank conflicts on the 8-byte writes,
    // none on the reads) and leaves as four 16-byte-per-lane stores that each cover 8 rows x 128
    // contiguous bytes, i.e. whole cache lines. The staging area is the wave's own, so no barrier;
    // the slice copies in flight never touch it.
    const int nt = L % p.ntiles_n;
    const int col_wave = MODE == MODE_GATE_UP ? nt * 128 + 64 * wn : nt * BW + 128 * wn;
    uint8_t* const stage = reinterpret_cast<uint8_t*>(epi_stage + wave * (32 * 64));
    if (active) {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        // fp8: dequantisation by the activation row's and the weight rows' scales.
        const float sa = FP8 ? sc_a[tpar][64 * wm + 32 * mi + lr] : 1.0f;
#pragma unroll
        for (int tp = 0; tp < NT_OUT / 2; ++tp) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int to = 2 * tp + tt;
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              f32x4_t sw0 = {1.0f, 1.0f, 1.0f, 1.0f}, sw1 = sw0;
              if (FP8) {
                const float* swp = &sc_w[tpar][128 * wn + 32 * to + 8 * gq + 4 * lh];
                sw0 = *reinterpret_cast<const f32x4_t*>(swp) * sa;
                if (MODE == MODE_GATE_UP) sw1 = *reinterpret_cast<const f32x4_t*>(swp + 64) * sa;
              }
              uint32_t v[2];
#pragma unroll
              for (int h2 = 0; h2 < 2; ++h2) {
                const int i = 4 * gq + 2 * h2;
                const float a0 = FP8 ? acc[to][mi][i] * sw0[2 * h2] : acc[to][mi][i];
                const float a1 = FP8 ? acc[to][mi][i + 1] * sw0[2 * h2 + 1] : acc[to][mi][i + 1];
                if (MODE == MODE_GATE_UP) {
                  // Reference rounding (inference.py:90-96): bf16 gate and up, bf16 silu(gate),
                  // bf16 product; each bf16 rounding is one packed RNE conversion of two values.
                  const float b0 = FP8 ? acc[to + 2][mi][i] * sw1[2 * h2] : acc[to + 2][mi][i];
                  const float b1 = FP8 ? acc[to + 2][mi][i + 1] * sw1[2 * h2 + 1] : acc[to + 2][mi][i + 1];
                  float g0, g1, u0, u1, s0, s1;
                  unpack_bf16x2(pack_bf16x2(a0, a1), g0, g1);
                  unpack_bf16x2(pack_bf16x2(b0, b1), u0, u1);
                  unpack_bf16x2(pack_bf16x2(g0 * __builtin_amdgcn_rcpf(1.0f + __expf(-g0)),
                                            g1 * __builtin_amdgcn_rcpf(1.0f + __expf(-g1))), s0, s1);
                  v[h2] = pack_bf16x2(s0 * u0, s1 * u1);
                } else {
                  v[h2] = pack_bf16x2(a0, a1);
                }
              }
              const int ch = 4 * tt + gq;
              *reinterpret_cast<uint2*>(stage + lr * 128 + ((ch ^ ((lr >> 1) & 7)) << 4) + 8 * lh) =
                  make_uint2(v[0], v[1]);
            }
          }
          // Every lane stores (lanes past the tile's rows or columns into the sink), so each
          // wave issues exactly EPI_STORES stores per tile, which the slice waits count.
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3), ch = lane & 7;
            const u32x4_t d = *reinterpret_cast<const u32x4_t*>(stage + row * 128 + ((ch ^ ((row >> 1) & 7)) << 4));
            const int r = 64 * wm + 32 * mi + row;
            const int col = col_wave + 64 * tp + 8 * ch;
            uint16_t* dst = p.C + (int64_t)(ti.y + r) * p.N + col;
            // Down's Y rows (201 MB at config 2, read once by the combine) are written
            // non-temporally so that they do not displace the weights and activations from the
            // 256 MB MALL; gate/up's H rows, which down reads right away, are cached.
            if (MODE == MODE_DOWN) st16_stream(r < ti.z && col < p.N ? dst : sink, d);
            else st16(r < ti.z && col < p.N ? dst : sink, d);
          }
          if constexpr (SAVE_GU) {
            // The same 32 rows x 64 columns of g (half 0) and of u (half 1), staged and stored
            // like H (the staging area's earlier reads precede these writes: one wave's LDS
            // operations complete in order).
#pragma unroll
            for (int half = 0; half < 2; ++half) {
#pragma unroll
              for (int tt = 0; tt < 2; ++tt) {
                const int to = 2 * tp + tt + 2 * half;
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                  const int i = 4 * gq;
                  const uint32_t v0 = pack_bf16x2(acc[to][mi][i], acc[to][mi][i + 1]);
                  const uint32_t v1 = pack_bf16x2(acc[to][mi][i + 2], acc[to][mi][i + 3]);
                  const int ch = 4 * tt + gq;
                  *reinterpret_cast<uint2*>(stage + lr * 128 + ((ch ^ ((lr >> 1) & 7)) << 4) + 8 * lh) =
                      make_uint2(v0, v1);
                }
              }
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int row = 8 * j + (lane >> 3), ch = lane & 7;
                const u32x4_t d = *reinterpret_cast<const u32x4_t*>(stage + row * 128 + ((ch ^ ((row >> 1) & 7)) << 4));
                const int r = 64 * wm + 32 * mi + row;
                const int col = col_wave + 64 * tp + 8 * ch;
                uint16_t* dst = p.GU + (int64_t)(ti.y + r) * 2 * p.N + half * p.N + col;
                st16(r < ti.z && col < p.N ? dst : sink, d);
              }
            }
          }
        }
      }
    }
    stores_prev = active ? EPI_STORES : 0;
    if (!has_next) break;
    tpar ^= 1;
    L = Ln;
    ti = tin;
    rot = rot_of(ti, L);
    Ln = Lnn;
    tin = tinn;
#pragma unroll
    for (int q = 0; q < NCOPY; ++q) src[q] = src_n[q];
  }
#undef Q38_ISSUE
#undef Q38_SCALES
  // No LDS copy may still be landing when the workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

int gemm_block_m() { return BM; }

// One workgroup per CU (the kernel is persistent), never more than there are tiles.
static unsigned grid_for(int max_mtiles, int ntiles_n) {
  const int cus = device_cus();
  const int64_t tiles = (int64_t)max_mtiles * ntiles_n;
  return (unsigned)(tiles < cus ? tiles : cus);
}

// K is in elements; e4m3 operands pass it to the kernel in 16-bit units (two elements each).
static hipError_t gate_up_impl(const void* x, const int32_t* perm, const int4* tiles,
                               const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                               const void* w_gate_up, const void* ws_gate, const void* ws_up,
                               uint16_t* H, int N, int K, int E, int topk, bool fp8,
                               const float* a_scale, const float* w_scale, const float* ws_scale_gate,
                               const float* ws_scale_up, hipStream_t stream, uint16_t* GU = nullptr) {
  GemmParams p;
  p.A = static_cast<const uint16_t*>(x);
  p.GU = GU;
  p.perm = perm;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.ntiles_host = tiles != nullptr ? 0 : (int)((M_dense + BM - 1) / BM);
  p.M = M_dense;
  p.W = static_cast<const uint16_t*>(w_gate_up);
  p.Ws_a = static_cast<const uint16_t*>(ws_gate);
  p.Ws_b = static_cast<const uint16_t*>(ws_up);
  p.C = H;
  p.P = P;
  p.N = N;
  p.K = fp8 ? K / 2 : K;
  p.E = E;
  p.topk = topk;
  p.ntiles_n = (N + 127) / 128;
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.ws_scale_a = ws_scale_gate;
  p.ws_scale_b = ws_scale_up;
  const int mt = tiles != nullptr ? max_mtiles : p.ntiles_host;
  if (mt == 0) return hipSuccess;
  const dim3 grid(grid_for(mt, p.ntiles_n));
  const bool async_rows = p.K / BK >= 2 * (NA - 1) + 1;
  if (fp8 && async_rows)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, true, true>), grid, dim3(NTHREADS), 0, stream, p);
  else if (fp8)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, false, true>), grid, dim3(NTHREADS), 0, stream, p);
  else if (GU != nullptr && async_rows)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, true, false, false, true>), grid, dim3(NTHREADS), 0, stream, p);
  else if (GU != nullptr)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, false, false, false, true>), grid, dim3(NTHREADS), 0, stream, p);
  else if (async_rows)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, true, false>), grid, dim3(NTHREADS), 0, stream, p);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATE_UP, false, false>), grid, dim3(NTHREADS), 0, stream, p);
  return hipGetLastError();
}

static hipError_t down_impl(const void* H, const int4* tiles, const int32_t* ntiles_dev,
                            int max_mtiles, int64_t M_dense, const void* w_down, const void* ws_down,
                            uint16_t* Y, int N, int K, int E, bool fp8, const float* a_scale,
                            const float* w_scale, const float* ws_scale, hipStream_t stream) {
  GemmParams p;
  p.A = static_cast<const uint16_t*>(H);
  p.GU = nullptr;
  p.perm = nullptr;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.ntiles_host = tiles != nullptr ? 0 : (int)((M_dense + BM - 1) / BM);
  p.M = M_dense;
  p.W = static_cast<const uint16_t*>(w_down);
  p.Ws_a = static_cast<const uint16_t*>(ws_down);
  p.Ws_b = nullptr;
  p.C = Y;
  p.P = 0;
  p.N = N;
  p.K = fp8 ? K / 2 : K;
  p.E = E;
  p.topk = 1;
  p.ntiles_n = (N + BW - 1) / BW;
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.ws_scale_a = ws_scale;
  p.ws_scale_b = nullptr;
  const int mt = tiles != nullptr ? max_mtiles : p.ntiles_host;
  if (mt == 0) return hipSuccess;
  const dim3 grid(grid_for(mt, p.ntiles_n));
  if (fp8)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_DOWN, false, true>), grid, dim3(NTHREADS), 0, stream, p);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_DOWN, false, false>), grid, dim3(NTHREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_gate_up_save(const uint16_t* x, const int32_t* perm, const int4* tiles, const int32_t* ntiles_dev,
                               int max_mtiles, int P, const uint16_t* w_gate_up, uint16_t* H, uint16_t* GU, int N,
                               int K, int E, int topk, hipStream_t stream) {
  return gate_up_impl(x, perm, tiles, ntiles_dev, max_mtiles, 0, P, w_gate_up, nullptr, nullptr, H, N, K, E, topk,
                      false, nullptr, nullptr, nullptr, nullptr, stream, GU);
}

hipError_t launch_down_kn(const uint16_t* A, const int4* tiles, const int32_t* ntiles_dev, int max_mtiles,
                          const uint16_t* w_kn, uint16_t* Y, int N, int K, int E, hipStream_t stream) {
  GemmParams p = {};
  p.A = A;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.W = w_kn;
  p.C = Y;
  p.N = N;
  p.K = K;
  p.E = E;
  p.topk = 1;
  p.ntiles_n = (N + BW - 1) / BW;
  if (max_mtiles == 0) return hipSuccess;
  const dim3 grid(grid_for(max_mtiles, p.ntiles_n));
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE_DOWN, false, false, true>), grid, dim3(NTHREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_gather_gemm(const uint16_t* A, const int32_t* perm, const int4* tiles,
                              const int32_t* ntiles_dev, int max_mtiles, const uint16_t* W, uint16_t* C,
                              int N, int K, int E, int topk, hipStream_t stream) {
  GemmParams p = {};
  p.A = A;
  p.perm = perm;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.W = W;
  p.C = C;
  p.N = N;
  p.K = K;
  p.E = E;
  p.topk = topk;
  p.ntiles_n = (N + BW - 1) / BW;
  if (max_mtiles == 0) return hipSuccess;
  const dim3 grid(grid_for(max_mtiles, p.ntiles_n));
  if (K / BK >= 2 * (NA - 1) + 1)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATHER, true, false>), grid, dim3(NTHREADS), 0, stream, p);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATHER, false, false>), grid, dim3(NTHREADS), 0, stream, p);
  return hipGetLastError();
}

// Q38MOE_GEMM_WAVES=8 (read once) keeps the gate/up launches (bf16 and e4m3) on the eight-wave kernel
// where the four-wave one (q38moe_gemm4w.hip) would run: for A/B timing. Results differ only in fp32
// summation order.
static bool use_gemm4w(int N, int K, int64_t a_rows) {
  static const bool off = [] {
    const char* e = std::getenv("Q38MOE_GEMM_WAVES");
    return e != nullptr && std::strcmp(e, "8") == 0;
  }();
  return !off && gemm4w_supported(N, K, a_rows);
}

hipError_t launch_gate_up(const uint16_t* x, const int32_t* perm, const int4* tiles,
                          const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                          const uint16_t* w_gate_up, const uint16_t* ws_gate,
                          const uint16_t* ws_up, uint16_t* H, int N, int K, int E, int topk,
                          hipStream_t stream) {
  // x rows: T = P / topk tokens (tile tables) or the dense rows.
  const int64_t x_rows = tiles != nullptr ? (int64_t)P / (topk > 0 ? topk : 1) : M_dense;
  if (use_gemm4w(N, K, x_rows))
    return launch_gate_up_4w(x, x_rows, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, w_gate_up, ws_gate, ws_up, H,
                             N, K, E, topk, stream);
  return gate_up_impl(x, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, w_gate_up, ws_gate, ws_up, H, N, K,
                      E, topk, false, nullptr, nullptr, nullptr, nullptr, stream);
}

hipError_t launch_down(const uint16_t* H, const int4* tiles, const int32_t* ntiles_dev,
                       int max_mtiles, int64_t M_dense, const uint16_t* w_down,
                       const uint16_t* ws_down, uint16_t* Y, int N, int K, int E,
                       hipStream_t stream) {
  return down_impl(H, tiles, ntiles_dev, max_mtiles, M_dense, w_down, ws_down, Y, N, K, E, false, nullptr,
                   nullptr, nullptr, stream);
}

hipError_t launch_gate_up_fp8(const uint8_t* xq, const int32_t* perm, const int4* tiles,
                              const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                              const float* a_scale, const uint8_t* wq_gate_up, const float* s_gate_up,
                              const uint8_t* wq_sh_gate, const float* s_sh_gate,
                              const uint8_t* wq_sh_up, const float* s_sh_up, uint16_t* H, int N,
                              int K, int E, int topk, hipStream_t stream) {
  const int64_t x_rows = tiles != nullptr ? (int64_t)P / (topk > 0 ? topk : 1) : M_dense;
  if (K % 2 == 0 && use_gemm4w(N, K / 2, x_rows))
    return launch_gate_up_4w_fp8(xq, x_rows, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, a_scale, wq_gate_up,
                                 s_gate_up, wq_sh_gate, s_sh_gate, wq_sh_up, s_sh_up, H, N, K, E, topk, stream);
  return gate_up_impl(xq, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, wq_gate_up, wq_sh_gate, wq_sh_up, H,
                      N, K, E, topk, true, a_scale, s_gate_up, s_sh_gate, s_sh_up, stream);
}

hipError_t launch_down_fp8(const uint8_t* Hq, const int4* tiles, const int32_t* ntiles_dev,
                           int max_mtiles, int64_t M_dense, const float* a_scale,
                           const uint8_t* wq_down, const float* s_down, const uint8_t* wq_sh_down,
                           const float* s_sh_down, uint16_t* Y, int N, int K, int E,
                           hipStream_t stream) {
  return down_impl(Hq, tiles, ntiles_dev, max_mtiles, M_dense, wq_down, wq_sh_down, Y, N, K, E, true, a_scale,
                   s_down, s_sh_down, stream);
}

}  // namespace q38
