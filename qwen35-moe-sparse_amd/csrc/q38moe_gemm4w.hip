// Four-wave grouped gate/up GEMM + SwiGLU on bf16 or e4m3 MFMA (R5, R6, R9, R14): the gate/up launch
// of the block when K (= h; e4m3: h / 2) is a multiple of 256 (>= 512) and the H columns fill whole
// tiles. Same products, roundings, tile table and unit order as grouped_gemm_kernel<MODE_GATE_UP>
// (q38moe_gemm.hip), a different data path:
//
//   H[r, n] = bf16(bf16(silu(bf16(a_r.Wg[n]))) * bf16(a_r.Wu[n])), a_r = x[perm[r] / k] for routed
//   rows (inference.py:74, 83-96) or x[r - P] for shared-expert rows (x[r] for a dense launch).
//
// A unit is 256 activation rows x 256 weight rows (128 gate rows of 128 H columns and the matching
// 128 up rows). One 256-thread workgroup per CU, one wave per SIMD; every wave multiplies 64
// activation rows by all 256 weight rows (64 blocks of mfma_f32_16x16x32_bf16, 256 fp32 accumulators
// per lane in AGPRs), so each activation row is used by exactly one wave and goes straight from
// global memory into MFMA operand registers: lane l of a 16-row fragment loads 16 bytes of row
// l % 16, the four lanes of a row one contiguous 64-byte run. Those loads run 3 K steps (3 x 32 K)
// ahead in four register buffers. The weight rows go through LDS: a ring of four 32 KiB slots,
// each holding the unit's 256 weight rows x 64 K (128 bytes per row: 8 whole rows x 128 B per load
// instruction), XOR-swizzled so that the 16-lane phases of the fragment reads cover all banks.
// Weight slices are staged through registers: slice j's first K step stores slice j + 2 into its
// slot and loads slice j + 3, one store and one load after every other MFMA group, so each weight
// load has a whole slice to arrive and each store a whole slice to land before the barrier that
// publishes it. Fragment reads run G4_WIN MFMA groups ahead of their use in a rolling window.
//
// Activation rows are dealt to the waves in 16-row groups round-robin (wave w, fragment f: rows
// 16 (4 f + w) ..), so a unit of at most 128 rows leaves every wave two fragments instead of idling
// whole SIMDs; such units run the body specialised for two fragments (half the MFMAs).
//
// The last, partial round of units: with at most half as many units left as workgroups, each of them
// runs as two column halves (64 H columns: 64 gate + 64 up weight rows, 8 fragments per K step) on
// two workgroups, so the round ends in about half the time and no workgroup idles through it. Every
// output element keeps its products and K order, so the bits do not change.
//
// e4m3 operands (gemm4w_gate_up_kernel<true>, the fp8 path's gate/up): the same units, ring, staging
// and activation loads, which move the same bytes (a row of K e4m3 values is K / 2 16-bit units).
// Each mfma_f32_16x16x128_f8f6f4 takes a whole 128-byte slice of both operands, so a slice runs its
// MFMAs once on the activation bytes of both bf16 steps. The epilogue dequantises first:
// acc * (s_w * s_a), weight-row and activation-row scales staged in LDS per unit (as the eight-wave
// kernel's e4m3 epilogue).
//
// The MFMAs are inline asm (see g4_mfma); every global and LDS access is an ordinary
// compiler-visible load or store, so the compiler's own waits track all of them, and the only
// hand-written synchronisation is the per-slice barrier.
#include "q38moe_common.h"
#include "q38moe_kernels.h"

namespace q38 {
namespace {

constexpr int G4_THREADS = 256;
constexpr int G4_BM = 256;                 // activation rows per unit (the tile table's block)
constexpr int G4_SLOT = 256 * 128;         // ring slot bytes: 256 weight rows x 64 K
constexpr int G4_NSLOT = 4;                // slices in the ring: multiplied, next, two being filled
constexpr int G4_PITCH = 256 + 16;         // epilogue staging row: 128 H columns, padded 16 bytes
constexpr int G4_STAGE = 16 * G4_PITCH;    // epilogue staging per wave: one 16-row fragment
constexpr int G4_XBUF = 4;                 // activation register buffers: loads run 3 K steps ahead
constexpr int G4_WIN = 8;                  // weight-fragment register window (MFMA groups ahead)

struct G4Params {
  const uint16_t* A;          // x [T, K]
  const int32_t* perm;        // routed rows: sorted row -> pair
  const int4* tiles;          // {group (E = shared expert), row0, rows, -}; nullptr = dense rows
  const int32_t* ntiles_dev;  // valid entries in tiles (device)
  int ntiles_host;            // dense launch: row tiles
  int64_t M;                  // dense launch: rows
  const uint16_t* W;          // routed weights: gate/up [E, 2N, K]
  const uint16_t* Ws_a;       // shared expert: gate [N, K]
  const uint16_t* Ws_b;       // shared expert: up [N, K]
  uint16_t* C;                // output rows H [*, N]
  int P;                      // first shared-expert row of the row space
  int N, K, E, topk;          // K: 16-bit units per row (bf16 elements, or pairs of e4m3 values)
  int ntiles_n;               // output-column tiles per row tile (N / 128)
  uint32_t a_bytes;           // bytes of A (rows x K x 2 < 2^32)
  // e4m3 operands only: dequantisation scales.
  const float* a_scale;       // per row of the row space (the H rows)
  const float* w_scale;       // routed weight rows [E, 2N]
  const float* ws_scale_a;    // shared expert gate rows [N]
  const float* ws_scale_b;    // shared expert up rows [N]
};

__device__ __forceinline__ int4 g4_tile_entry(const G4Params& p, int mt) {
  if (p.tiles != nullptr) {
    const uint64_t xy = load_uniform(reinterpret_cast<const uint64_t*>(p.tiles + mt));
    const int z = load_uniform(reinterpret_cast<const int*>(p.tiles + mt) + 2);
    return make_int4((int)(uint32_t)xy, (int)(uint32_t)(xy >> 32), z, 0);
  }
  const int row0 = mt * G4_BM;
  return make_int4(p.E, row0, (int)min((int64_t)G4_BM, p.M - (int64_t)row0), 0);
}

// Active 16-row fragments of wave w in a unit of z rows: fragment f covers rows 16 (4 f + w) ...
__device__ __forceinline__ int g4_nfrag(int z, int w) {
  const int groups = (z + 15) >> 4;
  return groups > w ? (groups - w + 3) >> 2 : 0;
}

// Buffer resource over `bytes` bytes at p (gfx9 dword 3): loads take a 32-bit per-lane offset and a
// scalar offset, so the base stays in SGPRs; reads past the range return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t g4_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t g4_bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Per-unit state: the unit's entry and the sources of its two operand streams.
struct G4Unit {
  int4 ti;
  int nt;                 // output-column tile
  int half;               // -1: all 128 columns of the tile; 0, 1: that 64-column half
  int rot;                // K-slice rotation (64-K slices)
  const uint8_t* wb;      // wave-uniform: the first of the 64 weight rows this wave stages (all K)
  uint32_t xo[4];         // byte offset of this lane's activation row of fragment f (+ 16 (lane / 16))
};

// Unit L's entry, rotation and the wave-uniform base of the weight rows it stages. K-slice order is
// rotated per expert (slice j of a unit of expert e is K slice (j + e) mod nk; shared-expert units
// rotate by row tile): the units of an expert run together on one XCD and meet in its L2 on the
// same rows at the same time, while different experts spread over the L2 channels.
// Work item L: unit L below U0; past it (split > 0), column half (L - U0) % 2 of unit U0 + (L - U0) / 2.
__device__ __forceinline__ void g4_unit_head(const G4Params& p, int L, int nk, int wave, int U0, bool split,
                                             G4Unit& u) {
  int Lu = L;
  u.half = -1;
  if (split && L >= U0) {
    Lu = U0 + ((L - U0) >> 1);
    u.half = (L - U0) & 1;
  }
  u.ti = g4_tile_entry(p, Lu / p.ntiles_n);
  u.nt = Lu % p.ntiles_n;
  u.rot = (u.ti.x < p.E ? u.ti.x : Lu / p.ntiles_n) % nk;
  const bool shared_grp = u.ti.x >= p.E;
  const int64_t K = p.K;
  // Staging load i of wave w carries weight rows 64 w + 8 i + lane / 8 of the unit: rows [0, 128)
  // are the gate rows of H columns nt * 128 + [0, 128), rows [128, 256) the matching up rows. A
  // column half has 128 weight rows, wave w staging rows 32 w + 8 i + lane / 8 (i < 4): rows
  // [0, 64) the gate rows of H columns nt * 128 + 64 half + [0, 64), rows [64, 128) the up rows.
  const bool up = wave >= 2;
  const uint16_t* base = shared_grp ? (up ? p.Ws_b : p.Ws_a)
                                    : p.W + (int64_t)u.ti.x * 2 * p.N * K + (up ? (int64_t)p.N * K : 0);
  const int row0 = u.half < 0 ? u.nt * 128 + 64 * (wave & 1) : u.nt * 128 + 64 * u.half + 32 * (wave & 1);
  u.wb = reinterpret_cast<const uint8_t*>(base + (int64_t)row0 * K);
}

// Row tile of work item L (the mapping of g4_unit_head).
__device__ __forceinline__ int g4_tile_index(const G4Params& p, int L, int U0, bool split) {
  return (split && L >= U0 ? U0 + ((L - U0) >> 1) : L) / p.ntiles_n;
}

// Source row index of this lane's fragment-f activation row: the sorted pair of a routed row (a
// load, resolved later by g4_unit_rows), else the row itself. Rows past the unit read its first
// row; their products reach only outputs that are never stored.
__device__ __forceinline__ void g4_row_sources(const G4Params& p, int4 ti, int wave, int lane, int (&src)[4]) {
  const bool gathered = ti.x < p.E;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int r = 16 * (4 * f + wave) + (lane & 15);
    const int row = ti.y + (r < ti.z ? r : 0);
    src[f] = gathered ? p.perm[row] : row;
  }
}

__device__ __forceinline__ void g4_unit_rows(const G4Params& p, int4 ti, int lane, const int (&src)[4], G4Unit& u) {
  const bool gathered = ti.x < p.E;
  const bool shared_grp = ti.x >= p.E && p.tiles != nullptr;
  const uint32_t K2 = 2u * (uint32_t)p.K;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    int row = src[f];
    if (gathered) row = row / p.topk;
    else if (shared_grp) row -= p.P;
    u.xo[f] = (uint32_t)row * K2 + 16u * (uint32_t)(lane >> 4);
  }
}

// Byte offset of 32-K step q (0 .. 2 nk - 1) of a unit with rotation rot.
__device__ __forceinline__ uint32_t g4_kbyte(int q, int rot, int nk) {
  int s = (q >> 1) + rot;
  s = s >= nk ? s - nk : s;
  return (uint32_t)s * 128u + (uint32_t)(q & 1) * 64u;
}

// Staging load i (0..7) of 64-K slice j of a unit: weight rows 64 w + 8 i + lane / 8, 16-byte chunk
// (lane % 8) ^ swizzle(row), swizzle(row) = (row / 2) % 8 = (4 i + lane / 16) % 8; the address is the
// unit's wave-uniform base plus this lane's offset wl[i % 2] (row lane / 8, its chunk). Its store,
// lane l's 16 bytes at byte 16 l of the wave's 1 KiB block i of a slot (8 rows x 128 B), puts row r's
// chunk c at position c ^ swizzle(r).
__device__ __forceinline__ u32x4_t g4_wload(const G4Unit& u, int j, int nk, uint32_t K2, const uint32_t (&wl)[2],
                                           int i) {
  int s = j + u.rot;
  s = s >= nk ? s - nk : s;
  return ld16(u.wb + (uint32_t)s * 128u + (size_t)i * 8u * K2 + wl[i & 1]);
}

// Per-slice barrier: publishes slice j (multiplied next) and slice j + 1 (whose first fragments the
// window reads during slice j's second step), both stored during earlier slices' first steps; this
// wave's stores and its reads of the slot the next stores refill are complete (LDS operations
// complete in order, and only the last G4_WIN fragment reads, which target slice j, may still be in
// flight: the second step of a slice stores nothing).
__device__ __forceinline__ void g4_barrier() { asm volatile("s_waitcnt lgkmcnt(8)\n\ts_barrier" ::: "memory"); }

// The MFMAs are issued from inline asm with the accumulator tied to its own AGPRs ("+a": dst = srcC).
// Through the builtin, the compiler at this register pressure (256 accumulators beside the operand
// and address registers) moved accumulators between AGPRs and VGPRs around half of the MFMAs. Being
// volatile, the asm MFMAs also keep the source order relative to the loads between them. Their
// operands come from compiler-visible loads, so the compiler still waits for those. The hazards it
// cannot see: a VALU write of an operand VGPR within two wait states before an MFMA (the compiler
// may keep an operand in AGPRs and copy it back with v_accvgpr_read just before its use) would be
// read stale; the build (csrc/build.py) scans this kernel's generated code and fails if any such
// write exists, so the MFMAs carry no s_nop. MFMA results read by VALU instructions are covered by
// g4_mfma_drain before every epilogue.
__device__ __forceinline__ void g4_mfma(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same with two wait states ahead: where AGPRs are free (a unit's first step, before its
// accumulators exist; the column-half units, which use half of them) the compiler parks operand
// VGPRs there and copies them back (v_accvgpr_read, a VALU write) right before their MFMA.
__device__ __forceinline__ void g4_mfma_nop(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void g4_mfma_first_nop(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}
// e4m3 x e4m3 (the f8f6f4 form with both formats e4m3, no block scales), 128 K per instruction:
// lane l holds 32 bytes of row l % 16 of each operand. The kernel fills them with bytes
// 16 (l / 16) .. + 16 and 64 + 16 (l / 16) .. + 16 of a 128-byte slice, in both operands, so each
// output is the dot product over the slice's 128 K in another order than the instruction's own.
__device__ __forceinline__ void g4_mfma8(f32x4_t& acc, const i32x8_t& a, const i32x8_t& b) {
  asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void g4_mfma8_nop(f32x4_t& acc, const i32x8_t& a, const i32x8_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void g4_mfma8_first_nop(f32x4_t& acc, const i32x8_t& a, const i32x8_t& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}
// Wait states between the last MFMA and VALU reads of its result (ample for the 8-pass bf16 and the
// 16-pass e4m3 XDL ops).
__device__ __forceinline__ void g4_mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Lane id computed in place (volatile: not hoisted or shared), so the epilogue's lane-derived
// offsets need no registers across the K loop.
__device__ __forceinline__ int g4_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Epilogue of one 16-row fragment: SwiGLU on the 4-column runs of the gate and up accumulators, then
// through the wave's staging area (rows padded by 16 bytes, so the 16 rows a write instruction spans
// start 4 banks apart: conflict-free writes and reads, and per-block offsets that are immediates) to
// whole-line stores (4 rows x 256 B per instruction).
// NW: weight fragments per K step (16; 8 for a column half: 64 columns, 2 rows x 128 B per store).
// FP8: the accumulators are dequantised first, acc * (s_w * s_a) with the weight row's and the
// activation row's scales (sc: 256 activation-row scales, then the unit's weight-row scales).
template <int NF, int NW, bool FP8>
__device__ __forceinline__ void g4_epilogue_frag(const G4Params& p, const f32x4_t (&acc)[NW][NF], const G4Unit& u,
                                                 int f, int wave, uint8_t* stage, const float* sc) {
  constexpr int NG = NW / 2;  // gate fragments (the up fragments follow)
  const int lane = g4_lane();
  const int lr = lane & 15, lq = lane >> 4;
  const int rbase = 16 * (4 * f + wave);
  uint8_t* const wr = stage + lr * G4_PITCH + 8 * lq;
  // Lane l holds weight rows 16 t + 4 (l / 16) + i (i = 0..3) of activation row rbase + l % 16. The
  // scales of fragment t + 1 are read before fragment t's arithmetic, so their LDS latency is hidden.
  const float sa = FP8 ? sc[rbase + lr] : 1.0f;
  const f32x4_t* const swp = reinterpret_cast<const f32x4_t*>(sc + 256 + 4 * lq);
  f32x4_t swg_n = {1.0f, 1.0f, 1.0f, 1.0f}, swu_n = swg_n;
  if constexpr (FP8) {
    swg_n = swp[0];
    swu_n = swp[4 * NG];
  }
#pragma unroll
  for (int t = 0; t < NG; ++t) {
    f32x4_t swg = swg_n, swu = swu_n;
    if constexpr (FP8) {
      swg *= sa;
      swu *= sa;
      if (t + 1 < NG) {
        swg_n = swp[4 * (t + 1)];
        swu_n = swp[4 * (t + 1 + NG)];
      }
    }
    uint32_t v[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      // Reference rounding (inference.py:90-96): bf16 gate and up, bf16 silu(gate), bf16 product.
      float g0, g1, u0, u1, s0, s1;
      if constexpr (FP8) {
        unpack_bf16x2(pack_bf16x2(acc[t][f][2 * h2] * swg[2 * h2], acc[t][f][2 * h2 + 1] * swg[2 * h2 + 1]), g0, g1);
        unpack_bf16x2(pack_bf16x2(acc[t + NG][f][2 * h2] * swu[2 * h2], acc[t + NG][f][2 * h2 + 1] * swu[2 * h2 + 1]),
                      u0, u1);
      } else {
        unpack_bf16x2(pack_bf16x2(acc[t][f][2 * h2], acc[t][f][2 * h2 + 1]), g0, g1);
        unpack_bf16x2(pack_bf16x2(acc[t + NG][f][2 * h2], acc[t + NG][f][2 * h2 + 1]), u0, u1);
      }
      unpack_bf16x2(pack_bf16x2(g0 * __builtin_amdgcn_rcpf(1.0f + __expf(-g0)),
                                g1 * __builtin_amdgcn_rcpf(1.0f + __expf(-g1))), s0, s1);
      v[h2] = pack_bf16x2(s0 * u0, s1 * u1);
    }
    *reinterpret_cast<uint2*>(wr + 32 * t) = make_uint2(v[0], v[1]);
  }
  if constexpr (NW == 16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = 4 * j + lq;
      const u32x4_t d = *reinterpret_cast<const u32x4_t*>(stage + rr * G4_PITCH + 16 * lr);
      const int r = rbase + rr;
      if (r < u.ti.z) st16(p.C + (int64_t)(u.ti.y + r) * p.N + u.nt * 128 + 8 * lr, d);
    }
  } else {
    const int l8 = lane & 7;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rr = 8 * j + (lane >> 3);
      const u32x4_t d = *reinterpret_cast<const u32x4_t*>(stage + rr * G4_PITCH + 16 * l8);
      const int r = rbase + rr;
      if (r < u.ti.z) st16(p.C + (int64_t)(u.ti.y + r) * p.N + u.nt * 128 + 64 * u.half + 8 * l8, d);
    }
  }
}

// Shared state of the unit loop, by reference into the specialised unit bodies.
struct G4State {
  uint8_t* ring;          // LDS ring base
  uint8_t* stage;         // this wave's staging area
  float* sc;              // e4m3: the unit's dequantisation scales (256 activation rows, then weight rows)
  uint32_t rd_off[2];     // this lane's fragment-read offset within a slot, for step half s = 0, 1
  uint32_t wl[2];         // this lane's staging-load source offsets (even, odd loads)
  uint32_t ws_lane;       // this lane's staging-store offset within the wave's block (16 lane)
  int wave;
  __amdgpu_buffer_rsrc_t xrs;  // the activation rows A
  int gslice;             // slices started so far (ring slot of the slice being multiplied = gslice % 4)
  int nk;                 // 64-K slices per unit
  uint32_t K2;
};

__device__ __forceinline__ int g4_slot(int g) { return g & (G4_NSLOT - 1); }

// This lane's read address of step half s's fragments in ring slot `slot` (fragment t at + 2048 t).
// The empty asm keeps the compiler from precomputing it for every slot outside the loops (those
// values would stay live across the whole kernel).
__device__ __forceinline__ const uint8_t* g4_frag_base(const G4State& st, int slot, int s) {
  uint32_t off = (uint32_t)(slot * G4_SLOT) + st.rd_off[s];
  asm volatile("" : "+v"(off));
  return st.ring + off;
}
__device__ __forceinline__ u32x4_t g4_frag(const uint8_t* base, int t) {
  return *reinterpret_cast<const u32x4_t*>(base + 2048 * t);
}
// The same for the staging stores of ring slot `slot`, for a unit (half: a column half, whose waves
// stage 32 rows each).
__device__ __forceinline__ uint8_t* g4_store_base(const G4State& st, int slot, bool half) {
  uint32_t off = (uint32_t)(slot * G4_SLOT) + (half ? 4096u : 8192u) * (uint32_t)st.wave + st.ws_lane;
  asm volatile("" : "+v"(off));
  return st.ring + off;
}

// One 32-K step: for each of the 16 weight fragments t, the NF MFMAs with activation buffer XB,
// then the read of fragment t + G4_WIN (this step's, from rcur; past 15 the next step's, from
// rnext, unless !RNEXT). After groups 1, 5, 9 and 13 the lookahead loads of the activation step 3
// ahead (XNF fragments into buffer XL, offsets xo at kb). WS (a slice's first step): after every
// other group, staging store i (wst[i] into the slot at wdst) and staging load i (slice wj of unit
// wu into wst[i]), so one memory instruction follows every MFMA group: all four waves run in step
// (the slice barriers), and a burst of them from each would queue at the CU's texture addresser
// while the waves waiting to issue leave their matrix pipes idle. FIRST: the unit's first step,
// whose MFMAs add to zero.
// NW (16, or 8 for a column half) groups; the activation loads then follow groups 1, 3, 5, 7. RT: the
// staged slices may belong to a unit of the other kind (the next unit's first slices, at a unit's
// end), so the counts of staging stores (nst) and loads (nld), 8 for a whole unit and 4 for a column
// half, are taken at run time.
template <int NF, int XNF, int XB, int XL, bool RNEXT, bool WS, bool FIRST, int NW, bool RT>
__device__ __forceinline__ void g4_step(f32x4_t (&acc)[NW][NF], u32x4_t (&wf)[G4_WIN], u32x4_t (&xb)[G4_XBUF][4],
                                        u32x4_t (&wst)[8], const G4State& st, const uint32_t (&xo)[4], uint32_t kb,
                                        const uint8_t* rcur, const uint8_t* rnext, uint8_t* wdst, const G4Unit& wu,
                                        int wj, int nst, int nld) {
  constexpr int XS = NW / 4;
#pragma unroll
  for (int t = 0; t < NW; ++t) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      // A unit's first step (its accumulators' AGPRs still free) and the column halves: see g4_mfma_nop.
      if (FIRST) g4_mfma_first_nop(acc[t][f], wf[t % G4_WIN], xb[XB][f]);
      else if constexpr (NW == 8) g4_mfma_nop(acc[t][f], wf[t % G4_WIN], xb[XB][f]);
      else g4_mfma(acc[t][f], wf[t % G4_WIN], xb[XB][f]);
    }
    if (t + G4_WIN < NW) wf[t % G4_WIN] = g4_frag(rcur, t + G4_WIN);
    else if (RNEXT) wf[t % G4_WIN] = g4_frag(rnext, t + G4_WIN - NW);
    if (t % XS == 1 && t / XS < XNF) xb[XL][t / XS] = g4_bload(st.xrs, xo[t / XS], kb);
    if (WS && (t & 1) == 0) {
      const int i = t >> 1;
      if (!RT || i < nst) *reinterpret_cast<u32x4_t*>(wdst + 1024 * i) = wst[i];
      if (!RT || i < nld) wst[i] = g4_wload(wu, wj, st.nk, st.K2, st.wl, i);
    }
  }
}

// One unit for a wave with NF (4, or 2 for units of at most 128 rows) fragments: 2 nk K steps, then
// the epilogue. On entry wf holds step 0's first G4_WIN fragments, xb[0..2] steps 0-2's activation
// loads, the ring slices 0 and 1 and wst slice 2 (loads issued); on exit the same holds for the next
// unit. Iterations of four slices (eight steps, two rounds of the activation buffers): the first (its
// first step starts the accumulators), steady ones, and the last, whose activation lookahead moves on
// to the next unit (its steps 0-2, all four fragments: its row count may differ). Slice j's first
// step stores slice j + 2 into the slot slice j - 2 used and loads slice j + 3 (this unit's, or the
// next unit's past the end).
template <int NF, int NW>
__device__ __forceinline__ void g4_unit(const G4Params& p, G4State& st, u32x4_t (&wf)[G4_WIN],
                                        u32x4_t (&xb)[G4_XBUF][4], u32x4_t (&wst)[8], const G4Unit& cur,
                                        const G4Unit& nxt, int wave) {
  // The unit's accumulators (AGPRs). Every value they take is an MFMA result (the first K step adds
  // to a zero operand): a zero initialisation, or values carried from unit to unit, would make the
  // compiler hold them in VGPRs across the K loop and copy them into AGPRs for every MFMA.
  f32x4_t acc[NW][NF];
  const int nk = st.nk, S = 2 * nk;
  // Staging counts and layout of the next unit (its first slices are staged during this unit's last
  // iteration).
  const bool nxt_half = nxt.half >= 0;
  const int nxt_n = nxt_half ? 4 : 8;
  // Step K_ (0..7) of the iteration starting at slice J: multiplies buffer K_ % 4, reads the next
  // step's fragments (none after the unit's last step), loads activation step q + 3 into buffer
  // (K_ + 3) % 4 (this unit's while q + 3 < S, else the next unit's step q + 3 - S).
#define Q38_G4_STEP(J, K_, FIRST_, LAST_)                                                                \
  do {                                                                                                  \
    const int j_ = (J) + (K_) / 2, q_ = 2 * j_ + ((K_) & 1);                                            \
    const uint8_t* rc_ = g4_frag_base(st, g4_slot(st.gslice), (K_) & 1);                                \
    const uint8_t* rn_ = g4_frag_base(st, g4_slot(st.gslice + ((K_) & 1)), ((K_) & 1) ^ 1);             \
    const bool sc_ = j_ + 2 < nk, wc_ = j_ + 3 < nk; /* slices j + 2, j + 3 this unit's */              \
    uint8_t* ws_ = nullptr;                                                                             \
    if (((K_) & 1) == 0) {                                                                              \
      g4_barrier();                                                                                     \
      ws_ = g4_store_base(st, g4_slot(st.gslice + 2), (LAST_) && !sc_ ? nxt_half : NW == 8);            \
    }                                                                                                   \
    const int nst_ = (LAST_) && !sc_ ? nxt_n : NW / 2, nld_ = (LAST_) && !wc_ ? nxt_n : NW / 2;         \
    if (!(LAST_) || (K_) < 5)                                                                           \
      g4_step<NF, NF, (K_) & 3, ((K_) + 3) & 3, true, ((K_) & 1) == 0, FIRST_ && (K_) == 0, NW, LAST_>(  \
          acc, wf, xb, wst, st, cur.xo, g4_kbyte(q_ + 3, cur.rot, nk), rc_, rn_, ws_, wc_ ? cur : nxt,  \
          wc_ ? j_ + 3 : j_ + 3 - nk, nst_, nld_);                                                      \
    else                                                                                                \
      g4_step<NF, 4, (K_) & 3, ((K_) + 3) & 3, (K_) != 7, ((K_) & 1) == 0, false, NW, LAST_>(            \
          acc, wf, xb, wst, st, nxt.xo, g4_kbyte(q_ + 3 - S, nxt.rot, nk), rc_, rn_, ws_, wc_ ? cur : nxt, \
          wc_ ? j_ + 3 : j_ + 3 - nk, nst_, nld_);                                                      \
    if ((K_) & 1) ++st.gslice;                                                                          \
  } while (0)
#define Q38_G4_ITER(J, FIRST_, LAST_)                                                                   \
  do {                                                                                                  \
    Q38_G4_STEP(J, 0, FIRST_, LAST_); Q38_G4_STEP(J, 1, FIRST_, LAST_);                                 \
    Q38_G4_STEP(J, 2, FIRST_, LAST_); Q38_G4_STEP(J, 3, FIRST_, LAST_);                                 \
    Q38_G4_STEP(J, 4, FIRST_, LAST_); Q38_G4_STEP(J, 5, FIRST_, LAST_);                                 \
    Q38_G4_STEP(J, 6, FIRST_, LAST_); Q38_G4_STEP(J, 7, FIRST_, LAST_);                                 \
  } while (0)
  Q38_G4_ITER(0, true, false);
  for (int j = 4; j < nk - 4; j += 4) Q38_G4_ITER(j, false, false);
  Q38_G4_ITER(nk - 4, false, true);
#undef Q38_G4_ITER
#undef Q38_G4_STEP
  g4_mfma_drain();
  const int nf = g4_nfrag(cur.ti.z, wave);
#pragma unroll
  for (int f = 0; f < NF; ++f)
    if (f < nf) g4_epilogue_frag<NF, NW, false>(p, acc, cur, f, wave, st.stage, st.sc);
  // The next unit's first fragments (its slice 0 was published by the last barrier).
  {
    const uint8_t* const rb = g4_frag_base(st, g4_slot(st.gslice), 0);
#pragma unroll
    for (int t = 0; t < G4_WIN; ++t) wf[t] = g4_frag(rb, t);
  }
}

// ---- e4m3 operands -------------------------------------------------------------------------------
// The same units, ring, staging and activation loads (a row of K e4m3 values is K / 2 16-bit units,
// so every byte offset above holds); an MFMA takes a whole 128-byte slice of its two operands, the
// bytes the two 32-K steps of the bf16 kernel load, so the MFMAs of a slice run once per slice on
// both halves together. Activation buffers hold whole slices (two: slice j multiplies one while
// slice j + 1 loads into the other), the weight window whole-slice fragment pairs.
constexpr int G4_WIN8 = 4;  // weight-fragment pairs read ahead (MFMA groups)

__device__ __forceinline__ i32x8_t g4_cat(const u32x4_t& lo, const u32x4_t& hi) {
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}
// Fragment t of a slice: its two step halves (bases of g4_frag_base with s = 0, 1).
__device__ __forceinline__ i32x8_t g4_frag8(const uint8_t* b0, const uint8_t* b1, int t) {
  return g4_cat(g4_frag(b0, t), g4_frag(b1, t));
}
// This lane's activation bytes of a slice: the two step halves at kb0, kb1 (g4_kbyte of steps 2j, 2j+1).
__device__ __forceinline__ i32x8_t g4_bload8(__amdgpu_buffer_rsrc_t r, uint32_t xo, uint32_t kb0, uint32_t kb1) {
  return g4_cat(g4_bload(r, xo, kb0), g4_bload(r, xo, kb1));
}

// One 128-K slice: for each of the NW weight fragments t, the NF MFMAs with activation buffer XB,
// then the read of pair t + G4_WIN8 (this slice's, from rc0/rc1; past NW - 1 the next slice's, from
// rn0/rn1, unless !RNEXT). After groups 0-7 the loads of the next slice's activation fragments, one
// per group (group t: step half t % 2 of fragment t / 2, for XNF fragments, into buffer XB ^ 1,
// offsets xo at kb0, kb1): every MFMA of a slice reads all four fragments, so they go in the first
// half. Staging store i (wst[i], loaded one slice earlier, into the slot at wdst) after group
// ST0 + i, staging load i (slice wj of unit wu into wst[i]) after group LD0 + i (>= ST0 + i). The
// stores end four groups before the slice does, so at least eight fragment reads (two per group)
// follow the last of them: the next slice's barrier waits for all but eight of this wave's LDS
// operations, which LDS completes in order, so it publishes every store. Bursts of memory instructions stall
// the issuing wave: all eight activation loads after groups 0 and 1 ran 5 us slower at
// configuration 4 than two after each of groups 0-3. FIRST, RT: as g4_step.
template <int NF, int XNF, int XB, bool RNEXT, bool FIRST, int NW, bool RT>
__device__ __forceinline__ void g4_slice8(f32x4_t (&acc)[NW][NF], i32x8_t (&wp)[G4_WIN8], i32x8_t (&xb)[2][4],
                                          u32x4_t (&wst)[8], const G4State& st, const uint32_t (&xo)[4],
                                          uint32_t kb0, uint32_t kb1, const uint8_t* rc0, const uint8_t* rc1,
                                          const uint8_t* rn0, const uint8_t* rn1, uint8_t* wdst, const G4Unit& wu,
                                          int wj, int nst, int nld) {
  constexpr int ST0 = NW / 2 - 4;          // staging stores after groups ST0 .. NW - 5
  constexpr int LD0 = NW == 16 ? 8 : 0;    // staging loads after groups LD0 .. LD0 + NW/2 - 1
#pragma unroll
  for (int t = 0; t < NW; ++t) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (FIRST) g4_mfma8_first_nop(acc[t][f], wp[t % G4_WIN8], xb[XB][f]);
      else if constexpr (NW == 8) g4_mfma8_nop(acc[t][f], wp[t % G4_WIN8], xb[XB][f]);
      else g4_mfma8(acc[t][f], wp[t % G4_WIN8], xb[XB][f]);
    }
    if (t + G4_WIN8 < NW) wp[t % G4_WIN8] = g4_frag8(rc0, rc1, t + G4_WIN8);
    else if (RNEXT) wp[t % G4_WIN8] = g4_frag8(rn0, rn1, t + G4_WIN8 - NW);
    if (t < 8 && (t >> 1) < XNF) {
      const u32x4_t h = g4_bload(st.xrs, xo[t >> 1], (t & 1) ? kb1 : kb0);
      i32x8_t& d = xb[XB ^ 1][t >> 1];
      if (t & 1) {
        d[4] = (int)h[0]; d[5] = (int)h[1]; d[6] = (int)h[2]; d[7] = (int)h[3];
      } else {
        d[0] = (int)h[0]; d[1] = (int)h[1]; d[2] = (int)h[2]; d[3] = (int)h[3];
      }
    }
    if (t >= ST0 && t - ST0 < NW / 2) {
      const int i = t - ST0;
      if (!RT || i < nst) *reinterpret_cast<u32x4_t*>(wdst + 1024 * i) = wst[i];
    }
    if (t >= LD0 && t - LD0 < NW / 2) {
      const int i = t - LD0;
      if (!RT || i < nld) wst[i] = g4_wload(wu, wj, st.nk, st.K2, st.wl, i);
    }
  }
}

// Dequantisation scale of weight row r (0 .. 16 NW - 1) of unit u (the staging rows' mapping).
__device__ __forceinline__ float g4_weight_scale(const G4Params& p, const G4Unit& u, int r) {
  const int nwr = u.half < 0 ? 256 : 128;
  const bool up = r >= nwr / 2;
  const int col = u.nt * 128 + (u.half < 0 ? 0 : 64 * u.half) + (up ? r - nwr / 2 : r);
  if (u.ti.x >= p.E) return (up ? p.ws_scale_b : p.ws_scale_a)[col];
  return p.w_scale[(int64_t)u.ti.x * 2 * p.N + (up ? p.N : 0) + col];
}

// One unit on e4m3 operands (as g4_unit): nk slices in iterations of four, then the epilogue. On
// entry wp holds slice 0's first G4_WIN8 pairs, xb[0] slice 0's activation loads, the ring slices 0
// and 1 and wst slice 2 (loads issued). The unit's scales are loaded at its start and stored to LDS
// after its first iteration, whose barriers have retired every read of the previous unit's.
template <int NF, int NW>
__device__ __forceinline__ void g4_unit8(const G4Params& p, G4State& st, i32x8_t (&wp)[G4_WIN8],
                                         i32x8_t (&xb)[2][4], u32x4_t (&wst)[8], const G4Unit& cur,
                                         const G4Unit& nxt, int wave) {
  f32x4_t acc[NW][NF];
  const int nk = st.nk;
  const bool nxt_half = nxt.half >= 0;
  const int nxt_n = nxt_half ? 4 : 8;
  const int tid = 64 * wave + g4_lane();
  const float s_a = p.a_scale[cur.ti.y + (tid < cur.ti.z ? tid : 0)];
  const float s_w = tid < 16 * NW ? g4_weight_scale(p, cur, tid) : 0.0f;
#define Q38_G8_SLICE(J, S_, FIRST_, LAST_)                                                               \
  do {                                                                                                  \
    const int j_ = (J) + (S_);                                                                          \
    const uint8_t* rc0_ = g4_frag_base(st, g4_slot(st.gslice), 0);                                      \
    const uint8_t* rc1_ = g4_frag_base(st, g4_slot(st.gslice), 1);                                      \
    const uint8_t* rn0_ = g4_frag_base(st, g4_slot(st.gslice + 1), 0);                                  \
    const uint8_t* rn1_ = g4_frag_base(st, g4_slot(st.gslice + 1), 1);                                  \
    const bool sc_ = j_ + 2 < nk, wc_ = j_ + 3 < nk; /* slices j + 2, j + 3 this unit's */              \
    g4_barrier();                                                                                       \
    uint8_t* ws_ = g4_store_base(st, g4_slot(st.gslice + 2), (LAST_) && !sc_ ? nxt_half : NW == 8);     \
    const int nst_ = (LAST_) && !sc_ ? nxt_n : NW / 2, nld_ = (LAST_) && !wc_ ? nxt_n : NW / 2;         \
    if (!(LAST_) || (S_) < 3)                                                                           \
      g4_slice8<NF, NF, (S_) & 1, true, FIRST_ && (S_) == 0, NW, LAST_>(                                \
          acc, wp, xb, wst, st, cur.xo, g4_kbyte(2 * j_ + 2, cur.rot, nk), g4_kbyte(2 * j_ + 3, cur.rot, nk), \
          rc0_, rc1_, rn0_, rn1_, ws_, wc_ ? cur : nxt, wc_ ? j_ + 3 : j_ + 3 - nk, nst_, nld_);         \
    else                                                                                                \
      g4_slice8<NF, 4, (S_) & 1, false, false, NW, LAST_>(                                              \
          acc, wp, xb, wst, st, nxt.xo, g4_kbyte(0, nxt.rot, nk), g4_kbyte(1, nxt.rot, nk), rc0_, rc1_, \
          rn0_, rn1_, ws_, wc_ ? cur : nxt, wc_ ? j_ + 3 : j_ + 3 - nk, nst_, nld_);                     \
    ++st.gslice;                                                                                        \
  } while (0)
#define Q38_G8_ITER(J, FIRST_, LAST_)                                                                   \
  do {                                                                                                  \
    Q38_G8_SLICE(J, 0, FIRST_, LAST_); Q38_G8_SLICE(J, 1, FIRST_, LAST_);                               \
    Q38_G8_SLICE(J, 2, FIRST_, LAST_); Q38_G8_SLICE(J, 3, FIRST_, LAST_);                               \
  } while (0)
  Q38_G8_ITER(0, true, false);
  st.sc[tid] = s_a;
  if (tid < 16 * NW) st.sc[256 + tid] = s_w;
  for (int j = 4; j < nk - 4; j += 4) Q38_G8_ITER(j, false, false);
  Q38_G8_ITER(nk - 4, false, true);
#undef Q38_G8_ITER
#undef Q38_G8_SLICE
  g4_mfma_drain();
  const int nf = g4_nfrag(cur.ti.z, wave);
#pragma unroll
  for (int f = 0; f < NF; ++f)
    if (f < nf) g4_epilogue_frag<NF, NW, true>(p, acc, cur, f, wave, st.stage, st.sc);
  {
    const uint8_t* const b0 = g4_frag_base(st, g4_slot(st.gslice), 0);
    const uint8_t* const b1 = g4_frag_base(st, g4_slot(st.gslice), 1);
#pragma unroll
    for (int t = 0; t < G4_WIN8; ++t) wp[t] = g4_frag8(b0, b1, t);
  }
}

// FP8: e4m3 activations and weights (g4_unit8) with per-row dequantisation scales.
template <bool FP8>
__global__ __launch_bounds__(G4_THREADS, 1) void gemm4w_gate_up_kernel(G4Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[G4_NSLOT * G4_SLOT];
  __shared__ __attribute__((aligned(16))) uint8_t stage[4 * G4_STAGE];
  __shared__ __attribute__((aligned(16))) float scales[FP8 ? 512 : 4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  // Slots are spread over the 8 XCDs in contiguous runs (workgroup b runs on XCD b % 8), so units
  // that share an expert's weights or gathered rows run in one XCD's L2 at the same time.
  const int slot = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
  const int units = (p.tiles != nullptr ? load_uniform(p.ntiles_dev) : p.ntiles_host) * p.ntiles_n;
  // The last, partial round (units U0 ..): split into column halves when they fit one round.
  const int U0 = units - units % G;
  const bool split = units > U0 && 2 * (units - U0) <= G;
  const int used = split ? U0 + 2 * (units - U0) : units;  // work items
  if (slot >= used) return;
  int L = slot;
  const int nk = p.K >> 6;

  G4State st;
  st.ring = ring;
  st.stage = stage + wave * G4_STAGE;
  st.sc = scales;
  st.gslice = 0;
  st.nk = nk;
  st.K2 = 2u * (uint32_t)p.K;
  st.xrs = g4_rsrc(p.A, p.a_bytes);
  st.ws_lane = 16u * (uint32_t)lane;
  st.wave = wave;
  {
    const uint32_t c0 = (uint32_t)((lane & 7) ^ (lane >> 4));
    st.wl[0] = (uint32_t)(lane >> 3) * st.K2 + 16u * c0;
    st.wl[1] = (uint32_t)(lane >> 3) * st.K2 + 16u * (c0 ^ 4u);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int row = lane & 15;
    const int c = 4 * s + (lane >> 4);
    st.rd_off[s] = (uint32_t)(row * 128 + ((c ^ ((lane >> 1) & 7)) << 4));
  }

  // Units: cur (L), nxt (L + G; the current one again past the end, whose loads then go unused),
  // and the row sources of the one after, loaded a unit ahead of their use.
  G4Unit cur, nxt;
  int src[4], src2[4];
  g4_unit_head(p, L, nk, wave, U0, split, cur);
  g4_row_sources(p, cur.ti, wave, lane, src);
  g4_unit_rows(p, cur.ti, lane, src, cur);
  int Ln = L + G < used ? L + G : L;
  g4_unit_head(p, Ln, nk, wave, U0, split, nxt);
  g4_row_sources(p, nxt.ti, wave, lane, src);
  g4_unit_rows(p, nxt.ti, lane, src, nxt);
  int Lnn = Ln + G < used ? Ln + G : Ln;
  int4 tinn = g4_tile_entry(p, g4_tile_index(p, Lnn, U0, split));
  g4_row_sources(p, tinn, wave, lane, src2);

  // Prologue: slices 0 and 1 into the ring, slice 2 in wst; activation steps 0-2 in flight (e4m3:
  // slice 0); step 0's fragments (e4m3: slice 0's first pairs).
  u32x4_t wst[8];
  const bool half0 = cur.half >= 0;
  const int n0 = half0 ? 4 : 8;
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < n0) wst[i] = g4_wload(cur, sl, nk, st.K2, st.wl, i);
    uint8_t* const dst = g4_store_base(st, sl, half0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < n0) *reinterpret_cast<u32x4_t*>(dst + 1024 * i) = wst[i];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (i < n0) wst[i] = g4_wload(cur, 2, nk, st.K2, st.wl, i);
  const int nf0 = cur.ti.z > 128 ? 4 : 2;
  // After a unit (Ln != L): on to the next one.
#define Q38_G4_NEXT()                                                                                    \
  L = Ln;                                                                                               \
  cur = nxt;                                                                                            \
  Ln = Lnn;                                                                                             \
  g4_unit_head(p, Ln, nk, wave, U0, split, nxt);                                                        \
  g4_unit_rows(p, nxt.ti, lane, src2, nxt);                                                             \
  Lnn = Ln + G < used ? Ln + G : Ln;                                                                    \
  tinn = g4_tile_entry(p, g4_tile_index(p, Lnn, U0, split));                                            \
  g4_row_sources(p, tinn, wave, lane, src2)
  // Units of at most 128 rows: every wave has at most two active fragments.
  if constexpr (FP8) {
    i32x8_t wp[G4_WIN8], xb[2][4];
#pragma unroll
    for (int f = 0; f < 4; ++f)
      if (f < nf0) xb[0][f] = g4_bload8(st.xrs, cur.xo[f], g4_kbyte(0, cur.rot, nk), g4_kbyte(1, cur.rot, nk));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int t = 0; t < G4_WIN8; ++t) wp[t] = g4_frag8(g4_frag_base(st, 0, 0), g4_frag_base(st, 0, 1), t);
    // (A loop of the same form as the bf16 one below left the register allocator 30 VGPRs short.)
    auto advance = [&]() -> bool {
      if (Ln == L) return false;
      Q38_G4_NEXT();
      return true;
    };
    do {
      if (cur.half < 0) {
        if (cur.ti.z > 128) g4_unit8<4, 16>(p, st, wp, xb, wst, cur, nxt, wave);
        else g4_unit8<2, 16>(p, st, wp, xb, wst, cur, nxt, wave);
      } else {
        if (cur.ti.z > 128) g4_unit8<4, 8>(p, st, wp, xb, wst, cur, nxt, wave);
        else g4_unit8<2, 8>(p, st, wp, xb, wst, cur, nxt, wave);
      }
    } while (advance());
  } else {
    u32x4_t wf[G4_WIN], xb[G4_XBUF][4];
#pragma unroll
    for (int q = 0; q < G4_XBUF - 1; ++q)
#pragma unroll
      for (int f = 0; f < 4; ++f)
        if (f < nf0) xb[q][f] = g4_bload(st.xrs, cur.xo[f], g4_kbyte(q, cur.rot, nk));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int t = 0; t < G4_WIN; ++t) wf[t] = g4_frag(g4_frag_base(st, 0, 0), t);
    for (;;) {
      if (cur.half < 0) {
        if (cur.ti.z > 128) g4_unit<4, 16>(p, st, wf, xb, wst, cur, nxt, wave);
        else g4_unit<2, 16>(p, st, wf, xb, wst, cur, nxt, wave);
      } else {
        if (cur.ti.z > 128) g4_unit<4, 8>(p, st, wf, xb, wst, cur, nxt, wave);
        else g4_unit<2, 8>(p, st, wf, xb, wst, cur, nxt, wave);
      }
      if (Ln == L) break;
      Q38_G4_NEXT();
    }
  }
#undef Q38_G4_NEXT
  // Retire the lookahead loads of the (absent) next unit before the wave ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace

// The four-wave kernel runs the bf16 gate/up launch when K (= h) is a multiple of 256 (>= 512: units
// are iterations of four 64-K slices, the first and the last distinct), the H columns fill whole
// units (N % 128 == 0) and the activation rows' byte offsets fit 32 bits. The down launch stays on
// the eight-wave kernel: at K = I = 256 its epilogue, which writes twice the columns of gate/up's, is
// a large share of each unit, and with one wave per SIMD nothing overlaps it.
bool gemm4w_supported(int N, int K, int64_t a_rows) {
  if (K < 512 || K % 256 != 0 || N % 128 != 0) return false;
  return a_rows * 2 * (int64_t)K < ((int64_t)1 << 32);
}

// K in 16-bit units (e4m3: K / 2 of the elements); scales only with fp8.
static hipError_t gate_up_4w_impl(const void* x, int64_t x_rows, const int32_t* perm, const int4* tiles,
                                  const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                                  const void* w_gate_up, const void* ws_gate, const void* ws_up, uint16_t* H,
                                  int N, int K, int E, int topk, bool fp8, const float* a_scale,
                                  const float* w_scale, const float* ws_scale_gate, const float* ws_scale_up,
                                  hipStream_t stream) {
  if (!gemm4w_supported(N, K, x_rows)) return hipErrorInvalidValue;
  G4Params p;
  p.A = static_cast<const uint16_t*>(x);
  p.perm = perm;
  p.tiles = tiles;
  p.ntiles_dev = ntiles_dev;
  p.ntiles_host = tiles != nullptr ? 0 : (int)((M_dense + G4_BM - 1) / G4_BM);
  p.M = M_dense;
  p.W = static_cast<const uint16_t*>(w_gate_up);
  p.Ws_a = static_cast<const uint16_t*>(ws_gate);
  p.Ws_b = static_cast<const uint16_t*>(ws_up);
  p.C = H;
  p.P = P;
  p.N = N;
  p.K = K;
  p.E = E;
  p.topk = topk;
  p.ntiles_n = N / 128;
  p.a_bytes = (uint32_t)(x_rows * 2 * (int64_t)K);
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.ws_scale_a = ws_scale_gate;
  p.ws_scale_b = ws_scale_up;
  const int mt = tiles != nullptr ? max_mtiles : p.ntiles_host;
  if (mt == 0) return hipSuccess;
  const int cus = device_cus();
  const int64_t units = (int64_t)mt * p.ntiles_n;
  const dim3 grid((unsigned)(units < cus ? units : cus));
  if (fp8) hipLaunchKernelGGL(gemm4w_gate_up_kernel<true>, grid, dim3(G4_THREADS), 0, stream, p);
  else hipLaunchKernelGGL(gemm4w_gate_up_kernel<false>, grid, dim3(G4_THREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_gate_up_4w(const uint16_t* x, int64_t x_rows, const int32_t* perm, const int4* tiles,
                             const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                             const uint16_t* w_gate_up, const uint16_t* ws_gate, const uint16_t* ws_up, uint16_t* H,
                             int N, int K, int E, int topk, hipStream_t stream) {
  return gate_up_4w_impl(x, x_rows, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, w_gate_up, ws_gate, ws_up, H, N,
                         K, E, topk, false, nullptr, nullptr, nullptr, nullptr, stream);
}

hipError_t launch_gate_up_4w_fp8(const uint8_t* xq, int64_t x_rows, const int32_t* perm, const int4* tiles,
                                 const int32_t* ntiles_dev, int max_mtiles, int64_t M_dense, int P,
                                 const float* a_scale, const uint8_t* wq_gate_up, const float* s_gate_up,
                                 const uint8_t* wq_sh_gate, const float* s_sh_gate, const uint8_t* wq_sh_up,
                                 const float* s_sh_up, uint16_t* H, int N, int K, int E, int topk,
                                 hipStream_t stream) {
  if (K % 2 != 0) return hipErrorInvalidValue;
  return gate_up_4w_impl(xq, x_rows, perm, tiles, ntiles_dev, max_mtiles, M_dense, P, wq_gate_up, wq_sh_gate,
                         wq_sh_up, H, N, K / 2, E, topk, true, a_scale, s_gate_up, s_sh_gate, s_sh_up, stream);
}

}  // namespace q38
