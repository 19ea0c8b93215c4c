// C ABI of libq38moe.so: argument validation, workspace carving and kernel sequencing.
// Declarations and the reference function each entry point replaces: include/q38moe.h.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <mutex>

#include "q38moe.h"
#include "q38moe_kernels.h"

namespace {

thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(Q38MOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define Q38_HIP(call, what)                      \
  do {                                           \
    hipError_t e_ = (call);                      \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_ptr(const void* p, const char* name) {
  if (p == nullptr) return fail(Q38MOE_EINVAL, "%s must not be NULL", name);
  if (!aligned16(p)) return fail(Q38MOE_EINVAL, "%s must be 16-byte aligned", name);
  return Q38MOE_OK;
}

int check_opt_ptr(const void* p, const char* name) {
  if (p != nullptr && !aligned16(p)) return fail(Q38MOE_EINVAL, "%s must be 16-byte aligned", name);
  return Q38MOE_OK;
}

int check_dtype(int32_t dtype) {
  if (dtype != Q38MOE_BF16 && dtype != Q38MOE_FP32)
    return fail(Q38MOE_EINVAL, "unsupported dtype %d (Q38MOE_BF16 or Q38MOE_FP32)", dtype);
  return Q38MOE_OK;
}

size_t elem_size(int32_t dtype) { return dtype == Q38MOE_FP32 ? 4 : 2; }

int check_routing(int64_t T, int32_t E, int32_t k) {
  if (T < 0) return fail(Q38MOE_EINVAL, "T must be >= 0 (got %lld)", (long long)T);
  if (E < 1 || E > 64) return fail(Q38MOE_EINVAL, "E must be in [1, 64] (got %d)", E);
  if (k < 1 || k > 8 || k > E) return fail(Q38MOE_EINVAL, "k must be in [1, min(8, E)] (got k=%d, E=%d)", k, E);
  if (T * (int64_t)k >= (int64_t)1 << 31) return fail(Q38MOE_EINVAL, "T*k must be < 2^31");
  return Q38MOE_OK;
}

int check_dim(int32_t v, const char* name) {
  if (v < 64 || v % 64 != 0) return fail(Q38MOE_EINVAL, "%s must be a positive multiple of 64 (got %d)", name, v);
  return Q38MOE_OK;
}

#define Q38_CHECK(expr)         \
  do {                          \
    int rc_ = (expr);           \
    if (rc_ != Q38MOE_OK) return rc_; \
  } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int64_t hist_blocks(int64_t T) { return (T + 63) / 64; }

// GEMM tiling by shape. The persistent kernels (q38moe_gemm.hip, q38moe_gemm4w.hip) hand each CU
// whole (256-row tile, 256 weight rows) units: with few rows per expert those units are few, each
// streams 512 KiB (h = 1024) of one expert's weights through one CU, and the kernels' time stays near
// 20-30 us (configuration 2's shapes) from T = 1 up to T ~ 1000. The small-tile kernels
// (q38moe_gemm_small.hip: 16 weight rows per workgroup, K split over its waves, every weight block in
// flight at once) take 6 us (gate/up) and 4 us (down) at T = 1 but grow with the rows per expert,
// since each workgroup walks its rows in 16-row blocks, and their cost per row grows with K. The
// rule takes the small tiles up to R(h, I) rows per group on average (E experts + the shared group),
// R = 32 (2^18 / (h I))^(1/3): the measured block crossovers (MI355X, both tilings forced) are about
// 32-40 rows per group at h = 1024, I = 256 (configuration 2; R = 32) and about 23 at h = 2048,
// I = 512 (configuration 4's shapes in bf16; R = 20). Q38MOE_GEMM_TILING=small|persistent (read once)
// overrides the rule, to time one tiling against the other on the same shapes.
int tiling_override() {
  static const int v = [] {
    const char* e = std::getenv("Q38MOE_GEMM_TILING");
    if (e == nullptr) return 0;
    if (std::strcmp(e, "small") == 0) return Q38MOE_TILING_SMALL;
    if (std::strcmp(e, "persistent") == 0) return Q38MOE_TILING_PERSISTENT;
    return 0;
  }();
  return v;
}
double small_rows_per_group(int32_t h, int32_t I) {
  const double r = 32.0 * std::cbrt(262144.0 / ((double)h * (double)I));
  return r < 8.0 ? 8.0 : (r > 64.0 ? 64.0 : r);
}
bool small_tiles(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows) {
  if (!q38::small_gemm_supported(h) || !q38::small_gemm_supported(I)) return false;
  if (tiling_override() != 0) return tiling_override() == Q38MOE_TILING_SMALL;
  return (double)(T * k + shared_rows) <= small_rows_per_group(h, I) * (double)(E + (shared_rows > 0 ? 1 : 0));
}

// The e4m3 path takes its small tiles (q38moe_gemm_small.hip, gemm_small_fp8_kernel) under the same
// kind of rule with F = 1.25 R rows per group: at configuration 4's shapes (h = 2048, I = 512) the
// measured block crossover with the persistent fp8 kernel is near T = 280 (26 rows per group: block
// 119.9 against 132.4 us at T = 200, 134.3 against 132.6 at T = 300; at T = 1, 72 against 95 us).
double small_rows_per_group_fp8(int32_t h, int32_t I) { return 1.25 * small_rows_per_group(h, I); }
bool small_tiles_fp8(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows) {
  if (!q38::small_gemm_fp8_supported(h) || !q38::small_gemm_fp8_supported(I)) return false;
  if (tiling_override() != 0) return tiling_override() == Q38MOE_TILING_SMALL;
  return (double)(T * k + shared_rows) <= small_rows_per_group_fp8(h, I) * (double)(E + (shared_rows > 0 ? 1 : 0));
}

hipError_t gate_up_fp8_any(const uint8_t* xq, const float* a_scale, const int32_t* perm, const int4* tiles,
                           const int32_t* tile_count, int max_tiles, int64_t T, int32_t k, int64_t shared_rows,
                           const uint8_t* wq, const float* sw, const uint8_t* wq_sg, const float* s_sg,
                           const uint8_t* wq_su, const float* s_su, uint16_t* H, int32_t I, int32_t h, int32_t E,
                           hipStream_t st) {
  if (small_tiles_fp8(T, h, E, k, I, shared_rows))
    return q38::launch_gate_up_small_fp8(xq, a_scale, perm, tiles, tile_count, max_tiles, (int)(T * k),
                                         (int)shared_rows, wq, sw, wq_sg, s_sg, wq_su, s_su, H, I, h, E, k, st);
  return q38::launch_gate_up_fp8(xq, perm, tiles, tile_count, max_tiles, 0, (int)(T * k), a_scale, wq, sw, wq_sg, s_sg,
                                 wq_su, s_su, H, I, h, E, k, st);
}

hipError_t down_fp8_any(const uint8_t* Hq, const float* a_scale, const int4* tiles, const int32_t* tile_count,
                        int max_tiles, int64_t T, int32_t k, int64_t shared_rows, const uint8_t* wq, const float* sw,
                        const uint8_t* wq_sd, const float* s_sd, uint16_t* Y, int32_t I, int32_t h, int32_t E,
                        hipStream_t st) {
  if (small_tiles_fp8(T, h, E, k, I, shared_rows))
    return q38::launch_down_small_fp8(Hq, a_scale, tiles, tile_count, max_tiles, (int)(T * k), (int)shared_rows, wq,
                                      sw, wq_sd, s_sd, Y, h, I, E, st);
  return q38::launch_down_fp8(Hq, tiles, tile_count, max_tiles, 0, a_scale, wq, sw, wq_sd, s_sd, Y, h, I, E, st);
}

hipError_t gate_up_bf16(const uint16_t* x, const int32_t* perm, const int4* tiles, const int32_t* tile_count,
                        int max_tiles, int64_t T, int32_t k, int64_t shared_rows, const uint16_t* w_gate_up,
                        const uint16_t* sh_gate, const uint16_t* sh_up, uint16_t* H, int32_t I, int32_t h, int32_t E,
                        hipStream_t st) {
  if (small_tiles(T, h, E, k, I, shared_rows))
    return q38::launch_gate_up_small(x, perm, tiles, tile_count, max_tiles, (int)(T * k), (int)shared_rows, w_gate_up,
                                     sh_gate, sh_up, H, I, h, E, k, st);
  return q38::launch_gate_up(x, perm, tiles, tile_count, max_tiles, 0, (int)(T * k), w_gate_up, sh_gate, sh_up, H, I,
                             h, E, k, st);
}

hipError_t down_bf16(const uint16_t* H, const int4* tiles, const int32_t* tile_count, int max_tiles, int64_t T,
                     int32_t k, int64_t shared_rows, const uint16_t* w_down, const uint16_t* sh_down, uint16_t* Y,
                     int32_t I, int32_t h, int32_t E, hipStream_t st) {
  if (small_tiles(T, h, E, k, I, shared_rows))
    return q38::launch_down_small(H, tiles, tile_count, max_tiles, (int)(T * k), (int)shared_rows, w_down, sh_down, Y,
                                  h, I, E, st);
  return q38::launch_down(H, tiles, tile_count, max_tiles, 0, w_down, sh_down, Y, h, I, E, st);
}

int64_t max_tiles_impl(int64_t T, int32_t E, int32_t k, int64_t shared_rows) {
  const int64_t bm = q38::gemm_block_m();
  return (T * k + bm - 1) / bm + E + (shared_rows + bm - 1) / bm;
}

// Workspace of the routed-experts pipeline. With shared_rows > 0 the shared expert's rows are
// appended to H and Y (rows T*k ..) and its tiles to the tile table.
struct ExpertsWs {
  size_t hist, counts, starts, perm, inv, tiles, tile_count, H, Y, end;
  int64_t max_tiles;
};

ExpertsWs experts_layout(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows,
                         size_t esz = 2) {
  ExpertsWs w;
  const int64_t P = T * k;
  const int64_t rows = P + shared_rows;
  w.max_tiles = max_tiles_impl(T, E, k, shared_rows);
  size_t off = 0;
  w.hist = off; off = align_up(off + sizeof(int32_t) * hist_blocks(T) * E);
  w.counts = off; off = align_up(off + sizeof(int32_t) * E);
  w.starts = off; off = align_up(off + sizeof(int32_t) * E);
  w.perm = off; off = align_up(off + sizeof(int32_t) * P);
  w.inv = off; off = align_up(off + sizeof(int32_t) * P);
  w.tiles = off; off = align_up(off + 4 * sizeof(int32_t) * w.max_tiles);
  w.tile_count = off; off = align_up(off + sizeof(int32_t));
  w.H = off; off = align_up(off + esz * (size_t)rows * I);
  w.Y = off; off = align_up(off + esz * (size_t)rows * h);
  w.end = off;
  return w;
}

struct BlockWs {
  ExpertsWs ex;
  bool fused;  // shared expert inside the grouped GEMMs (Is == I)
  size_t idx, w, gate, Hs, sh, lg, end;
};

// esz: bytes per activation element (2 = bf16, 4 = fp32). The fp32 block also keeps its router
// logits here when the caller does not ask for them (the selection reads them back).
BlockWs block_layout(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int32_t Is, size_t esz = 2) {
  BlockWs b;
  b.fused = Is == I;
  b.ex = experts_layout(T, h, E, k, I, b.fused ? T : 0, esz);
  size_t off = b.ex.end;
  const int64_t P = T * k;
  b.idx = off; off = align_up(off + sizeof(int32_t) * P);
  b.w = off; off = align_up(off + esz * (size_t)P);
  b.gate = off; off = align_up(off + esz * (size_t)T);
  b.Hs = off; off = align_up(off + (b.fused ? 0 : esz * (size_t)T * Is));
  b.sh = off; off = align_up(off + (b.fused ? 0 : esz * (size_t)T * h));
  b.lg = off; off = align_up(off + (esz == 4 ? sizeof(float) * (size_t)T * E : 0));
  b.end = off;
  return b;
}

// fp8 block workspace: the bf16 block's, plus the e4m3 tokens and SwiGLU rows with their scales.
struct Fp8Ws {
  BlockWs b;
  size_t xq, sx, sa, Hq, sH, end;
};

Fp8Ws fp8_layout(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I) {
  Fp8Ws f;
  f.b = block_layout(T, h, E, k, I, I);
  const int64_t rows = T * k + T;
  size_t off = f.b.end;
  f.xq = off; off = align_up(off + (size_t)T * h);
  f.sx = off; off = align_up(off + sizeof(float) * T);
  f.sa = off; off = align_up(off + sizeof(float) * rows);
  f.Hq = off; off = align_up(off + (size_t)rows * I);
  f.sH = off; off = align_up(off + sizeof(float) * rows);
  f.end = off;
  return f;
}

template <typename P>
P* at(void* base, size_t off) {
  return reinterpret_cast<P*>(static_cast<char*>(base) + off);
}

int check_rows(int64_t T, int32_t h, int32_t k) {
  if ((T * k + T) * (int64_t)h >= (int64_t)1 << 31)
    return fail(Q38MOE_EINVAL, "(T*k + T) * h must be < 2^31 (got T=%lld, h=%d)", (long long)T, h);
  return Q38MOE_OK;
}

// Routed experts (+ the shared expert when sh_* weights are given and fused) from routing
// indices/weights in device memory: permute, gate/up, down, combine.
int run_experts(const void* x, const void* idx, bool idx64, const void* topk_w,
                const void* w_gate_up, const void* w_down, const void* sh_gate,
                const void* sh_up, const void* sh_down, const void* shared_out,
                const void* gate, void* out, int64_t T, int32_t h, int32_t E, int32_t k,
                int32_t I, int64_t shared_rows, const int32_t* hist_ready, void* ws,
                const ExpertsWs& L, hipStream_t st, bool f32 = false) {
  const int bm = q38::gemm_block_m();
  int32_t* hist = at<int32_t>(ws, L.hist);
  int32_t* counts = at<int32_t>(ws, L.counts);
  int32_t* starts = at<int32_t>(ws, L.starts);
  int32_t* perm = at<int32_t>(ws, L.perm);
  int32_t* inv = at<int32_t>(ws, L.inv);
  int4* tiles = at<int4>(ws, L.tiles);
  int32_t* tile_count = at<int32_t>(ws, L.tile_count);
  const int64_t P = T * k;
  if (hist_ready == nullptr) {
    Q38_HIP(q38::launch_histogram(idx, idx64, hist, T, E, k, st), "histogram launch");
    hist_ready = hist;
  }
  Q38_HIP(q38::launch_permute(idx, idx64, hist_ready, counts, starts, perm, inv, tiles, tile_count,
                              bm, (int)L.max_tiles, (int)shared_rows, T, E, k, st),
          "permute launch");
  if (f32) {
    // fp32 path: the same permutation and tile table, fp32 GEMMs and combine.
    float* H = at<float>(ws, L.H);
    float* Y = at<float>(ws, L.Y);
    Q38_HIP(q38::launch_gate_up_f32(static_cast<const float*>(x), perm, tiles, tile_count, (int)L.max_tiles, 0,
                                    (int)P, static_cast<const float*>(w_gate_up), static_cast<const float*>(sh_gate),
                                    static_cast<const float*>(sh_up), H, I, h, E, k, st),
            "gate_up fp32 launch");
    Q38_HIP(q38::launch_plain_f32(H, tiles, tile_count, (int)L.max_tiles, 0, static_cast<const float*>(w_down),
                                  static_cast<const float*>(sh_down), Y, h, I, E, st),
            "down fp32 launch");
    const float* shared = shared_out != nullptr ? static_cast<const float*>(shared_out)
                                                : (shared_rows > 0 ? Y + P * h : nullptr);
    Q38_HIP(q38::launch_combine_f32(Y, inv, idx, idx64, static_cast<const float*>(topk_w), shared,
                                    static_cast<const float*>(gate), static_cast<float*>(out), T, h, E, k, st),
            "combine fp32 launch");
    return Q38MOE_OK;
  }
  uint16_t* H = at<uint16_t>(ws, L.H);
  uint16_t* Y = at<uint16_t>(ws, L.Y);
  Q38_HIP(gate_up_bf16(static_cast<const uint16_t*>(x), perm, tiles, tile_count, (int)L.max_tiles, T, k, shared_rows,
                       static_cast<const uint16_t*>(w_gate_up), static_cast<const uint16_t*>(sh_gate),
                       static_cast<const uint16_t*>(sh_up), H, I, h, E, st),
          "gate_up launch");
  Q38_HIP(down_bf16(H, tiles, tile_count, (int)L.max_tiles, T, k, shared_rows, static_cast<const uint16_t*>(w_down),
                    static_cast<const uint16_t*>(sh_down), Y, I, h, E, st),
          "down launch");
  const uint16_t* shared = shared_out != nullptr ? static_cast<const uint16_t*>(shared_out)
                                                 : (shared_rows > 0 ? Y + P * h : nullptr);
  Q38_HIP(q38::launch_combine(Y, inv, idx, idx64, static_cast<const uint16_t*>(topk_w), shared,
                              static_cast<const uint16_t*>(gate), static_cast<uint16_t*>(out), T, h, E, k, st),
          "combine launch");
  return Q38MOE_OK;
}

int check_block_args(const void* x, const void* w_router, const void* w_gate_up, const void* w_down,
                     const void* w_sh_gate, const void* w_sh_up, const void* w_sh_down, const void* w_sh_gate_proj,
                     const void* out, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int32_t Is,
                     int32_t dtype) {
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  Q38_CHECK(check_dim(Is, "Is"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_router, "w_router"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(w_sh_gate, "w_sh_gate"));
  Q38_CHECK(check_ptr(w_sh_up, "w_sh_up"));
  Q38_CHECK(check_ptr(w_sh_down, "w_sh_down"));
  Q38_CHECK(check_ptr(w_sh_gate_proj, "w_sh_gate_proj"));
  Q38_CHECK(check_ptr(out, "out"));
  return Q38MOE_OK;
}

// The whole block (modeling:824-835) on a workspace laid out by block_layout.
int run_block(const void* x, const void* w_router, const void* w_gate_up, const void* w_down, const void* w_sh_gate,
              const void* w_sh_up, const void* w_sh_down, const void* w_sh_gate_proj, const float* logit_bias,
              void* out, void* logits, int32_t* topk_idx, void* topk_w, int64_t T, int32_t h, int32_t E, int32_t k,
              int32_t I, int32_t Is, void* workspace, const BlockWs& L, hipStream_t st, bool f32 = false) {
  int32_t* idx = topk_idx != nullptr ? topk_idx : at<int32_t>(workspace, L.idx);
  int32_t* hist = at<int32_t>(workspace, L.ex.hist);
  if (f32) {
    // fp32 block: router logits and the shared gate logit in one dense fp32 GEMM (modeling:807, 831),
    // selection on them, shared expert (separate when Is != I), routed experts, gated sum.
    const float* xf = static_cast<const float*>(x);
    float* w = topk_w != nullptr ? static_cast<float*>(topk_w) : at<float>(workspace, L.w);
    float* gate = at<float>(workspace, L.gate);
    float* lg = logits != nullptr ? static_cast<float*>(logits) : at<float>(workspace, L.lg);
    const float* sh_out = nullptr;
    if (!L.fused) {
      float* Hs = at<float>(workspace, L.Hs);
      float* sh = at<float>(workspace, L.sh);
      Q38_HIP(q38::launch_gate_up_f32(xf, nullptr, nullptr, nullptr, 0, T, 0, nullptr,
                                      static_cast<const float*>(w_sh_gate), static_cast<const float*>(w_sh_up), Hs, Is,
                                      h, 0, 1, st),
              "shared gate_up fp32 launch");
      Q38_HIP(q38::launch_plain_f32(Hs, nullptr, nullptr, 0, T, nullptr, static_cast<const float*>(w_sh_down), sh, h,
                                    Is, 0, st),
              "shared down fp32 launch");
      sh_out = sh;
    }
    Q38_HIP(q38::launch_logits_f32(xf, static_cast<const float*>(w_router), static_cast<const float*>(w_sh_gate_proj),
                                   lg, gate, T, E, h, st),
            "router and shared gate logits fp32 launch");
    Q38_HIP(q38::launch_route_from_f32_logits(lg, logit_bias, idx, w, hist, T, E, k, st), "route fp32 launch");
    return run_experts(x, idx, false, w, w_gate_up, w_down, L.fused ? w_sh_gate : nullptr,
                       L.fused ? w_sh_up : nullptr, L.fused ? w_sh_down : nullptr, sh_out, gate, out, T, h, E, k, I,
                       L.fused ? T : 0, hist, workspace, L.ex, st, true);
  }
  uint16_t* w = topk_w != nullptr ? static_cast<uint16_t*>(topk_w) : at<uint16_t>(workspace, L.w);
  uint16_t* gate = at<uint16_t>(workspace, L.gate);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* sh_out = nullptr;
  if (!L.fused) {
    // Shared expert (modeling:827) as its own dense GEMMs when its width differs from I.
    uint16_t* Hs = at<uint16_t>(workspace, L.Hs);
    uint16_t* sh = at<uint16_t>(workspace, L.sh);
    Q38_HIP(q38::launch_gate_up(xb, nullptr, nullptr, nullptr, 0, T, 0, nullptr,
                                static_cast<const uint16_t*>(w_sh_gate), static_cast<const uint16_t*>(w_sh_up), Hs,
                                Is, h, E, 1, st),
            "shared gate_up launch");
    Q38_HIP(q38::launch_down(Hs, nullptr, nullptr, 0, T, nullptr, static_cast<const uint16_t*>(w_sh_down), sh, h,
                             Is, E, st),
            "shared down launch");
    sh_out = sh;
  }
  // Router + shared gate logit + histogram (modeling:828, 831).
  Q38_HIP(q38::launch_route(xb, static_cast<const uint16_t*>(w_router), static_cast<const uint16_t*>(w_sh_gate_proj),
                            nullptr, logit_bias, static_cast<uint16_t*>(logits), idx, w, gate, hist, T, h, E, k, st),
          "route launch");
  // Routed experts (+ the shared expert inside the same GEMMs) and the gated sum (modeling:829-833).
  return run_experts(x, idx, false, w, w_gate_up, w_down, L.fused ? w_sh_gate : nullptr,
                     L.fused ? w_sh_up : nullptr, L.fused ? w_sh_down : nullptr, sh_out, gate, out, T, h, E, k, I,
                     L.fused ? T : 0, hist, workspace, L.ex, st);
}

// Static scratch of q38moe_block_forward_noalloc: one copy per GPU, held until the process ends.
// In host code `scratch` only names the symbol; its device address (different on every GPU) comes
// from hipGetSymbolAddress with that GPU current, looked up once per device and kept in
// g_scratch_dev. Nothing in it needs clearing: every buffer the block carves from it is written in
// full before it is read.
constexpr size_t kScratchBytes = Q38MOE_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int scratch_for_current_device(hipStream_t stream, void** ptr) {
  int dev = -1;
  Q38_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(Q38MOE_EINVAL, "device %d out of range", dev);
  if (stream != nullptr) {
    int sdev = -1;
    Q38_HIP(hipStreamGetDevice(stream, &sdev), "hipStreamGetDevice");
    if (sdev != dev)
      return fail(Q38MOE_EINVAL, "stream belongs to device %d but device %d is current; make it current", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    Q38_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (p == nullptr || reinterpret_cast<uintptr_t>(p) % kAlign != 0)
      return fail(Q38MOE_EHIP, "static scratch has no 256-byte aligned device address");
    g_scratch_dev[dev] = p;
  }
  *ptr = g_scratch_dev[dev];
  return Q38MOE_OK;
}

}  // namespace

extern "C" {

int q38moe_abi_version(void) { return Q38MOE_ABI_VERSION; }

const char* q38moe_last_error(void) { return g_err; }

int64_t q38moe_max_tiles(int64_t T, int32_t E, int32_t k, int64_t shared_rows) {
  if (T < 0 || E < 1 || k < 1 || shared_rows < 0) return -1;
  return max_tiles_impl(T, E, k, shared_rows);
}

int32_t q38moe_gemm_block_m(void) { return q38::gemm_block_m(); }

int32_t q38moe_gemm_tiling(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows) {
  return small_tiles(T, h, E, k, I, shared_rows) ? Q38MOE_TILING_SMALL : Q38MOE_TILING_PERSISTENT;
}

int32_t q38moe_gemm_tiling_fp8(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows) {
  return small_tiles_fp8(T, h, E, k, I, shared_rows) ? Q38MOE_TILING_SMALL : Q38MOE_TILING_PERSISTENT;
}

int q38moe_route(const void* x, const void* w_router, const void* w_shared_gate,
                 const float* logit_bias, void* logits, int32_t* topk_idx, void* topk_w,
                 void* shared_gate_logit, int32_t* hist, int64_t T, int32_t h, int32_t E,
                 int32_t k, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_router, "w_router"));
  Q38_CHECK(check_opt_ptr(w_shared_gate, "w_shared_gate"));
  if (topk_idx == nullptr || topk_w == nullptr) return fail(Q38MOE_EINVAL, "topk_idx and topk_w must not be NULL");
  if (shared_gate_logit != nullptr && w_shared_gate == nullptr)
    return fail(Q38MOE_EINVAL, "shared_gate_logit requires w_shared_gate");
  (void)hipGetLastError();
  if (dtype == Q38MOE_FP32) {
    // fp32: logits as a dense fp32 GEMM into the caller's logits buffer, then the selection on them.
    if (logits == nullptr) return fail(Q38MOE_EINVAL, "dtype FP32: logits must not be NULL (the selection reads them)");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Q38_HIP(q38::launch_logits_f32(static_cast<const float*>(x), static_cast<const float*>(w_router),
                                   shared_gate_logit != nullptr ? static_cast<const float*>(w_shared_gate) : nullptr,
                                   static_cast<float*>(logits), static_cast<float*>(shared_gate_logit), T, E, h, st),
            "router logits fp32 launch");
    Q38_HIP(q38::launch_route_from_f32_logits(static_cast<const float*>(logits), logit_bias, topk_idx,
                                              static_cast<float*>(topk_w), hist, T, E, k, st),
            "route fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(q38::launch_route(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w_router),
                            static_cast<const uint16_t*>(w_shared_gate), nullptr, logit_bias,
                            static_cast<uint16_t*>(logits), topk_idx, static_cast<uint16_t*>(topk_w),
                            static_cast<uint16_t*>(shared_gate_logit), hist, T, h, E, k,
                            static_cast<hipStream_t>(stream)),
          "route launch");
  return Q38MOE_OK;
}

int q38moe_route_from_logits(const void* logits, const float* logit_bias, int32_t* topk_idx,
                             void* topk_w, int32_t* hist, int64_t T, int32_t E, int32_t k,
                             int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  if (T == 0) return Q38MOE_OK;
  if (logits == nullptr || topk_idx == nullptr || topk_w == nullptr)
    return fail(Q38MOE_EINVAL, "logits, topk_idx and topk_w must not be NULL");
  (void)hipGetLastError();
  if (dtype == Q38MOE_FP32) {
    Q38_HIP(q38::launch_route_from_f32_logits(static_cast<const float*>(logits), logit_bias, topk_idx,
                                              static_cast<float*>(topk_w), hist, T, E, k,
                                              static_cast<hipStream_t>(stream)),
            "route_from_logits fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(q38::launch_route(nullptr, nullptr, nullptr, static_cast<const uint16_t*>(logits),
                            logit_bias, nullptr, topk_idx, static_cast<uint16_t*>(topk_w), nullptr,
                            hist, T, 64, E, k, static_cast<hipStream_t>(stream)),
          "route_from_logits launch");
  return Q38MOE_OK;
}

int q38moe_histogram(const void* topk_idx, int32_t idx_is_int64, int32_t* hist, int64_t T,
                     int32_t E, int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  if (T == 0) return Q38MOE_OK;
  if (topk_idx == nullptr || hist == nullptr) return fail(Q38MOE_EINVAL, "topk_idx and hist must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_histogram(topk_idx, idx_is_int64 != 0, hist, T, E, k,
                                static_cast<hipStream_t>(stream)),
          "histogram launch");
  return Q38MOE_OK;
}

int q38moe_permute(const void* topk_idx, int32_t idx_is_int64, const int32_t* hist,
                   int32_t* counts, int32_t* starts, int32_t* perm, int32_t* inv, int32_t* tiles,
                   int32_t* tile_count, int64_t shared_rows, int64_t T, int32_t E, int32_t k,
                   void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  if (shared_rows < 0 || shared_rows > (int64_t)1 << 30) return fail(Q38MOE_EINVAL, "bad shared_rows");
  if (counts == nullptr || starts == nullptr) return fail(Q38MOE_EINVAL, "counts and starts must not be NULL");
  if (T > 0 && (topk_idx == nullptr || hist == nullptr || perm == nullptr))
    return fail(Q38MOE_EINVAL, "topk_idx, hist and perm must not be NULL");
  if (tiles != nullptr && !aligned16(tiles)) return fail(Q38MOE_EINVAL, "tiles must be 16-byte aligned");
  (void)hipGetLastError();
  const int64_t mt = tiles != nullptr ? max_tiles_impl(T, E, k, shared_rows) : 0;
  Q38_HIP(q38::launch_permute(topk_idx, idx_is_int64 != 0, hist, counts, starts, perm, inv,
                              reinterpret_cast<int4*>(tiles), tile_count, q38::gemm_block_m(), (int)mt,
                              (int)shared_rows, T, E, k, static_cast<hipStream_t>(stream)),
          "permute launch");
  return Q38MOE_OK;
}

int q38moe_gate_up(const void* x, const void* w_gate_up, const void* w_sh_gate,
                   const void* w_sh_up, const int32_t* perm, const int32_t* tiles,
                   const int32_t* tile_count, int64_t shared_rows, void* H, int64_t T, int32_t h,
                   int32_t E, int32_t k, int32_t I, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr || tile_count == nullptr) return fail(Q38MOE_EINVAL, "perm and tile_count must not be NULL");
  if (shared_rows < 0 || shared_rows > T) return fail(Q38MOE_EINVAL, "shared_rows must be in [0, T]");
  if (shared_rows > 0) {
    Q38_CHECK(check_ptr(w_sh_gate, "w_sh_gate"));
    Q38_CHECK(check_ptr(w_sh_up, "w_sh_up"));
  }
  (void)hipGetLastError();
  if (dtype == Q38MOE_FP32) {
    Q38_HIP(q38::launch_gate_up_f32(static_cast<const float*>(x), perm, reinterpret_cast<const int4*>(tiles),
                                    tile_count, (int)max_tiles_impl(T, E, k, shared_rows), 0, (int)(T * k),
                                    static_cast<const float*>(w_gate_up), static_cast<const float*>(w_sh_gate),
                                    static_cast<const float*>(w_sh_up), static_cast<float*>(H), I, h, E, k,
                                    static_cast<hipStream_t>(stream)),
            "gate_up fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(gate_up_bf16(static_cast<const uint16_t*>(x), perm, reinterpret_cast<const int4*>(tiles), tile_count,
                       (int)max_tiles_impl(T, E, k, shared_rows), T, k, shared_rows,
                       static_cast<const uint16_t*>(w_gate_up), static_cast<const uint16_t*>(w_sh_gate),
                       static_cast<const uint16_t*>(w_sh_up), static_cast<uint16_t*>(H), I, h, E,
                       static_cast<hipStream_t>(stream)),
          "gate_up launch");
  return Q38MOE_OK;
}

int q38moe_down(const void* H, const void* w_down, const void* w_sh_down, const int32_t* tiles,
                const int32_t* tile_count, int64_t shared_rows, void* Y, int64_t T, int32_t h,
                int32_t E, int32_t k, int32_t I, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(Y, "Y"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (tile_count == nullptr) return fail(Q38MOE_EINVAL, "tile_count must not be NULL");
  if (shared_rows < 0 || shared_rows > T) return fail(Q38MOE_EINVAL, "shared_rows must be in [0, T]");
  if (shared_rows > 0) Q38_CHECK(check_ptr(w_sh_down, "w_sh_down"));
  (void)hipGetLastError();
  if (dtype == Q38MOE_FP32) {
    Q38_HIP(q38::launch_plain_f32(static_cast<const float*>(H), reinterpret_cast<const int4*>(tiles), tile_count,
                                  (int)max_tiles_impl(T, E, k, shared_rows), 0, static_cast<const float*>(w_down),
                                  static_cast<const float*>(w_sh_down), static_cast<float*>(Y), h, I, E,
                                  static_cast<hipStream_t>(stream)),
            "down fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(down_bf16(static_cast<const uint16_t*>(H), reinterpret_cast<const int4*>(tiles), tile_count,
                    (int)max_tiles_impl(T, E, k, shared_rows), T, k, shared_rows,
                    static_cast<const uint16_t*>(w_down), static_cast<const uint16_t*>(w_sh_down),
                    static_cast<uint16_t*>(Y), I, h, E, static_cast<hipStream_t>(stream)),
          "down launch");
  return Q38MOE_OK;
}

int q38moe_gather_gemm(const void* x, const int32_t* perm, const void* w, const int32_t* tiles,
                       const int32_t* tile_count, void* C, int64_t T, int32_t K, int32_t N, int32_t E,
                       int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(K, "K"));
  Q38_CHECK(check_dim(N, "N"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, K, k));
  Q38_CHECK(check_rows(T, N, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w, "w"));
  Q38_CHECK(check_ptr(C, "C"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr || tile_count == nullptr) return fail(Q38MOE_EINVAL, "perm and tile_count must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_gather_gemm(static_cast<const uint16_t*>(x), perm, reinterpret_cast<const int4*>(tiles),
                                  tile_count, (int)max_tiles_impl(T, E, k, 0), static_cast<const uint16_t*>(w),
                                  static_cast<uint16_t*>(C), N, K, E, k, static_cast<hipStream_t>(stream)),
          "gather gemm launch");
  return Q38MOE_OK;
}

int q38moe_gate_up_save(const void* x, const void* w_gate_up, const int32_t* perm, const int32_t* tiles,
                        const int32_t* tile_count, void* H, void* GU, int64_t T, int32_t h, int32_t E, int32_t k,
                        int32_t I, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_rows(T, 2 * I, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(GU, "GU"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr || tile_count == nullptr) return fail(Q38MOE_EINVAL, "perm and tile_count must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_gate_up_save(static_cast<const uint16_t*>(x), perm, reinterpret_cast<const int4*>(tiles),
                                   tile_count, (int)max_tiles_impl(T, E, k, 0), (int)(T * k),
                                   static_cast<const uint16_t*>(w_gate_up), static_cast<uint16_t*>(H),
                                   static_cast<uint16_t*>(GU), I, h, E, k, static_cast<hipStream_t>(stream)),
          "gate_up_save launch");
  return Q38MOE_OK;
}

int q38moe_down_kn(const void* A, const void* w_kn, const int32_t* tiles, const int32_t* tile_count, void* Y,
                   int64_t T, int32_t K, int32_t N, int32_t E, int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(K, "K"));
  Q38_CHECK(check_dim(N, "N"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, K, k));
  Q38_CHECK(check_rows(T, N, k));
  Q38_CHECK(check_ptr(A, "A"));
  Q38_CHECK(check_ptr(w_kn, "w_kn"));
  Q38_CHECK(check_ptr(Y, "Y"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (tile_count == nullptr) return fail(Q38MOE_EINVAL, "tile_count must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_down_kn(static_cast<const uint16_t*>(A), reinterpret_cast<const int4*>(tiles), tile_count,
                              (int)max_tiles_impl(T, E, k, 0), static_cast<const uint16_t*>(w_kn),
                              static_cast<uint16_t*>(Y), N, K, E, static_cast<hipStream_t>(stream)),
          "down_kn launch");
  return Q38MOE_OK;
}

int q38moe_pair_dots(const void* dout, const void* Y, const int32_t* inv, const void* topk_idx,
                     int32_t idx_is_int64, const void* topk_w, void* dw, void* d_raw, int64_t T, int32_t h,
                     int32_t E, int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(dout, "dout"));
  Q38_CHECK(check_ptr(Y, "Y"));
  if (inv == nullptr || dw == nullptr || topk_idx == nullptr)
    return fail(Q38MOE_EINVAL, "inv, topk_idx and dw must not be NULL");
  if (d_raw != nullptr && topk_w == nullptr) return fail(Q38MOE_EINVAL, "d_raw needs topk_w");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_pair_dots(static_cast<const uint16_t*>(dout), static_cast<const uint16_t*>(Y), inv, topk_idx,
                                idx_is_int64 != 0, static_cast<const uint16_t*>(topk_w), static_cast<uint16_t*>(dw),
                                static_cast<uint16_t*>(d_raw), T, h, E, k, static_cast<hipStream_t>(stream)),
          "pair dots launch");
  return Q38MOE_OK;
}

int q38moe_gather_rows(const void* src, const int32_t* perm, const void* w, const int32_t* starts,
                       const int32_t* counts, void* dst, int64_t T, int32_t h, int32_t E, int32_t k,
                       void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(src, "src"));
  Q38_CHECK(check_ptr(dst, "dst"));
  if (perm == nullptr || starts == nullptr || counts == nullptr)
    return fail(Q38MOE_EINVAL, "perm, starts and counts must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_gather_rows(static_cast<const uint16_t*>(src), perm, static_cast<const uint16_t*>(w), starts,
                                  counts, static_cast<uint16_t*>(dst), T * k, h, E, k,
                                  static_cast<hipStream_t>(stream)),
          "gather rows launch");
  return Q38MOE_OK;
}

int q38moe_transpose_experts(const void* src, void* dst, int32_t E, int32_t R, int32_t C, void* stream) {
  g_err[0] = 0;
  if (E < 0) return fail(Q38MOE_EINVAL, "E must be >= 0 (got %d)", E);
  Q38_CHECK(check_dim(R, "R"));
  Q38_CHECK(check_dim(C, "C"));
  if (E == 0) return Q38MOE_OK;
  if ((int64_t)E * R * C >= (int64_t)1 << 40) return fail(Q38MOE_EINVAL, "E * R * C is too large");
  Q38_CHECK(check_ptr(src, "src"));
  Q38_CHECK(check_ptr(dst, "dst"));
  const uintptr_t s0 = (uintptr_t)src, d0 = (uintptr_t)dst, n = (uintptr_t)E * R * C * 2;
  if (s0 < d0 + n && d0 < s0 + n) return fail(Q38MOE_EINVAL, "src and dst overlap");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_transpose_experts(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), E, R, C,
                                        static_cast<hipStream_t>(stream)),
          "transpose launch");
  return Q38MOE_OK;
}

int q38moe_expert_wgrad(const void* G, const void* X, const int32_t* perm, const int32_t* starts,
                        const int32_t* counts, void* dW, int64_t T, int32_t M, int32_t N, int32_t E,
                        int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(M, "M"));
  Q38_CHECK(check_dim(N, "N"));
  Q38_CHECK(check_ptr(dW, "dW"));
  if ((int64_t)E * M * N >= (int64_t)1 << 40) return fail(Q38MOE_EINVAL, "E * M * N is too large");
  if (T > 0) {
    Q38_CHECK(check_rows(T, M > N ? M : N, k));
    Q38_CHECK(check_ptr(G, "G"));
    Q38_CHECK(check_ptr(X, "X"));
  }
  if (T > 0 && (starts == nullptr || counts == nullptr))
    return fail(Q38MOE_EINVAL, "starts and counts must not be NULL");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_expert_wgrad(static_cast<const uint16_t*>(G), static_cast<const uint16_t*>(X), perm, starts,
                                   counts, static_cast<uint16_t*>(dW), T * k, E, M, N, k,
                                   static_cast<hipStream_t>(stream)),
          "expert wgrad launch");
  return Q38MOE_OK;
}

int q38moe_swiglu_backward(const void* dH, const void* GU, void* dGU, int64_t rows, int32_t I,
                           void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dim(I, "I"));
  if (rows < 0) return fail(Q38MOE_EINVAL, "rows must be >= 0");
  if (rows == 0) return Q38MOE_OK;
  if (rows * (int64_t)I * 2 >= (int64_t)1 << 31) return fail(Q38MOE_EINVAL, "rows * 2I must be < 2^31");
  Q38_CHECK(check_ptr(dH, "dH"));
  Q38_CHECK(check_ptr(GU, "GU"));
  Q38_CHECK(check_ptr(dGU, "dGU"));
  (void)hipGetLastError();
  Q38_HIP(q38::launch_swiglu_backward(static_cast<const uint16_t*>(dH), static_cast<const uint16_t*>(GU),
                                      static_cast<uint16_t*>(dGU), rows, I, static_cast<hipStream_t>(stream)),
          "swiglu backward launch");
  return Q38MOE_OK;
}

int q38moe_shared_expert(const void* x, const void* w_gate, const void* w_up,
                         const void* w_down, void* Hs, void* out, int64_t T, int32_t h,
                         int32_t Is, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  if (T < 0) return fail(Q38MOE_EINVAL, "T must be >= 0");
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(Is, "Is"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, 0));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate, "w_gate"));
  Q38_CHECK(check_ptr(w_up, "w_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(Hs, "Hs"));
  Q38_CHECK(check_ptr(out, "out"));
  (void)hipGetLastError();
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q38MOE_FP32) {
    Q38_HIP(q38::launch_gate_up_f32(static_cast<const float*>(x), nullptr, nullptr, nullptr, 0, T, 0, nullptr,
                                    static_cast<const float*>(w_gate), static_cast<const float*>(w_up),
                                    static_cast<float*>(Hs), Is, h, 0, 1, st),
            "shared gate_up fp32 launch");
    Q38_HIP(q38::launch_plain_f32(static_cast<const float*>(Hs), nullptr, nullptr, 0, T, nullptr,
                                  static_cast<const float*>(w_down), static_cast<float*>(out), h, Is, 0, st),
            "shared down fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(q38::launch_gate_up(static_cast<const uint16_t*>(x), nullptr, nullptr, nullptr, 0, T, 0, nullptr,
                              static_cast<const uint16_t*>(w_gate), static_cast<const uint16_t*>(w_up),
                              static_cast<uint16_t*>(Hs), Is, h, 0, 1, st),
          "shared gate_up launch");
  Q38_HIP(q38::launch_down(static_cast<const uint16_t*>(Hs), nullptr, nullptr, 0, T, nullptr,
                           static_cast<const uint16_t*>(w_down), static_cast<uint16_t*>(out), h, Is, 0, st),
          "shared down launch");
  return Q38MOE_OK;
}

int q38moe_combine(const void* Y, const int32_t* inv, const void* topk_idx, int32_t idx_is_int64,
                   const void* topk_w, const void* shared_out, const void* shared_gate_logit,
                   void* out, int64_t T, int32_t h, int32_t E, int32_t k, int32_t dtype,
                   void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(Y, "Y"));
  Q38_CHECK(check_ptr(out, "out"));
  Q38_CHECK(check_opt_ptr(shared_out, "shared_out"));
  if (inv == nullptr || topk_w == nullptr) return fail(Q38MOE_EINVAL, "inv and topk_w must not be NULL");
  if (shared_out != nullptr && shared_gate_logit == nullptr)
    return fail(Q38MOE_EINVAL, "shared_out requires shared_gate_logit");
  (void)hipGetLastError();
  if (dtype == Q38MOE_FP32) {
    Q38_HIP(q38::launch_combine_f32(static_cast<const float*>(Y), inv, topk_idx, idx_is_int64 != 0,
                                    static_cast<const float*>(topk_w), static_cast<const float*>(shared_out),
                                    static_cast<const float*>(shared_gate_logit), static_cast<float*>(out), T, h, E,
                                    k, static_cast<hipStream_t>(stream)),
            "combine fp32 launch");
    return Q38MOE_OK;
  }
  Q38_HIP(q38::launch_combine(static_cast<const uint16_t*>(Y), inv, topk_idx, idx_is_int64 != 0,
                              static_cast<const uint16_t*>(topk_w), static_cast<const uint16_t*>(shared_out),
                              static_cast<const uint16_t*>(shared_gate_logit), static_cast<uint16_t*>(out), T, h,
                              E, k, static_cast<hipStream_t>(stream)),
          "combine launch");
  return Q38MOE_OK;
}

int q38moe_experts_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int32_t dtype,
                                   size_t* bytes) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (bytes == nullptr) return fail(Q38MOE_EINVAL, "bytes must not be NULL");
  *bytes = experts_layout(T, h, E, k, I, 0, elem_size(dtype)).end;
  return Q38MOE_OK;
}

int q38moe_experts_forward(const void* x, const void* topk_idx, int32_t idx_is_int64,
                           const void* topk_w, const void* w_gate_up, const void* w_down,
                           void* out, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                           void* workspace, size_t workspace_bytes, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(out, "out"));
  if (topk_idx == nullptr || topk_w == nullptr) return fail(Q38MOE_EINVAL, "topk_idx and topk_w must not be NULL");
  const ExpertsWs L = experts_layout(T, h, E, k, I, 0, elem_size(dtype));
  if (workspace == nullptr || workspace_bytes < L.end)
    return fail(Q38MOE_EWORKSPACE, "workspace needs %zu bytes (got %zu)", L.end, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
    return fail(Q38MOE_EINVAL, "workspace must be 256-byte aligned");
  (void)hipGetLastError();
  return run_experts(x, topk_idx, idx_is_int64 != 0, topk_w, w_gate_up, w_down, nullptr, nullptr, nullptr,
                     nullptr, nullptr, out, T, h, E, k, I, 0, nullptr, workspace, L, static_cast<hipStream_t>(stream),
                     dtype == Q38MOE_FP32);
}

int q38moe_block_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                 int32_t Is, int32_t dtype, size_t* bytes) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  Q38_CHECK(check_dim(Is, "Is"));
  if (bytes == nullptr) return fail(Q38MOE_EINVAL, "bytes must not be NULL");
  *bytes = block_layout(T, h, E, k, I, Is, elem_size(dtype)).end;
  return Q38MOE_OK;
}

int q38moe_block_forward(const void* x, const void* w_router, const void* w_gate_up,
                         const void* w_down, const void* w_sh_gate, const void* w_sh_up,
                         const void* w_sh_down, const void* w_sh_gate_proj,
                         const float* logit_bias, void* out, void* logits, int32_t* topk_idx,
                         void* topk_w, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                         int32_t Is, void* workspace, size_t workspace_bytes, int32_t dtype,
                         void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_block_args(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, out, T,
                             h, E, k, I, Is, dtype));
  if (T == 0) return Q38MOE_OK;
  const BlockWs L = block_layout(T, h, E, k, I, Is, elem_size(dtype));
  if (workspace == nullptr || workspace_bytes < L.end)
    return fail(Q38MOE_EWORKSPACE, "workspace needs %zu bytes (got %zu)", L.end, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
    return fail(Q38MOE_EINVAL, "workspace must be 256-byte aligned");
  (void)hipGetLastError();
  return run_block(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, logit_bias, out,
                   logits, topk_idx, topk_w, T, h, E, k, I, Is, workspace, L, static_cast<hipStream_t>(stream),
                   dtype == Q38MOE_FP32);
}

size_t q38moe_block_noalloc_scratch_bytes(void) { return kScratchBytes; }

int q38moe_block_forward_noalloc(const void* x, const void* w_router, const void* w_gate_up,
                                 const void* w_down, const void* w_sh_gate, const void* w_sh_up,
                                 const void* w_sh_down, const void* w_sh_gate_proj,
                                 const float* logit_bias, void* out, void* logits, int32_t* topk_idx,
                                 void* topk_w, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                 int32_t Is, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_block_args(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, out, T,
                             h, E, k, I, Is, dtype));
  if (T == 0) return Q38MOE_OK;
  const BlockWs L = block_layout(T, h, E, k, I, Is, elem_size(dtype));
  if (L.end > kScratchBytes)
    return fail(Q38MOE_EWORKSPACE,
                "q38moe_block_forward_noalloc: this shape needs %zu bytes of scratch, the static scratch holds %zu "
                "(T=%lld is too large: call q38moe_block_forward with a workspace)",
                L.end, kScratchBytes, (long long)T);
  void* ws = nullptr;
  Q38_CHECK(scratch_for_current_device(static_cast<hipStream_t>(stream), &ws));
  (void)hipGetLastError();
  return run_block(x, w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj, logit_bias, out,
                   logits, topk_idx, topk_w, T, h, E, k, I, Is, ws, L, static_cast<hipStream_t>(stream),
                   dtype == Q38MOE_FP32);
}

// ---- fp8 expert path (R14) --------------------------------------------------------------------

int q38moe_quantize_rows(const void* x, void* q, float* scale, int64_t R, int32_t C, void* stream) {
  g_err[0] = 0;
  if (R < 0) return fail(Q38MOE_EINVAL, "R must be >= 0");
  if (C < 64 || C % 64 != 0 || C > 4096) return fail(Q38MOE_EINVAL, "C must be a multiple of 64 in [64, 4096] (got %d)", C);
  if (R == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(x, "x"));
  if (q == nullptr || scale == nullptr) return fail(Q38MOE_EINVAL, "q and scale must not be NULL");
  if (reinterpret_cast<uintptr_t>(q) % 8 != 0) return fail(Q38MOE_EINVAL, "q must be 8-byte aligned");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_quant_rows(static_cast<const uint16_t*>(x), static_cast<uint8_t*>(q), scale, R, C,
                                 static_cast<hipStream_t>(stream)),
          "quantize_rows launch");
  return Q38MOE_OK;
}

int q38moe_block_fp8_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, size_t* bytes) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (bytes == nullptr) return fail(Q38MOE_EINVAL, "bytes must not be NULL");
  *bytes = fp8_layout(T, h, E, k, I).end;
  return Q38MOE_OK;
}

int q38moe_gate_up_fp8(const void* xq, const float* row_scale, const void* wq_gate_up, const float* s_gate_up,
                       const void* wq_sh_gate, const float* s_sh_gate, const void* wq_sh_up,
                       const float* s_sh_up, const int32_t* perm, const int32_t* tiles,
                       const int32_t* tile_count, int64_t shared_rows, void* H, int64_t T, int32_t h,
                       int32_t E, int32_t k, int32_t I, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(xq, "xq"));
  Q38_CHECK(check_ptr(wq_gate_up, "wq_gate_up"));
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr || tile_count == nullptr || row_scale == nullptr || s_gate_up == nullptr)
    return fail(Q38MOE_EINVAL, "perm, tile_count, row_scale and s_gate_up must not be NULL");
  if (shared_rows < 0 || shared_rows > T) return fail(Q38MOE_EINVAL, "shared_rows must be in [0, T]");
  if (shared_rows > 0) {
    Q38_CHECK(check_ptr(wq_sh_gate, "wq_sh_gate"));
    Q38_CHECK(check_ptr(wq_sh_up, "wq_sh_up"));
    if (s_sh_gate == nullptr || s_sh_up == nullptr) return fail(Q38MOE_EINVAL, "shared-expert scales must not be NULL");
  }
  (void)hipGetLastError();
  Q38_HIP(gate_up_fp8_any(static_cast<const uint8_t*>(xq), row_scale, perm, reinterpret_cast<const int4*>(tiles),
                          tile_count, (int)max_tiles_impl(T, E, k, shared_rows), T, k, shared_rows,
                          static_cast<const uint8_t*>(wq_gate_up), s_gate_up, static_cast<const uint8_t*>(wq_sh_gate),
                          s_sh_gate, static_cast<const uint8_t*>(wq_sh_up), s_sh_up, static_cast<uint16_t*>(H), I, h,
                          E, static_cast<hipStream_t>(stream)),
          "gate_up_fp8 launch");
  return Q38MOE_OK;
}

int q38moe_down_fp8(const void* Hq, const float* row_scale, const void* wq_down, const float* s_down,
                    const void* wq_sh_down, const float* s_sh_down, const int32_t* tiles,
                    const int32_t* tile_count, int64_t shared_rows, void* Y, int64_t T, int32_t h,
                    int32_t E, int32_t k, int32_t I, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(Hq, "Hq"));
  Q38_CHECK(check_ptr(wq_down, "wq_down"));
  Q38_CHECK(check_ptr(Y, "Y"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (tile_count == nullptr || row_scale == nullptr || s_down == nullptr)
    return fail(Q38MOE_EINVAL, "tile_count, row_scale and s_down must not be NULL");
  if (shared_rows < 0 || shared_rows > T) return fail(Q38MOE_EINVAL, "shared_rows must be in [0, T]");
  if (shared_rows > 0) {
    Q38_CHECK(check_ptr(wq_sh_down, "wq_sh_down"));
    if (s_sh_down == nullptr) return fail(Q38MOE_EINVAL, "s_sh_down must not be NULL");
  }
  (void)hipGetLastError();
  Q38_HIP(down_fp8_any(static_cast<const uint8_t*>(Hq), row_scale, reinterpret_cast<const int4*>(tiles), tile_count,
                       (int)max_tiles_impl(T, E, k, shared_rows), T, k, shared_rows,
                       static_cast<const uint8_t*>(wq_down), s_down, static_cast<const uint8_t*>(wq_sh_down), s_sh_down,
                       static_cast<uint16_t*>(Y), I, h, E, static_cast<hipStream_t>(stream)),
          "down_fp8 launch");
  return Q38MOE_OK;
}

int q38moe_block_forward_fp8(const void* x, const void* w_router, const void* wq_gate_up, const float* s_gate_up,
                             const void* wq_down, const float* s_down, const void* wq_sh_gate,
                             const float* s_sh_gate, const void* wq_sh_up, const float* s_sh_up,
                             const void* wq_sh_down, const float* s_sh_down, const void* w_sh_gate_proj,
                             const float* logit_bias, void* out, void* logits, int32_t* topk_idx, void* topk_w,
                             int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, void* workspace,
                             size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (h > 4096 || I > 4096) return fail(Q38MOE_EINVAL, "fp8 path: h and I must be <= 4096");
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_rows(T, h, k));
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_router, "w_router"));
  Q38_CHECK(check_ptr(wq_gate_up, "wq_gate_up"));
  Q38_CHECK(check_ptr(wq_down, "wq_down"));
  Q38_CHECK(check_ptr(wq_sh_gate, "wq_sh_gate"));
  Q38_CHECK(check_ptr(wq_sh_up, "wq_sh_up"));
  Q38_CHECK(check_ptr(wq_sh_down, "wq_sh_down"));
  Q38_CHECK(check_ptr(w_sh_gate_proj, "w_sh_gate_proj"));
  Q38_CHECK(check_ptr(out, "out"));
  if (s_gate_up == nullptr || s_down == nullptr || s_sh_gate == nullptr || s_sh_up == nullptr || s_sh_down == nullptr)
    return fail(Q38MOE_EINVAL, "weight scales must not be NULL");
  const Fp8Ws F = fp8_layout(T, h, E, k, I);
  const BlockWs& L = F.b;
  if (workspace == nullptr || workspace_bytes < F.end)
    return fail(Q38MOE_EWORKSPACE, "workspace needs %zu bytes (got %zu)", F.end, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
    return fail(Q38MOE_EINVAL, "workspace must be 256-byte aligned");
  (void)hipGetLastError();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t P = T * k;
  int32_t* idx = topk_idx != nullptr ? topk_idx : at<int32_t>(workspace, L.idx);
  uint16_t* w = topk_w != nullptr ? static_cast<uint16_t*>(topk_w) : at<uint16_t>(workspace, L.w);
  uint16_t* gate = at<uint16_t>(workspace, L.gate);
  const ExpertsWs& X = L.ex;
  int32_t* hist = at<int32_t>(workspace, X.hist);
  int32_t* inv = at<int32_t>(workspace, X.inv);
  int32_t* perm = at<int32_t>(workspace, X.perm);
  int4* tiles = at<int4>(workspace, X.tiles);
  int32_t* tile_count = at<int32_t>(workspace, X.tile_count);
  uint16_t* H = at<uint16_t>(workspace, X.H);
  uint16_t* Y = at<uint16_t>(workspace, X.Y);
  uint8_t* xq = at<uint8_t>(workspace, F.xq);
  float* sx = at<float>(workspace, F.sx);
  float* sa = at<float>(workspace, F.sa);
  uint8_t* Hq = at<uint8_t>(workspace, F.Hq);
  float* sH = at<float>(workspace, F.sH);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  // Router, shared gate logit and histogram in bf16 (modeling:828, 831), then the tokens in e4m3.
  Q38_HIP(q38::launch_route(xb, static_cast<const uint16_t*>(w_router), static_cast<const uint16_t*>(w_sh_gate_proj),
                            nullptr, logit_bias, static_cast<uint16_t*>(logits), idx, w, gate, hist, T, h, E, k, st),
          "route launch");
  Q38_HIP(q38::launch_quant_rows(xb, xq, sx, T, h, st), "quantize x launch");
  // Permutation; each sorted row takes its token's scale (shared rows P + t: token t).
  Q38_HIP(q38::launch_permute(idx, false, hist, at<int32_t>(workspace, X.counts), at<int32_t>(workspace, X.starts),
                              perm, inv, tiles, tile_count, q38::gemm_block_m(), (int)X.max_tiles, (int)T, T, E, k, st,
                              sx, sa),
          "permute launch");
  Q38_HIP(gate_up_fp8_any(xq, sa, perm, tiles, tile_count, (int)X.max_tiles, T, k, T,
                          static_cast<const uint8_t*>(wq_gate_up), s_gate_up, static_cast<const uint8_t*>(wq_sh_gate),
                          s_sh_gate, static_cast<const uint8_t*>(wq_sh_up), s_sh_up, H, I, h, E, st),
          "gate_up_fp8 launch");
  // SwiGLU rows to e4m3, one scale per row (routed pairs in sorted order, then the shared rows).
  Q38_HIP(q38::launch_quant_rows(H, Hq, sH, P + T, I, st), "quantize H launch");
  Q38_HIP(down_fp8_any(Hq, sH, tiles, tile_count, (int)X.max_tiles, T, k, T, static_cast<const uint8_t*>(wq_down),
                       s_down, static_cast<const uint8_t*>(wq_sh_down), s_sh_down, Y, I, h, E, st),
          "down_fp8 launch");
  Q38_HIP(q38::launch_combine(Y, inv, idx, false, w, Y + P * h, gate, static_cast<uint16_t*>(out), T, h, E, k, st),
          "combine launch");
  return Q38MOE_OK;
}

}  // extern "C"
