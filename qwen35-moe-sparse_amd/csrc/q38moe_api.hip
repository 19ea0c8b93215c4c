// C ABI of libq38moe.so: argument validation, workspace carving and kernel sequencing.
// Declarations and the reference function each entry point replaces: include/q38moe.h.
#include <cstdarg>
#include <cstdio>
#include <cstring>

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
  if (dtype != Q38MOE_BF16) return fail(Q38MOE_EINVAL, "unsupported dtype %d (only Q38MOE_BF16)", dtype);
  return Q38MOE_OK;
}

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

int64_t max_tiles_impl(int64_t T, int32_t E, int32_t k, int32_t bm) {
  return (T * k + bm - 1) / bm + E;
}

// Workspace of the routed-experts pipeline.
struct ExpertsWs {
  size_t hist, counts, starts, perm, tiles, H, y, end;
};

ExpertsWs experts_layout(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I) {
  ExpertsWs w;
  const int64_t P = T * k;
  size_t off = 0;
  w.hist = off; off = align_up(off + sizeof(int32_t) * hist_blocks(T) * E);
  w.counts = off; off = align_up(off + sizeof(int32_t) * E);
  w.starts = off; off = align_up(off + sizeof(int32_t) * E);
  w.perm = off; off = align_up(off + sizeof(int32_t) * P);
  w.tiles = off; off = align_up(off + 4 * sizeof(int32_t) * max_tiles_impl(T, E, k, q38::gemm_block_m()));
  w.H = off; off = align_up(off + 2 * (size_t)P * I);
  w.y = off; off = align_up(off + 2 * (size_t)P * h);
  w.end = off;
  return w;
}

struct BlockWs {
  ExpertsWs ex;
  size_t idx, w, gate, Hs, sh, end;
};

BlockWs block_layout(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int32_t Is) {
  BlockWs b;
  b.ex = experts_layout(T, h, E, k, I);
  size_t off = b.ex.end;
  const int64_t P = T * k;
  b.idx = off; off = align_up(off + sizeof(int32_t) * P);
  b.w = off; off = align_up(off + 2 * (size_t)P);
  b.gate = off; off = align_up(off + 2 * (size_t)T);
  b.Hs = off; off = align_up(off + 2 * (size_t)T * Is);
  b.sh = off; off = align_up(off + 2 * (size_t)T * h);
  b.end = off;
  return b;
}

template <typename P>
P* at(void* base, size_t off) {
  return reinterpret_cast<P*>(static_cast<char*>(base) + off);
}

// Routed experts from routing indices/weights already in device memory.
int run_experts(const void* x, const void* idx, bool idx64, const uint16_t* topk_w,
                const void* w_gate_up, const void* w_down, const uint16_t* shared,
                const uint16_t* gate, void* out, int64_t T, int32_t h, int32_t E, int32_t k,
                int32_t I, const int32_t* hist_ready, void* ws, const ExpertsWs& L,
                hipStream_t st) {
  const int bm = q38::gemm_block_m();
  const int64_t mt = max_tiles_impl(T, E, k, bm);
  int32_t* hist = at<int32_t>(ws, L.hist);
  int32_t* counts = at<int32_t>(ws, L.counts);
  int32_t* starts = at<int32_t>(ws, L.starts);
  int32_t* perm = at<int32_t>(ws, L.perm);
  int4* tiles = at<int4>(ws, L.tiles);
  uint16_t* H = at<uint16_t>(ws, L.H);
  uint16_t* y = at<uint16_t>(ws, L.y);
  if (hist_ready == nullptr) {
    Q38_HIP(q38::launch_histogram(idx, idx64, hist, T, E, k, st), "histogram launch");
    hist_ready = hist;
  }
  Q38_HIP(q38::launch_permute(idx, idx64, hist_ready, counts, starts, perm, tiles, bm, (int)mt, T,
                              E, k, st),
          "permute launch");
  const uint16_t* wgu = static_cast<const uint16_t*>(w_gate_up);
  Q38_HIP(q38::launch_gate_up(static_cast<const uint16_t*>(x), perm, tiles, (int)mt, wgu,
                              wgu + (int64_t)I * h, (int64_t)2 * I * h, H, T * k, I, h, k, st),
          "gate_up launch");
  Q38_HIP(q38::launch_down(H, perm, tiles, (int)mt, static_cast<const uint16_t*>(w_down),
                           (int64_t)h * I, topk_w, y, T * k, h, I, st),
          "down launch");
  Q38_HIP(q38::launch_combine(y, idx, idx64, shared, gate, static_cast<uint16_t*>(out), T, h, E,
                              k, st),
          "combine launch");
  return Q38MOE_OK;
}

}  // namespace

extern "C" {

int q38moe_abi_version(void) { return Q38MOE_ABI_VERSION; }

const char* q38moe_last_error(void) { return g_err; }

int64_t q38moe_max_tiles(int64_t T, int32_t E, int32_t k, int32_t block_m) {
  if (T < 0 || E < 1 || k < 1 || block_m < 1) return -1;
  return max_tiles_impl(T, E, k, block_m);
}

int32_t q38moe_gemm_block_m(void) { return q38::gemm_block_m(); }

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
                   int32_t* counts, int32_t* starts, int32_t* perm, int32_t* tiles,
                   int32_t block_m, int64_t T, int32_t E, int32_t k, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  if (counts == nullptr || starts == nullptr)
    return fail(Q38MOE_EINVAL, "counts and starts must not be NULL");
  if (T > 0 && (topk_idx == nullptr || hist == nullptr || perm == nullptr))
    return fail(Q38MOE_EINVAL, "topk_idx, hist and perm must not be NULL");
  if (tiles != nullptr && (block_m < 1 || block_m > 4096))
    return fail(Q38MOE_EINVAL, "block_m must be in [1, 4096] (got %d)", block_m);
  if (tiles != nullptr && !aligned16(tiles)) return fail(Q38MOE_EINVAL, "tiles must be 16-byte aligned");
  (void)hipGetLastError();
  const int64_t mt = tiles != nullptr ? max_tiles_impl(T, E, k, block_m) : 0;
  Q38_HIP(q38::launch_permute(topk_idx, idx_is_int64 != 0, hist, counts, starts, perm,
                              reinterpret_cast<int4*>(tiles), tiles != nullptr ? block_m : 1,
                              (int)mt, T, E, k, static_cast<hipStream_t>(stream)),
          "permute launch");
  return Q38MOE_OK;
}

int q38moe_gate_up(const void* x, const void* w_gate_up, const int32_t* perm,
                   const int32_t* tiles, void* H, int64_t T, int32_t h, int32_t E, int32_t k,
                   int32_t I, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr) return fail(Q38MOE_EINVAL, "perm must not be NULL");
  (void)hipGetLastError();
  const int64_t mt = max_tiles_impl(T, E, k, q38::gemm_block_m());
  const uint16_t* w = static_cast<const uint16_t*>(w_gate_up);
  Q38_HIP(q38::launch_gate_up(static_cast<const uint16_t*>(x), perm,
                              reinterpret_cast<const int4*>(tiles), (int)mt, w, w + (int64_t)I * h,
                              (int64_t)2 * I * h, static_cast<uint16_t*>(H), T * k, I, h, k,
                              static_cast<hipStream_t>(stream)),
          "gate_up launch");
  return Q38MOE_OK;
}

int q38moe_down(const void* H, const void* w_down, const int32_t* perm, const int32_t* tiles,
                const void* topk_w, void* y, int64_t T, int32_t h, int32_t E, int32_t k,
                int32_t I, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(H, "H"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(y, "y"));
  Q38_CHECK(check_ptr(tiles, "tiles"));
  if (perm == nullptr || topk_w == nullptr) return fail(Q38MOE_EINVAL, "perm and topk_w must not be NULL");
  (void)hipGetLastError();
  const int64_t mt = max_tiles_impl(T, E, k, q38::gemm_block_m());
  Q38_HIP(q38::launch_down(static_cast<const uint16_t*>(H), perm,
                           reinterpret_cast<const int4*>(tiles), (int)mt,
                           static_cast<const uint16_t*>(w_down), (int64_t)h * I,
                           static_cast<const uint16_t*>(topk_w), static_cast<uint16_t*>(y), T * k,
                           h, I, static_cast<hipStream_t>(stream)),
          "down launch");
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
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate, "w_gate"));
  Q38_CHECK(check_ptr(w_up, "w_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(Hs, "Hs"));
  Q38_CHECK(check_ptr(out, "out"));
  (void)hipGetLastError();
  hipStream_t st = static_cast<hipStream_t>(stream);
  Q38_HIP(q38::launch_gate_up(static_cast<const uint16_t*>(x), nullptr, nullptr, 0,
                              static_cast<const uint16_t*>(w_gate), static_cast<const uint16_t*>(w_up),
                              0, static_cast<uint16_t*>(Hs), T, Is, h, 1, st),
          "shared gate_up launch");
  Q38_HIP(q38::launch_down(static_cast<const uint16_t*>(Hs), nullptr, nullptr, 0,
                           static_cast<const uint16_t*>(w_down), 0, nullptr,
                           static_cast<uint16_t*>(out), T, h, Is, st),
          "shared down launch");
  return Q38MOE_OK;
}

int q38moe_combine(const void* y, const void* topk_idx, int32_t idx_is_int64,
                   const void* shared_out, const void* shared_gate_logit, void* out, int64_t T,
                   int32_t h, int32_t E, int32_t k, int32_t dtype, void* stream) {
  g_err[0] = 0;
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(y, "y"));
  Q38_CHECK(check_ptr(out, "out"));
  Q38_CHECK(check_opt_ptr(shared_out, "shared_out"));
  if (shared_out != nullptr && shared_gate_logit == nullptr)
    return fail(Q38MOE_EINVAL, "shared_out requires shared_gate_logit");
  (void)hipGetLastError();
  Q38_HIP(q38::launch_combine(static_cast<const uint16_t*>(y), topk_idx, idx_is_int64 != 0,
                              static_cast<const uint16_t*>(shared_out),
                              static_cast<const uint16_t*>(shared_gate_logit),
                              static_cast<uint16_t*>(out), T, h, E, k,
                              static_cast<hipStream_t>(stream)),
          "combine launch");
  return Q38MOE_OK;
}

int q38moe_experts_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                   size_t* bytes) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  if (bytes == nullptr) return fail(Q38MOE_EINVAL, "bytes must not be NULL");
  *bytes = experts_layout(T, h, E, k, I).end;
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
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(out, "out"));
  if (topk_idx == nullptr || topk_w == nullptr) return fail(Q38MOE_EINVAL, "topk_idx and topk_w must not be NULL");
  const ExpertsWs L = experts_layout(T, h, E, k, I);
  if (workspace == nullptr || workspace_bytes < L.end)
    return fail(Q38MOE_EWORKSPACE, "workspace needs %zu bytes (got %zu)", L.end, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
    return fail(Q38MOE_EINVAL, "workspace must be 256-byte aligned");
  (void)hipGetLastError();
  return run_experts(x, topk_idx, idx_is_int64 != 0, static_cast<const uint16_t*>(topk_w),
                     w_gate_up, w_down, nullptr, nullptr, out, T, h, E, k, I, nullptr, workspace, L,
                     static_cast<hipStream_t>(stream));
}

int q38moe_block_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                 int32_t Is, size_t* bytes) {
  g_err[0] = 0;
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  Q38_CHECK(check_dim(Is, "Is"));
  if (bytes == nullptr) return fail(Q38MOE_EINVAL, "bytes must not be NULL");
  *bytes = block_layout(T, h, E, k, I, Is).end;
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
  Q38_CHECK(check_dtype(dtype));
  Q38_CHECK(check_routing(T, E, k));
  Q38_CHECK(check_dim(h, "h"));
  Q38_CHECK(check_dim(I, "I"));
  Q38_CHECK(check_dim(Is, "Is"));
  if (T == 0) return Q38MOE_OK;
  Q38_CHECK(check_ptr(x, "x"));
  Q38_CHECK(check_ptr(w_router, "w_router"));
  Q38_CHECK(check_ptr(w_gate_up, "w_gate_up"));
  Q38_CHECK(check_ptr(w_down, "w_down"));
  Q38_CHECK(check_ptr(w_sh_gate, "w_sh_gate"));
  Q38_CHECK(check_ptr(w_sh_up, "w_sh_up"));
  Q38_CHECK(check_ptr(w_sh_down, "w_sh_down"));
  Q38_CHECK(check_ptr(w_sh_gate_proj, "w_sh_gate_proj"));
  Q38_CHECK(check_ptr(out, "out"));
  const BlockWs L = block_layout(T, h, E, k, I, Is);
  if (workspace == nullptr || workspace_bytes < L.end)
    return fail(Q38MOE_EWORKSPACE, "workspace needs %zu bytes (got %zu)", L.end, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
    return fail(Q38MOE_EINVAL, "workspace must be 256-byte aligned");
  (void)hipGetLastError();
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* idx = topk_idx != nullptr ? topk_idx : at<int32_t>(workspace, L.idx);
  uint16_t* w = topk_w != nullptr ? static_cast<uint16_t*>(topk_w) : at<uint16_t>(workspace, L.w);
  uint16_t* gate = at<uint16_t>(workspace, L.gate);
  uint16_t* Hs = at<uint16_t>(workspace, L.Hs);
  uint16_t* sh = at<uint16_t>(workspace, L.sh);
  int32_t* hist = at<int32_t>(workspace, L.ex.hist);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  // Shared expert (modeling:827).
  Q38_HIP(q38::launch_gate_up(xb, nullptr, nullptr, 0, static_cast<const uint16_t*>(w_sh_gate),
                              static_cast<const uint16_t*>(w_sh_up), 0, Hs, T, Is, h, 1, st),
          "shared gate_up launch");
  Q38_HIP(q38::launch_down(Hs, nullptr, nullptr, 0, static_cast<const uint16_t*>(w_sh_down), 0,
                           nullptr, sh, T, h, Is, st),
          "shared down launch");
  // Router + shared gate logit + histogram (modeling:828, 831).
  Q38_HIP(q38::launch_route(xb, static_cast<const uint16_t*>(w_router),
                            static_cast<const uint16_t*>(w_sh_gate_proj), nullptr, logit_bias,
                            static_cast<uint16_t*>(logits), idx, w, gate, hist, T, h, E, k, st),
          "route launch");
  // Routed experts and the gated sum (modeling:829, 831-833).
  return run_experts(x, idx, false, w, w_gate_up, w_down, sh, gate, out, T, h, E, k, I, hist,
                     workspace, L.ex, st);
}

}  // extern "C"
