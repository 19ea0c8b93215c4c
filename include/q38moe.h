/*
 * q38moe.h — C ABI of the MI355X (gfx950) Q38 MoE feed-forward prefill library (libq38moe.so).
 *
 * The reference implements this path in Python/Triton; there is no C interface to mirror, so each
 * entry point below names the reference function whose semantics it replaces (paths relative to
 * the reference repository root; "modeling" = q38/models/qwen3_8_moe/modeling_qwen3_8_moe.py).
 *
 * Conventions shared by every entry point
 *  - All tensor arguments are device pointers to caller-allocated, contiguous, row-major memory.
 *    The library never allocates or frees device memory; scratch space is a caller-provided
 *    workspace whose size comes from the matching *_workspace_bytes query (except for
 *    q38moe_block_forward_noalloc, which uses a static per-GPU array instead).
 *  - bf16 tensors are passed as raw 16-bit storage (torch.bfloat16 bit patterns).
 *  - Expert/token indices produced by the library are int32. q38moe_experts_forward also accepts
 *    the int64 indices torch.topk returns (idx_is_int64 = 1).
 *  - `stream` is a hipStream_t (NULL = the legacy default stream). All work is enqueued
 *    asynchronously on it; no entry point synchronises the host or the device.
 *  - Return value: 0 on success, negative on error (Q38MOE_E*); q38moe_last_error() then returns a
 *    thread-local, human-readable message. A launch failure reports the HIP error string.
 *  - Shapes: T tokens (T*k < 2^31), hidden h, E experts, top-k k, routed intermediate I, shared
 *    intermediate Is. Supported: 1 <= E <= 64, 1 <= k <= min(8, E), h % 64 == 0,
 *    I % 64 == 0, Is % 64 == 0; every pointer 16-byte aligned.
 *  - dtype: Q38MOE_BF16 (bf16 tensors, the reference's bf16 rounding sequence), or Q38MOE_FP32
 *    for the forward entry points that take a dtype (route, route_from_logits, gate_up, down,
 *    shared_expert, combine, experts_forward, block_forward[_noalloc]): fp32 tensors, fp32
 *    products and sums with no intermediate roundings, as the reference computes fp32 models
 *    (q38/inference.py:54-57, 172: Triton dots with input_precision="ieee"; the eager module in
 *    the parameters' dtype). Every float tensor of a call has the call's dtype (routing weights,
 *    logits and the shared gate logit included); indices stay int32/int64. The fp8 and backward
 *    entry points are bf16 only.
 *  - Apart from the static scratch of q38moe_block_forward_noalloc, the library keeps no mutable
 *    global state, so calls on different streams may overlap as long as they use different
 *    workspaces and outputs.
 */
#ifndef Q38MOE_H
#define Q38MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q38MOE_ABI_VERSION 13

#define Q38MOE_OK 0
#define Q38MOE_EINVAL (-1)   /* bad shape, null pointer, misalignment, unsupported dtype */
#define Q38MOE_EWORKSPACE (-2) /* workspace missing or too small */
#define Q38MOE_EHIP (-3)     /* a HIP runtime call or kernel launch failed */

#define Q38MOE_BF16 1
#define Q38MOE_FP32 2

/* Library ABI version (Q38MOE_ABI_VERSION). */
int q38moe_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* q38moe_last_error(void);

/*
 * Router, R1-R2: replaces Qwen3_8MoeTopKRouter.forward (modeling:805-813).
 *   logits[t,e] = bf16(sum_c x[t,c] * w_router[e,c])                         (F.linear, :807)
 *   probs = softmax(float(logits) (+ logit_bias), fp32)                       (:808)
 *     -- computed bit for bit as torch's CPU softmax (AVX512 kernel) computes it: SLEEF expf_u10
 *        of x - max, the 16-lane vector reduction order of the sum, multiply by 1/sum.
 *   (v, topk_idx) = torch CPU topk(probs, k, largest, sorted)                 (:809)
 *     -- selection on those probabilities with the tie order of ATen/native/TopKImpl.h
 *        (std::nth_element + std::sort with a value-only comparator, NaN first;
 *        std::partial_sort when k*64 <= E), so distinct logits whose probabilities round to
 *        one fp32 value tie exactly as on the CPU.
 *   topk_w = bf16(v / sum(v))                                                 (:810-811)
 *     -- sum(v) in torch's CPU row-sum order (4-way interleaved for k = 5..7, else left to
 *        right), then IEEE division: weights bit-identical to the CPU's.
 * Optional extras:
 *   w_shared_gate [h] (NULL to skip): shared_gate_logit[t] = bf16(x[t] . w_shared_gate), the
 *     shared_expert_gate projection of modeling:831, computed from the same pass over x.
 *   logit_bias [E] fp32 (NULL = reference behaviour): added to the logits before the softmax
 *     (the routing-skew workload; no reference counterpart).
 *   logits [T,E] bf16 (NULL to skip): the router_logits element of the returned tuple.
 *   hist [ceil(T/64), E] int32 (NULL to skip): per-64-token-block expert counts, the input of
 *     q38moe_permute.
 * Outputs: topk_idx [T,k] int32, topk_w [T,k] bf16.
 * Q38MOE_FP32: x, w_router, w_shared_gate fp32; logits = x . w_router^T in fp32 (no rounding) and
 *   must not be NULL (the selection reads it back); topk_w and shared_gate_logit fp32 (the
 *   probabilities, selection and renormalisation as above, no bf16 rounding of the weights).
 */
int q38moe_route(const void* x, const void* w_router, const void* w_shared_gate,
                 const float* logit_bias, void* logits, int32_t* topk_idx, void* topk_w,
                 void* shared_gate_logit, int32_t* hist, int64_t T, int32_t h, int32_t E,
                 int32_t k, int32_t dtype, void* stream);

/*
 * Router selection only (R2) from given logits [T,E] (bf16, or fp32 with Q38MOE_FP32):
 * modeling:808-812 with the logits of :807 supplied by the caller. Same outputs and tie semantics
 * as q38moe_route (topk_w in the logits' dtype).
 */
int q38moe_route_from_logits(const void* logits, const float* logit_bias, int32_t* topk_idx,
                             void* topk_w, int32_t* hist, int64_t T, int32_t E, int32_t k,
                             int32_t dtype, void* stream);

/*
 * Per-64-token-block expert histogram of given routing indices (int32, or int64 when
 * idx_is_int64): hist [ceil(T/64), E]. Indices outside [0,E) are not counted (the sentinel rows
 * transformers' grouped_mm drops, integrations/moe.py:405-420).
 */
int q38moe_histogram(const void* topk_idx, int32_t idx_is_int64, int32_t* hist, int64_t T,
                     int32_t E, int32_t k, void* stream);

/*
 * Permutation, R3-R4: replaces the stable sort + searchsorted of inference.py:163-171 and the
 * block mapping of inference.py:39-50 / 174-183.
 *   counts[e] = #{p : ids[p] == e}; starts = exclusive prefix sum of counts;
 *   perm[starts[e] + r] = the r-th pair p (ascending p = t*k + j) routed to expert e
 *   (identical to torch.sort(ids, stable=True).indices); inv[perm[r]] = r (NULL to skip).
 *   tiles[i] = {group, first row, valid rows, 0}: the row tiles of the grouped GEMMs, each expert
 *   padded to a multiple of q38moe_gemm_block_m() rows (never to a global capacity), experts
 *   ascending; then, when shared_rows > 0, the shared-expert rows [T*k, T*k + shared_rows) as
 *   group E; then unused entries {-1, 0, 0, 0}. *tile_count = number of used entries.
 *   tiles must hold q38moe_max_tiles(T, E, k, shared_rows) entries of int32[4].
 * hist comes from q38moe_route or q38moe_histogram of the same indices.
 */
int q38moe_permute(const void* topk_idx, int32_t idx_is_int64, const int32_t* hist,
                   int32_t* counts, int32_t* starts, int32_t* perm, int32_t* inv, int32_t* tiles,
                   int32_t* tile_count, int64_t shared_rows, int64_t T, int32_t E, int32_t k,
                   void* stream);

/* Entries of the tile table: ceil(T*k / BM) + E + ceil(shared_rows / BM) (cf. the grid bound of
 * inference.py:179), BM = q38moe_gemm_block_m(). */
int64_t q38moe_max_tiles(int64_t T, int32_t E, int32_t k, int64_t shared_rows);

/* Rows per grouped-GEMM tile of this build. */
int32_t q38moe_gemm_block_m(void);

/* Which grouped-GEMM kernels the bf16 gate/up and down entry points (and the forward entry points
 * built on them) run for a shape (T tokens, hidden h, E experts, top-k k, intermediate I,
 * shared_rows fused shared-expert rows): Q38MOE_TILING_PERSISTENT (a persistent grid, one
 * 256-row x 256-column tile per CU at a time) or Q38MOE_TILING_SMALL (16 weight rows x up to 64
 * rows per workgroup with K split over its waves, for few rows per expert). Both compute the same
 * roundings. Rule: small tiles when h and I are in {128, 256, 512, 1024, 2048} and
 * T*k + shared_rows <= R * (E + (shared_rows > 0)), i.e. at most R rows per group on average, with
 * R = 32 * cbrt(2^18 / (h * I)) clamped to [8, 64] (32 at h = 1024, I = 256; 20.2 at h = 2048,
 * I = 512: the measured crossovers at those shapes, the small tiles' cost per row growing with K);
 * the environment variable
 * Q38MOE_GEMM_TILING=small|persistent, read once, overrides the row condition. The reference picks
 * its Triton tiles per shape by timing candidates on the first call (inference.py:133-155, 181-183);
 * this is the build's fixed, shape-keyed counterpart, and the query lets callers and tests see
 * which kernels a shape runs. */
#define Q38MOE_TILING_PERSISTENT 1
#define Q38MOE_TILING_SMALL 2
int32_t q38moe_gemm_tiling(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows);

/* The same for the e4m3 entry points (q38moe_gate_up_fp8, q38moe_down_fp8, q38moe_block_forward_fp8):
 * small tiles (e4m3 16x16x128 MFMA, K split over the workgroup's waves, the same decomposition as
 * the bf16 small tiles) when h and I are in {512, 1024, 2048} and T*k + shared_rows <= F * (E +
 * (shared_rows > 0)), F = 1.25 R (R as above: 25.2 at h = 2048, I = 512, the measured crossover
 * with the persistent fp8 kernel); Q38MOE_GEMM_TILING overrides it as for bf16. The fp32 entry points have
 * one tiling (the persistent fp32 kernels) at every T. No counterpart in the reference (it has no
 * fp8 path). */
int32_t q38moe_gemm_tiling_fp8(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int64_t shared_rows);

/*
 * Grouped gate/up GEMM with fused SwiGLU, R5-R6 (+R9 first half): replaces _gate_up_kernel
 * (inference.py:60-96). Row r of a routed tile (expert e, token = perm[r] / k):
 *   g = bf16(x[token] . w_gate_up[e, n, :]), u = bf16(x[token] . w_gate_up[e, I+n, :]),
 *   H[r, n] = bf16(bf16(silu(g)) * u).
 * Rows r >= T*k of shared tiles (group E) compute the same with token r - T*k and the shared
 * expert's gate_proj / up_proj weights (w_sh_gate, w_sh_up [I,h]; needed iff shared_rows > 0,
 * which also requires Is == I).
 * w_gate_up [E, 2I, h] bf16 (experts.gate_up_proj). H [T*k + shared_rows, I] bf16.
 * Q38MOE_FP32: every tensor fp32 and H[r, n] = silu(g) * u in fp32 with no rounding.
 */
int q38moe_gate_up(const void* x, const void* w_gate_up, const void* w_sh_gate,
                   const void* w_sh_up, const int32_t* perm, const int32_t* tiles,
                   const int32_t* tile_count, int64_t shared_rows, void* H, int64_t T, int32_t h,
                   int32_t E, int32_t k, int32_t I, int32_t dtype, void* stream);

/*
 * Grouped down GEMM, R7 without its routing-weight factor (applied by q38moe_combine with the
 * same rounding): replaces _down_kernel (inference.py:99-130).
 *   Y[r, c] = bf16(H[r] . w_down[e, c, :]) for routed rows (expert e of the row's tile), and with
 *   w_sh_down [h, I] (shared_expert.down_proj) for shared rows. Y [T*k + shared_rows, h] bf16,
 *   expert-sorted row order. Q38MOE_FP32: fp32 tensors, Y unrounded.
 */
int q38moe_down(const void* H, const void* w_down, const void* w_sh_down, const int32_t* tiles,
                const int32_t* tile_count, int64_t shared_rows, void* Y, int64_t T, int32_t h,
                int32_t E, int32_t k, int32_t I, int32_t dtype, void* stream);

/*
 * Shared expert alone, R9 (Qwen3_8MoeMLP.forward, modeling:751-753):
 *   out[t] = bf16(bf16(bf16(silu(bf16(x.Wg^T))) * bf16(x.Wu^T)) . Wd^T).
 * w_gate [Is,h], w_up [Is,h], w_down [h,Is] bf16; Hs workspace [T,Is] bf16; out [T,h] bf16.
 * Q38MOE_FP32: fp32 tensors, no roundings.
 */
int q38moe_shared_expert(const void* x, const void* w_gate, const void* w_up,
                         const void* w_down, void* Hs, void* out, int64_t T, int32_t h,
                         int32_t Is, int32_t dtype, void* stream);

/*
 * Combine, R7 weight + R8 (+ the block tail of modeling:831-833), for pairs p = t*k + j:
 *   y_p = bf16(Y[inv[p]] * topk_w[p])                                          (inference.py:128-130)
 *   routed[t] = bf16(sum_j fp32(y_p))                                          (inference.py:199)
 *   shared_out == NULL: out = routed;
 *   otherwise:          out = bf16(routed + bf16(bf16(sigmoid(gate_logit[t])) * shared_out[t])).
 * topk_idx (NULL = all pairs valid; int32 or int64 per idx_is_int64): pairs whose index lies
 * outside [0,E) contribute nothing. shared_out may point into Y (rows T*k..) when the shared
 * expert ran inside the grouped GEMMs.
 * Q38MOE_FP32: Y, topk_w, shared_out, shared_gate_logit and out fp32;
 *   out = sum_j Y[inv[p]] * w[p] (+ sigmoid(gate_logit[t]) * shared_out[t]) with no roundings.
 */
int q38moe_combine(const void* Y, const int32_t* inv, const void* topk_idx, int32_t idx_is_int64,
                   const void* topk_w, const void* shared_out, const void* shared_gate_logit,
                   void* out, int64_t T, int32_t h, int32_t E, int32_t k, int32_t dtype,
                   void* stream);

/*
 * Routed experts, R3-R8: the ExpertsInterface contract
 *   fn(self, hidden_states[T,h], top_k_index[T,k], top_k_weights[T,k]) -> [T,h]
 * (transformers integrations/moe.py:567-570; implementations inference.py:158-199 and
 * modeling:769-793). Runs histogram, permute, gate/up, down and combine. Requires
 * T*h < 2^31. With Q38MOE_FP32 x, topk_w, the weights and out are fp32 (the workspace query takes
 * the same dtype: the intermediates are twice as large).
 */
int q38moe_experts_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I, int32_t dtype,
                                   size_t* bytes);
int q38moe_experts_forward(const void* x, const void* topk_idx, int32_t idx_is_int64,
                           const void* topk_w, const void* w_gate_up, const void* w_down,
                           void* out, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                           void* workspace, size_t workspace_bytes, int32_t dtype, void* stream);

/*
 * Whole MoE block, R0: Qwen3_8MoeSparseMoeBlock.forward (modeling:824-835) on hidden_states
 * viewed as [T,h]: shared expert, router, routed experts, sigmoid shared gate, sum.
 *   w_router [E,h]; w_gate_up [E,2I,h]; w_down [E,h,I]; w_sh_gate/w_sh_up [Is,h];
 *   w_sh_down [h,Is]; w_sh_gate_proj [1,h] (shared_expert_gate.weight); all bf16.
 *   logit_bias [E] fp32 or NULL. out [T,h] bf16.
 *   Optional router outputs (NULL to skip): logits [T,E] bf16, topk_idx [T,k] int32,
 *   topk_w [T,k] bf16.
 * With Is == I the shared expert runs inside the routed grouped GEMM launches.
 * Q38MOE_FP32: every float tensor fp32 (logits and topk_w too); the router logits and the shared
 *   gate logit are fp32 GEMMs, and nothing is rounded below fp32 (configuration 1 and fp32 models).
 */
int q38moe_block_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                 int32_t Is, int32_t dtype, size_t* bytes);
int q38moe_block_forward(const void* x, const void* w_router, const void* w_gate_up,
                         const void* w_down, const void* w_sh_gate, const void* w_sh_up,
                         const void* w_sh_down, const void* w_sh_gate_proj,
                         const float* logit_bias, void* out, void* logits, int32_t* topk_idx,
                         void* topk_w, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                         int32_t Is, void* workspace, size_t workspace_bytes, int32_t dtype,
                         void* stream);

/*
 * Whole MoE block without a workspace argument and without allocating. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments, outputs and kernels as
 * q38moe_block_forward, minus workspace / workspace_bytes; the scratch is a static device array of
 * Q38MOE_NOALLOC_SCRATCH_BYTES (32 MiB) per GPU, held until the process ends, whose address is
 * looked up on the first call on each device (which must be the current device, and the stream's).
 * Shapes whose block workspace (q38moe_block_workspace_bytes, same dtype) exceeds it are rejected with
 * Q38MOE_EWORKSPACE (at h = 1024, E = 64, k = 5, I = Is = 256 it holds T <= 2173). Every call on a
 * GPU shares that GPU's scratch: calls that overlap on one GPU (different streams, or threads)
 * race and must be serialised by the caller. Nothing carried over from a previous call is read.
 */
#define Q38MOE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
size_t q38moe_block_noalloc_scratch_bytes(void);
int q38moe_block_forward_noalloc(const void* x, const void* w_router, const void* w_gate_up,
                                 const void* w_down, const void* w_sh_gate, const void* w_sh_up,
                                 const void* w_sh_down, const void* w_sh_gate_proj,
                                 const float* logit_bias, void* out, void* logits, int32_t* topk_idx,
                                 void* topk_w, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                 int32_t Is, int32_t dtype, void* stream);

/*
 * FP8 expert path, R14. There is no reference function: the benchmark set's fp8 configuration
 * (e4m3 expert weights with per-output-channel fp32 scales, per-token e4m3 activations, bf16
 * outputs) defines it, and these entry points fix its arithmetic. e4m3 is the OCP format
 * (torch.float8_e4m3fn, largest finite 448), stored one byte per value.
 *
 * Per-row quantisation of x [R,C] bf16 (C % 64 == 0, C <= 4096):
 *   amax[r] = max_c |x[r,c]| (NaN if the row holds a NaN); inv = amax > 0 ? 448/amax : 0 (fp32)
 *   q[r,c] = e4m3(round-to-nearest-even(clamp(x[r,c]*inv, -448, 448))); scale[r] = amax/448
 * so x ~ q * scale. Quantises expert weights at load time (rows = output channels:
 * gate_up [E*2I, h], down [E*h, I], shared [I,h]/[h,I]) and, inside the fp8 block, the tokens
 * and the SwiGLU rows. q must be 8-byte aligned.
 */
int q38moe_quantize_rows(const void* x, void* q, float* scale, int64_t R, int32_t C, void* stream);

/*
 * Grouped gate/up GEMM on e4m3 operands (R6 in fp8): as q38moe_gate_up, with
 *   acc = sum_c xq[tok,c] * wq[n,c] (exact e4m3 products, fp32 accumulation)
 *   g = bf16(acc_g * row_scale[r] * s_gate_up[e, n]), u likewise with row I + n; H as q38moe_gate_up.
 * xq [T,h] e4m3 tokens; row_scale [T*k + shared_rows] fp32 in sorted row order (the token scale of
 * each row; q38moe_block_forward_fp8 derives it in its permutation pass); wq_gate_up [E,2I,h]
 * e4m3 + s_gate_up [E,2I]; shared rows use wq_sh_gate/wq_sh_up [I,h] + s_sh_gate/s_sh_up [I].
 */
int q38moe_gate_up_fp8(const void* xq, const float* row_scale, const void* wq_gate_up,
                       const float* s_gate_up, const void* wq_sh_gate, const float* s_sh_gate,
                       const void* wq_sh_up, const float* s_sh_up, const int32_t* perm,
                       const int32_t* tiles, const int32_t* tile_count, int64_t shared_rows,
                       void* H, int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                       void* stream);

/*
 * Grouped down GEMM on e4m3 operands (R7 in fp8): Y[r,c] = bf16((sum_i Hq[r,i] wq[c,i]) *
 * row_scale[r] * s_down[e,c]). Hq [T*k + shared_rows, I] e4m3 with row_scale per row
 * (q38moe_quantize_rows of H); wq_down [E,h,I] e4m3 + s_down [E,h]; shared rows use wq_sh_down
 * [h,I] + s_sh_down [h].
 */
int q38moe_down_fp8(const void* Hq, const float* row_scale, const void* wq_down, const float* s_down,
                    const void* wq_sh_down, const float* s_sh_down, const int32_t* tiles,
                    const int32_t* tile_count, int64_t shared_rows, void* Y, int64_t T, int32_t h,
                    int32_t E, int32_t k, int32_t I, void* stream);

/*
 * MoE block with fp8 experts (R0 over R14): q38moe_block_forward's pipeline with the routed and
 * shared expert GEMMs on e4m3 (Is == I: the shared expert runs inside the grouped GEMMs). The
 * router and the shared-expert gate logit stay bf16 on x; x is quantised per token, the SwiGLU
 * rows per row; combine and the gated shared sum as in bf16. Weights as for q38moe_gate_up_fp8 /
 * q38moe_down_fp8. Workspace from q38moe_block_fp8_workspace_bytes. h, I <= 4096.
 */
int q38moe_block_fp8_workspace_bytes(int64_t T, int32_t h, int32_t E, int32_t k, int32_t I,
                                     size_t* bytes);
int q38moe_block_forward_fp8(const void* x, const void* w_router, const void* wq_gate_up,
                             const float* s_gate_up, const void* wq_down, const float* s_down,
                             const void* wq_sh_gate, const float* s_sh_gate, const void* wq_sh_up,
                             const float* s_sh_up, const void* wq_sh_down, const float* s_sh_down,
                             const void* w_sh_gate_proj, const float* logit_bias, void* out,
                             void* logits, int32_t* topk_idx, void* topk_w, int64_t T, int32_t h,
                             int32_t E, int32_t k, int32_t I, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Experts backward (the differentiable experts path, inference.py:358-384, whose gradients of x,
 * top_k_weights, gate_up_proj and down_proj scripts/check_q38_kernels.py:19-27 checks). The Python
 * layer chains these with q38moe_down_kn (the weights untransposed) and q38moe_combine (unit
 * weights) on the permutation and tile table of the forward, built without shared-expert rows.
 *
 * Gathered grouped GEMM: C[r] = bf16(x[perm[r] / k] . w[e]^T) for the T*k sorted rows of the tile
 * table (e = the row's expert); w [E,N,K], x [T,K], C [T*k,N] bf16; K, N multiples of 64. Used to
 * recompute the gate/up pre-activations [g | u] (w = gate_up_proj, N = 2I, K = h).
 */
int q38moe_gather_gemm(const void* x, const int32_t* perm, const void* w, const int32_t* tiles,
                       const int32_t* tile_count, void* C, int64_t T, int32_t K, int32_t N, int32_t E,
                       int32_t k, void* stream);

/*
 * Training forward of the routed experts' gate/up (the padded path's bmm gate/up and SiLU * up,
 * inference.py:370-378, whose inputs its backward needs): q38moe_gate_up on routed rows only (tile
 * table without shared-expert rows), which also writes the rounded pre-activations
 *   GU[r] = [bf16(x_r . w_gate_up[e, :I]) | bf16(x_r . w_gate_up[e, I:])]   [T*k, 2I] bf16
 * next to H [T*k, I]. They are the values H is computed from, bit-identical to q38moe_gather_gemm
 * on the same tiles, so the backward's SwiGLU step reads them instead of recomputing them.
 * Shared-expert tiles in the table (group E, from q38moe_permute with shared_rows > 0) are skipped:
 * their rows are neither read nor written.
 */
int q38moe_gate_up_save(const void* x, const void* w_gate_up, const int32_t* perm, const int32_t* tiles,
                        const int32_t* tile_count, void* H, void* GU, int64_t T, int32_t h, int32_t E, int32_t k,
                        int32_t I, void* stream);

/*
 * Grouped product with K-major expert weights, for the input-gradient products of the padded
 * path's bmm backward (inference.py:374-380), which multiply by the expert weights themselves:
 *   Y[r, n] = bf16(sum_j A[r, j] * w_kn[e, j, n])   for the T*k sorted rows of the tile table
 * (e = the row's expert; tables built without shared-expert rows). A [T*k,K], w_kn [E,K,N],
 * Y [T*k,N] bf16; K, N multiples of 64. The same products, K order and rounding as q38moe_down
 * on the per-expert transposes of w_kn (bit-identical results), without the transposes:
 *   dH rows:       A = routed rows' gradient (K = h), w_kn = down_proj [E,h,I]     -> N = I
 *   dx rows:       A = [d_g | d_u] (K = 2I),          w_kn = gate_up_proj [E,2I,h] -> N = h
 * Shared-expert tiles in the table (group E) are skipped: their rows are neither read nor written.
 */
int q38moe_down_kn(const void* A, const void* w_kn, const int32_t* tiles, const int32_t* tile_count, void* Y,
                   int64_t T, int32_t K, int32_t N, int32_t E, int32_t k, void* stream);

/*
 * Routing-weight gradient (routed = raw * top_k_weights, inference.py:381):
 *   dw[p] = bf16(sum_c fp32(bf16(dout[t,c] * Y[inv[p],c])))   for pairs p = t*k + j,
 * Y the unweighted down rows in sorted order [T*k,h]; pairs whose expert lies outside [0,E) get 0.
 * With d_raw (and topk_w [T*k] bf16) given, the same pass writes the routed raw rows' gradient in
 * sorted order, d_raw[inv[p]] = bf16(dout[t] * topk_w[p]) (as q38moe_gather_rows with w), rows of
 * dropped pairs left unwritten; d_raw [T*k,h] bf16. topk_w and d_raw may be NULL.
 */
int q38moe_pair_dots(const void* dout, const void* Y, const int32_t* inv, const void* topk_idx,
                     int32_t idx_is_int64, const void* topk_w, void* dw, void* d_raw, int64_t T, int32_t h,
                     int32_t E, int32_t k, void* stream);

/*
 * Rows in sorted order: dst[r] = bf16(src[perm[r] / k] * w[perm[r]]), or the plain gathered row
 * when w is NULL (the routed raw rows' gradient dout * top_k_weights), for the rows
 * r < starts[E-1] + counts[E-1] that the permutation filled (fewer than T*k when indices outside
 * [0,E) were dropped; the count is read on the device, no host synchronisation). src [T,h],
 * w [T*k], starts/counts [E] from q38moe_permute, dst [T*k,h] bf16 (rows past the filled ones are
 * left unwritten).
 */
int q38moe_gather_rows(const void* src, const int32_t* perm, const void* w, const int32_t* starts,
                       const int32_t* counts, void* dst, int64_t T, int32_t h, int32_t E, int32_t k,
                       void* stream);

/*
 * Per-expert transpose dst[e] = src[e]^T, bf16 [E,R,C] -> [E,C,R], R and C multiples of 64 (the
 * transposes inside the padded path's bmm backward, inference.py:374-380): down_proj [E,h,I] ->
 * [E,I,h], gate_up_proj [E,2I,h] -> [E,h,2I], the operands of q38moe_down for the input-gradient
 * products (q38moe_down_kn takes the weights untransposed). src and dst must not overlap.
 */
int q38moe_transpose_experts(const void* src, void* dst, int32_t E, int32_t R, int32_t C, void* stream);

/*
 * Expert weight gradients (the per-expert weight products of the padded path's bmm backward,
 * inference.py:374-380): dW[e][m][n] = bf16(sum over expert e's sorted rows r of G[r][m] * X[s(r)][n])
 * with the rows of e = [starts[e], starts[e] + counts[e]) and s(r) = perm[r] / k (X = the tokens
 * [T,N], gathered) or s(r) = r when perm is NULL (X = sorted rows [T*k,N]). G [T*k,M], dW [E,M,N]
 * bf16, every element written (experts without rows, and every expert when T = 0, get zeros);
 * M, N multiples of 64.
 *   gate_up_proj's gradient: G = [d_g | d_u] (M = 2I), X = x, perm given      -> [E, 2I, h]
 *   down_proj's gradient:    G = routed rows' gradient (M = h), X = H, no perm -> [E, h, I]
 */
int q38moe_expert_wgrad(const void* G, const void* X, const int32_t* perm, const int32_t* starts,
                        const int32_t* counts, void* dW, int64_t T, int32_t M, int32_t N, int32_t E,
                        int32_t k, void* stream);

/*
 * SwiGLU backward (act = bf16(silu(g)), h = bf16(act * u), inference.py:378):
 *   d_u = bf16(dh * act), d_g = bf16(bf16(dh * u) * sigmoid(g) * (1 + g * (1 - sigmoid(g))))
 * dH [rows,I], GU = [g | u] [rows,2I], dGU = [d_g | d_u] [rows,2I] bf16; I a multiple of 64.
 */
int q38moe_swiglu_backward(const void* dH, const void* GU, void* dGU, int64_t rows, int32_t I,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q38MOE_H */
