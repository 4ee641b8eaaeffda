/*
 * C ABI of the MI355X (gfx950) W4A16 / MXFP4 quantized-matmul library.
 *
 * Every entry point takes plain device pointers, element counts and a
 * hipStream_t passed as void*. Nothing allocates, synchronises the device or
 * reads device memory on the host, so each call is safe inside HIP graph
 * capture. Return value: LK_OK, or an error code with a message available
 * from lk_last_error() (per calling thread).
 *
 * Layouts (engine/quant/w4a16.py:1-6, 46-47, 94-99 of the reference):
 *   bf16          uint16_t bit patterns
 *   packed        uint8_t [N, K/2]; byte j holds k=2j in the low nibble and
 *                 k=2j+1 in the high nibble; 4-bit two's complement codes
 *   scales        bf16 [N, K/G]; one scale per G consecutive k
 *   grouped banks packed [E, N, K/2], scales [E, N, K/G]
 *   MXFP4         packed uint8_t [N, K/2] E2M1 (low nibble first),
 *                 scale uint8_t [N, K/32] E8M0 (bias 127)
 * All tensors are dense row-major. G must be a multiple of 32 dividing K.
 * The reference fixes G=32 (engine/quant/w4a16.py:14); here G is an argument.
 *
 * Each declaration cites the reference interface it replaces.
 */
#ifndef LK_W4A16_H
#define LK_W4A16_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define LK_API __attribute__((visibility("default")))
#else
#define LK_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define LK_OK 0
#define LK_ERR_ARGUMENT 1
#define LK_ERR_HIP 2

/* Message describing the last failure on this thread ("" when none). */
LK_API const char* lk_last_error(void);

/* ABI version of this library. */
LK_API int lk_abi_version(void);

/* Kernel-form selection for this process. No reference counterpart: the
 * reference selects whole ops through its registry (KIMI_KERNELS), which this
 * library's Python layer keeps; these knobs choose among this library's own
 * forms of one op, so tests and measurements can run every form. Every knob
 * starts at "auto" (the library's measured choice) and the library reads no
 * environment variable. Knobs and choices:
 *   "moe_gemm"           auto | lds | stream16 | stream64  (expert-major GEMM)
 *   "moe_persist"        auto | off       (persistent 16-row expert GEMM)
 *   "dense_gemm"         auto | lds       (dense GEMM / fused QKV from 16 rows)
 *   "mxfp4_mfma"         auto | fp4 | bf16 (MXFP4 expert GEMM MFMA form)
 *   "moe_fused_schedule" auto | off       (router + schedule in one launch)
 *   "moe_split_swiglu"   auto | off       (split gate/up units, SwiGLU in the
 *                                          down GEMM's staging)
 * Process-wide; set it between calls, not while another thread launches.
 * lk_get_path returns the current choice's index (0 = auto), -1 for an
 * unknown knob. */
LK_API int lk_set_path(const char* knob, const char* choice);
LK_API int lk_get_path(const char* knob);

/* ---- codec: engine/quant/w4a16.py:68-105 (quantise), :108-129 (dequantise) */

/* weight bf16 [N,K] -> packed [N,K/2], scales bf16 [N,K/G]; bit-exact with
 * the reference encoder (absmax/7 scale stored as bf16, codes rounded half
 * to even against the stored scale, clamped to [-7, 7]). */
LK_API int lk_w4a16_quantise(const uint16_t* weight, uint8_t* packed, uint16_t* scales,
                      int64_t n, int64_t k, int64_t group_size, void* stream);

/* packed + scales -> out [N,K]: bf16(q * scale) as bf16 when out_f32 == 0,
 * or the exact q * scale as float32 when out_f32 != 0. */
LK_API int lk_w4a16_dequantise(const uint8_t* packed, const uint16_t* scales, void* out,
                               int64_t n, int64_t k, int64_t group_size, int out_f32,
                               void* stream);

/* ---- op w4a16_dense: engine/kernels/__init__.py:82-125 (signature),
 *      engine/kernels/w4a16_dense_gemv.py:312-336 (default variant)
 * y bf16 [M,N] = x bf16 [M,K] . dequant(W)^T, fp32 accumulation. */
LK_API int lk_w4a16_dense(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                   uint16_t* y, int64_t m, int64_t n, int64_t k, int64_t group_size,
                   void* stream);

/* Same op with the reference's rounding contract (weights rounded to bf16
 * before the fp32 multiply-add, one thread per output); the registry's
 * "reference" variant. engine/quant/triton_w4a16.py:151-188. */
LK_API int lk_w4a16_dense_reference(const uint16_t* x, const uint8_t* packed,
                             const uint16_t* scales, uint16_t* y, int64_t m, int64_t n,
                             int64_t k, int64_t group_size, void* stream);

/* ---- op w4a16_grouped: engine/kernels/__init__.py:26-79,
 *      engine/kernels/w4a16_gemv.py:610-635
 * out bf16 [T,R,N]: out[t,r] = x[t] . dequant(W[idx[t,r]])^T. */
LK_API int lk_w4a16_grouped(const uint16_t* x, const int64_t* expert_indices,
                     const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                     int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                     int64_t k, int64_t group_size, void* stream);

/* Reference-rounding variant (engine/kernels/w4a16_grouped.py:121-194). */
LK_API int lk_w4a16_grouped_reference(const uint16_t* x, const int64_t* expert_indices,
                               const uint8_t* packed, const uint16_t* scales,
                               uint16_t* out, int64_t tokens, int64_t routes,
                               int64_t experts, int64_t n, int64_t k,
                               int64_t group_size, void* stream);

/* ---- op w4a16_swiglu: engine/kernels/__init__.py:164-218,
 *      engine/kernels/w4a16_gemv.py:772-790
 * act bf16 [T,R,N] = bf16(bf16(silu(bf16(x.W1^T))) * bf16(x.W3^T)). */
LK_API int lk_w4a16_swiglu(const uint16_t* x, const int64_t* expert_indices,
                    const uint8_t* w1_packed, const uint16_t* w1_scales,
                    const uint8_t* w3_packed, const uint16_t* w3_scales, uint16_t* out,
                    int64_t tokens, int64_t routes, int64_t experts, int64_t n, int64_t k,
                    int64_t group_size, void* stream);

/* Elementwise bf16(silu(gate)) * up on bf16 tensors, as the reference
 * variant of w4a16_swiglu does after its two grouped calls
 * (engine/kernels/__init__.py:195-197). */
LK_API int lk_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t count,
                void* stream);

/* Route combine on precomputed expert outputs eo bf16 [T,R,H]:
 * y = bf16(bf16(sum_{r<R-1} eo[t,r] * cw[t,r]) + eo[t,R-1]); the last route
 * is the shared expert with weight 1 (engine/klinear/moe.py:327-334). */
LK_API int lk_route_combine(const uint16_t* expert_outputs, const float* combine_weights,
                            uint16_t* y, int64_t tokens, int64_t routes, int64_t h,
                            void* stream);

/* ---- fused W2 + route combine: engine/kernels/moe_combine.py:264-324
 *      (semantics: fused_w2_combine_reference, :209-261; klinear/moe.py:317-334)
 * y bf16 [T,H] = bf16(bf16(sum_{r<R-1} bf16(act[t,r].W2[idx]^T) * cw[t,r])
 *                     + bf16(act[t,R-1].W2[idx]^T)); cw[:, R-1] is ignored. */
LK_API int lk_w4a16_w2_combine(const uint16_t* activated, const int64_t* expert_indices,
                        const float* combine_weights, const uint8_t* w2_packed,
                        const uint16_t* w2_scales, uint16_t* y, int64_t tokens,
                        int64_t routes, int64_t experts, int64_t h, int64_t i,
                        int64_t group_size, void* stream);

/* ---- router logits: engine/klinear/router.py:50-51
 * logits fp32 [T,E] = fp32(x bf16 [T,H]) . fp32(w [E,H])^T with the router
 * weight w in bf16 (weight_f32 = 0; products exact) or fp32 (weight_f32 = 1);
 * fp32 sums in a fixed order (reruns bit-identical; not torch's order).
 * Requires H % 8 == 0 and H <= 4096. */
LK_API int lk_router_logits(const uint16_t* x, const void* w, float* logits, int64_t tokens,
                            int64_t experts, int64_t h, int weight_f32, void* stream);

/* ---- router: engine/klinear/router.py:47-85 (on precomputed fp32 logits)
 * idx int64 [T,top_k] in descending choice score (sigmoid + bias), ties to the
 * lower id; weights fp32 [T,top_k] = sigmoid gathered, renormalised by
 * (sum + 1e-20) when renormalize != 0 and top_k > 1, times scaling.
 * bias may be NULL (zero). Requires experts <= 1024, top_k <= 32. */
LK_API int lk_moe_router(const float* logits, const float* bias, int64_t* expert_indices,
                  float* weights, int64_t tokens, int64_t experts, int64_t top_k,
                  float routed_scaling_factor, int renormalize, void* stream);

/* ---- grouped top-k router: engine/klinear/router.py:62-80 (num_expert_group,
 *      topk_group; on precomputed fp32 logits)
 * Group score = sum of the group's two largest choice scores (the largest
 * alone when a group holds one expert); the topk_group best groups are kept
 * (ties to the lower group), every other expert's choice becomes 0.0, then
 * the selection and weights of lk_moe_router. Requires experts <= 1024,
 * experts % num_expert_group == 0, num_expert_group <= 64,
 * 1 <= topk_group <= num_expert_group, top_k <= 32. */
LK_API int lk_moe_router_grouped(const float* logits, const float* bias, int64_t* expert_indices,
                                 float* weights, int64_t tokens, int64_t experts, int64_t top_k,
                                 int64_t num_expert_group, int64_t topk_group,
                                 float routed_scaling_factor, int renormalize, void* stream);

/* ---- first stage of the MoE block: router + gate/up + SwiGLU in one launch
 *      (engine/klinear/router.py:47-85, engine/kernels/__init__.py:182-197)
 * Writes expert_indices int64 [T,top_k], weights fp32 [T,top_k] and
 * activated bf16 [T,top_k+1,I] (route top_k is the shared expert E-1). */
LK_API int lk_w4a16_moe_gateup(const uint16_t* x, const float* logits, const float* bias,
                               const uint8_t* w1_packed, const uint16_t* w1_scales,
                               const uint8_t* w3_packed, const uint16_t* w3_scales,
                               int64_t* expert_indices, float* weights, uint16_t* activated,
                               int64_t tokens, int64_t experts, int64_t h, int64_t i,
                               int64_t top_k, float routed_scaling_factor, int renormalize,
                               int64_t group_size, void* stream);

/* ---- the grouped W4A16 MoE block with its router, one decode step:
 *      engine/klinear/moe.py:278-334 + engine/klinear/router.py:47-85
 * Banks hold routed experts 0..E-2 and the shared expert at E-1.
 * Writes y bf16 [T,H], expert_indices int64 [T,top_k], weights fp32
 * [T,top_k] and the SwiGLU activations into activated bf16 [T,top_k+1,I]
 * (caller-owned workspace of lk_w4a16_moe_decode_workspace() bytes).
 * Route limit of this token-major path: R = top_k + 1 routes with either
 * I == 1024 and R <= 16, or R <= 32 and R * (I/32 * 68 + 32) <= 65536; other
 * shapes are rejected before anything is launched (the expert-major
 * lk_w4a16_moe_forward has no such limit). The workspace query returns -1 for
 * them. */
LK_API int64_t lk_w4a16_moe_decode_workspace(int64_t tokens, int64_t experts, int64_t h,
                                             int64_t i, int64_t top_k);
LK_API int lk_w4a16_moe_decode(const uint16_t* x, const float* logits, const float* bias,
                        const uint8_t* w1_packed, const uint16_t* w1_scales,
                        const uint8_t* w3_packed, const uint16_t* w3_scales,
                        const uint8_t* w2_packed, const uint16_t* w2_scales, uint16_t* y,
                        int64_t* expert_indices, float* weights, uint16_t* activated,
                        int64_t tokens, int64_t experts, int64_t h, int64_t i,
                        int64_t top_k, float routed_scaling_factor, int renormalize,
                        int64_t group_size, void* stream);

/* ---- expert-major schedule: engine/kernels/moe_grouped.py:77-95
 *      (build_expert_schedule: sorted union of experts, occurrences in
 *      row-major (token, slot) order), as counting-sort tables
 * The route table has R = routes (+1 when shared_expert >= 0) entries per
 * token: entry t*R + r is expert_indices[t*routes + r], and entry t*R + R-1
 * is shared_expert when shared_expert >= 0. Writes
 *   offsets int32 [E+2]: bucket b < E starts at offsets[b]; bucket E holds the
 *                        routes outside [0, E); offsets[E+1] = T*R
 *   perm int32 [T*R]:    sorted position -> entry, stable (row-major within
 *                        a bucket)
 *   tiles int32 [max_tiles,4]: (expert or -1, first position, rows <= tile_rows, 0),
 *                        tile_rows 16 or 64 (max_tiles covers both)
 *   tile_count int32 [1]
 * Requires experts <= 512. Sizes from lk_moe_schedule_sizes (R as above). */
LK_API int lk_moe_schedule_sizes(int64_t tokens, int64_t routes, int64_t experts,
                                 int64_t* max_tiles, int64_t* workspace_bytes);
LK_API int lk_moe_schedule(const int64_t* expert_indices, int64_t tokens, int64_t routes,
                           int64_t experts, int64_t shared_expert, int64_t tile_rows,
                           int32_t* offsets, int32_t* perm, int32_t* tiles, int32_t* tile_count,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* ---- op w4a16_grouped / w4a16_swiglu for many token-routes (the same
 *      contracts as lk_w4a16_grouped / lk_w4a16_swiglu above): expert-major
 *      MFMA GEMM, each expert's weights read once per 64-row tile.
 *      engine/kernels/moe_grouped.py:103-160 (expert-major evaluation).
 * workspace: device memory of lk_w4a16_grouped_gemm_workspace() bytes
 * (returns -1 for invalid dimensions). */
LK_API int64_t lk_w4a16_grouped_gemm_workspace(int64_t tokens, int64_t routes, int64_t experts);
LK_API int lk_w4a16_grouped_gemm(const uint16_t* x, const int64_t* expert_indices,
                                 const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                                 int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                                 int64_t k, int64_t group_size, void* workspace,
                                 int64_t workspace_bytes, void* stream);
LK_API int lk_w4a16_swiglu_gemm(const uint16_t* x, const int64_t* expert_indices,
                                const uint8_t* w1_packed, const uint16_t* w1_scales,
                                const uint8_t* w3_packed, const uint16_t* w3_scales,
                                uint16_t* out, int64_t tokens, int64_t routes, int64_t experts,
                                int64_t n, int64_t k, int64_t group_size, void* workspace,
                                int64_t workspace_bytes, void* stream);

/* ---- op w4a16_dense for many rows (prefill): MFMA GEMM, same contract as
 *      lk_w4a16_dense. engine/quant/triton_w4a16.py:151-188 (tl.dot GEMM). */
LK_API int lk_w4a16_dense_gemm(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                               uint16_t* y, int64_t m, int64_t n, int64_t k,
                               int64_t group_size, void* stream);

/* ---- fused QKV: engine/kernels/w4a16_fused_qkv.py:342-389
 * (q, k, v) bf16 [M,N] each = x . dequant(Wq|Wk|Wv)^T, one launch: M >= 16 the
 * MFMA GEMM over the three matrices; fewer rows the decode K-split GEMV over
 * the three matrices' row blocks (the reference's K7, grid (3, N/64) at M=1). */
LK_API int lk_w4a16_fused_qkv(const uint16_t* x, const uint8_t* q_packed,
                              const uint16_t* q_scales, const uint8_t* k_packed,
                              const uint16_t* k_scales, const uint8_t* v_packed,
                              const uint16_t* v_scales, uint16_t* q, uint16_t* k_out,
                              uint16_t* v, int64_t m, int64_t n, int64_t k, int64_t group_size,
                              void* stream);

/* ---- the two GEMMs above with a caller-owned workspace (same outputs):
 *      engine/kernels/__init__.py:82-125 (w4a16_dense), w4a16_fused_qkv.py:342-389
 * From 16 rows at G = 128 (k % 128 == 0) a pre-pass writes x paired in the
 * weight decode's k order with its 128-wide group sums into the workspace and
 * the 64-row GEMM loads its rows from there straight into LDS. The workspace
 * holds lk_w4a16_dense_gemm_workspace(m, k, group) bytes (0 where that form
 * does not apply; -1 on bad input); a smaller one is refused before any launch. */
LK_API int64_t lk_w4a16_dense_gemm_workspace(int64_t m, int64_t k, int64_t group_size);
LK_API int lk_w4a16_dense_gemm_ws(const uint16_t* x, const uint8_t* packed,
                                  const uint16_t* scales, uint16_t* y, int64_t m, int64_t n,
                                  int64_t k, int64_t group_size, void* workspace,
                                  int64_t workspace_bytes, void* stream);
LK_API int lk_w4a16_fused_qkv_ws(const uint16_t* x, const uint8_t* q_packed,
                                 const uint16_t* q_scales, const uint8_t* k_packed,
                                 const uint16_t* k_scales, const uint8_t* v_packed,
                                 const uint16_t* v_scales, uint16_t* q, uint16_t* k_out,
                                 uint16_t* v, int64_t m, int64_t n, int64_t k,
                                 int64_t group_size, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/* ---- the grouped W4A16 MoE block with its router, expert-major (batched
 *      decode and prefill): engine/klinear/moe.py:278-334 +
 *      engine/klinear/router.py:47-85, evaluated per expert as in
 *      engine/kernels/moe_grouped.py:103-160.
 * Router, schedule, gate/up + SwiGLU GEMM over expert tiles, down GEMM
 * scattered to (token, route) rows, combine. Same outputs as
 * lk_w4a16_moe_decode. workspace: lk_w4a16_moe_forward_workspace() bytes
 * (returns -1 for invalid dimensions). Requires experts <= 512, h % 8 == 0. */
LK_API int64_t lk_w4a16_moe_forward_workspace(int64_t tokens, int64_t experts, int64_t h,
                                              int64_t i, int64_t top_k);
LK_API int lk_w4a16_moe_forward(const uint16_t* x, const float* logits, const float* bias,
                                const uint8_t* w1_packed, const uint16_t* w1_scales,
                                const uint8_t* w3_packed, const uint16_t* w3_scales,
                                const uint8_t* w2_packed, const uint16_t* w2_scales, uint16_t* y,
                                int64_t* expert_indices, float* weights, void* workspace,
                                int64_t workspace_bytes, int64_t tokens, int64_t experts,
                                int64_t h, int64_t i, int64_t top_k,
                                float routed_scaling_factor, int renormalize, int64_t group_size,
                                void* stream);

/* ---- the block of lk_w4a16_moe_forward for callers that cannot allocate:
 * no reference counterpart. For code under HIP graph capture, tight serving
 * loops and harnesses that forbid hipMalloc: the same arguments minus the
 * workspace, which here is a static device array of
 * lk_w4a16_moe_forward_static_capacity() bytes (12 MiB) per GPU, held until
 * the process ends. Calls whose lk_w4a16_moe_forward_workspace() exceeds it
 * are rejected before anything is launched (up to 160 tokens at the
 * Kimi-Linear shape: hidden 2304, intermediate 1024, 257 experts, top-8).
 * Nothing is allocated or freed; the scratch needs no clearing (every table
 * and row in it is written before it is read). Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, two host
 * threads) race and must be serialised by the caller. Outputs are
 * bit-identical to lk_w4a16_moe_forward's (the same kernels). */
LK_API int64_t lk_w4a16_moe_forward_static_capacity(void);
LK_API int lk_w4a16_moe_forward_static(const uint16_t* x, const float* logits, const float* bias,
                                       const uint8_t* w1_packed, const uint16_t* w1_scales,
                                       const uint8_t* w3_packed, const uint16_t* w3_scales,
                                       const uint8_t* w2_packed, const uint16_t* w2_scales,
                                       uint16_t* y, int64_t* expert_indices, float* weights,
                                       int64_t tokens, int64_t experts, int64_t h, int64_t i,
                                       int64_t top_k, float routed_scaling_factor,
                                       int renormalize, int64_t group_size, void* stream);

/* ---- MXFP4 (OCP MX): E2M1 codes low nibble first, one E8M0 exponent per
 *      32 values along K; value = e2m1 * 2**(e8m0 - 127).
 *      engine/k3ref/dequant.py:18-73 (codec), engine/kernels/reference.py:29-80
 *      (dequantize + linear), engine/kernels/mxfp4_gemm.py:191-235 (GEMM op). */

/* weight bf16 [N,K] -> packed [N,K/2], scale uint8 [N,K/32]. The reference has
 * no encoder: shared exponent floor(log2(amax)) - 2 (bias 127, clamped to
 * [0, 254], 127 for an all-zero block), elements rounded to the E2M1 grid
 * with ties to the even code and saturation at +-6 (OCP MX v1.0). */
LK_API int lk_mxfp4_quantise(const uint16_t* weight, uint8_t* packed, uint8_t* scale, int64_t n,
                             int64_t k, void* stream);

/* packed + scale -> out [N,K]: float32 values when out_f32 != 0, else bf16
 * (one rounding of the exact value; -0.0 kept). */
LK_API int lk_mxfp4_dequantise(const uint8_t* packed, const uint8_t* scale, void* out, int64_t n,
                               int64_t k, int out_f32, void* stream);

/* y [M,N] = x [M,K] . dequant(W)^T, fp32 accumulation, output in the
 * activation type: bf16 (act_f16 == 0) or fp16 (act_f16 != 0).
 * engine/kernels/mxfp4_gemm.py:191-226. */
LK_API int lk_mxfp4_gemm(const uint16_t* x, const uint8_t* packed, const uint8_t* scale,
                         uint16_t* y, int64_t m, int64_t n, int64_t k, int act_f16, void* stream);

/* The same op as the reference variant: each weight decoded to the activation
 * type, then an fp32 dot, one thread per output
 * (engine/kernels/reference.py:67-80). */
LK_API int lk_mxfp4_gemm_reference(const uint16_t* x, const uint8_t* packed, const uint8_t* scale,
                                   uint16_t* y, int64_t m, int64_t n, int64_t k, int act_f16,
                                   void* stream);

/* Grouped MXFP4 banks packed [E,N,K/2], scale [E,N,K/32]; the contracts of
 * lk_w4a16_grouped_gemm / lk_w4a16_swiglu_gemm (bf16 activations; workspace
 * from lk_w4a16_grouped_gemm_workspace). */
LK_API int lk_mxfp4_grouped_gemm(const uint16_t* x, const int64_t* expert_indices,
                                 const uint8_t* packed, const uint8_t* scale, uint16_t* out,
                                 int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                                 int64_t k, void* workspace, int64_t workspace_bytes,
                                 void* stream);
LK_API int lk_mxfp4_swiglu_gemm(const uint16_t* x, const int64_t* expert_indices,
                                const uint8_t* w1_packed, const uint8_t* w1_scale,
                                const uint8_t* w3_packed, const uint8_t* w3_scale, uint16_t* out,
                                int64_t tokens, int64_t routes, int64_t experts, int64_t n,
                                int64_t k, void* workspace, int64_t workspace_bytes,
                                void* stream);

/* The MoE block of lk_w4a16_moe_forward with MXFP4 expert banks (the
 * Kimi-Linear SwiGLU block; workspace from lk_mxfp4_moe_forward_workspace).
 * With h and i multiples of 128, prefill-sized calls (64-row expert tiles,
 * more than 2048 token-routes) run the expert GEMMs on the scaled fp4 MFMA
 * (v_mfma_scale_f32_16x16x128_f8f6f4): raw E2M1 weights and E8M0 exponents,
 * activations split into fp8 hi + lo (lk_mxfp4_split_activations); decode
 * sizes use bf16 MFMA on weights decoded by the scaled fp4 convert. The
 * environment variable LK_MXFP4_MFMA=fp4 or =bf16 forces one form. */
LK_API int64_t lk_mxfp4_moe_forward_workspace(int64_t tokens, int64_t experts, int64_t h,
                                              int64_t i, int64_t top_k);
LK_API int lk_mxfp4_moe_forward(const uint16_t* x, const float* logits, const float* bias,
                                const uint8_t* w1_packed, const uint8_t* w1_scale,
                                const uint8_t* w3_packed, const uint8_t* w3_scale,
                                const uint8_t* w2_packed, const uint8_t* w2_scale, uint16_t* y,
                                int64_t* expert_indices, float* weights, void* workspace,
                                int64_t workspace_bytes, int64_t tokens, int64_t experts,
                                int64_t h, int64_t i, int64_t top_k,
                                float routed_scaling_factor, int renormalize, void* stream);

/* fp8 split of bf16 activations x [rows, k] (k % 32 == 0) for the scaled fp4
 * MFMA; no reference counterpart (the reference multiplies bf16 activations by
 * decoded weights). Per 32 values along k: x ~= hi * 2^e_hi + lo * 2^e_lo,
 * hi/lo uint8 [rows, k] OCP E4M3 codes (nearest, ties to even, magnitudes
 * below 2^-6 flushed), scales uint16 [rows, k/32] = (e_hi + 127) | (e_lo + 127) << 8,
 * e = clamp(floor(log2(block max)) - 7, -127, 127); lo encodes the exact
 * residual. */
LK_API int lk_mxfp4_split_activations(const uint16_t* x, uint8_t* hi, uint8_t* lo,
                                      uint16_t* scales, int64_t rows, int64_t k, void* stream);

/* One packed expert MLP with K3's SiTU activation:
 * engine/kernels/moe_grouped.py:163-194 (mxfp4_expert_mlp, situ_and_mul).
 * activated bf16 [M,I] = bf16(beta*tanh(g/beta)*sigmoid(g) * lb*tanh(u/lb))
 * with g, u the bf16 gate / up projections (no lb term when
 * situ_linear_beta <= 0); y bf16 [M,H] = activated . dequant(W2)^T. */
LK_API int lk_mxfp4_expert_mlp(const uint16_t* x, const uint8_t* w1_packed,
                               const uint8_t* w1_scale, const uint8_t* w3_packed,
                               const uint8_t* w3_scale, const uint8_t* w2_packed,
                               const uint8_t* w2_scale, uint16_t* y, uint16_t* activated,
                               int64_t m, int64_t h, int64_t i, float situ_beta,
                               float situ_linear_beta, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LK_W4A16_H */
