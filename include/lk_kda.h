/*
 * C ABI of the Kimi Delta Attention (KDA) decode kernels: the recurrent-state
 * step and its launch-fused preparation (short convolutions, gates).
 *
 * Same conventions as lk_w4a16.h: device pointers, element counts, a
 * hipStream_t passed as void*, LK_OK or an error code (message from
 * lk_last_error()); nothing allocates or synchronises, so every call can be
 * captured in a HIP graph. All tensors are dense row-major.
 *
 * Value dtype codes: LK_DTYPE_F32 = 0, LK_DTYPE_F16 = 1, LK_DTYPE_BF16 = 2
 * (fp16 / bf16 as uint16_t bit patterns).
 */
#ifndef LK_KDA_H
#define LK_KDA_H

#include "lk_w4a16.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LK_DTYPE_F32 0
#define LK_DTYPE_F16 1
#define LK_DTYPE_BF16 2

/* ---- one decode step of the KDA recurrence, state updated in place:
 *      engine/kernels/kda_step.py:273-293 (kda_decode_step; the recurrence of
 *      kda_decode_step_reference, :173-196)
 * state fp32 [B, H, d_k, d_v]; q, k, decay fp32 [B, H, d_k]; v fp32
 * [B, H, d_v]; beta fp32 [B, H]; out fp32 [B, H, d_v]:
 *   S <- S * exp(decay) (per key row); S <- S + beta * k (v - S^T k)^T;
 *   out = S^T (q * scale).
 * d_k <= 256. */
LK_API int lk_kda_decode_step(float* state, const float* q, const float* k, const float* v,
                              const float* decay, const float* beta, float* out, int64_t batch,
                              int64_t heads, int64_t d_k, int64_t d_v, float scale,
                              void* stream);

/* ---- the three width-4 decode convolutions in one launch:
 *      engine/kernels/kda_prepare.py:479-538 (fused_short_conv_triple)
 * inputs q/k/v_in [B, 1, C] and states [B, C, 4] in value_dtype; weights
 * [C, 4] (the [C, 1, 4] conv weight) in weight_dtype; outputs [B, 1, C] in
 * value_dtype. Per channel: window = (state[1], state[2], state[3], token),
 * out = silu(sum_j window[j] * weight[j]) in fp32, rounded to value_dtype;
 * the window becomes the state. */
LK_API int lk_kda_short_conv_triple(const void* q_in, const void* k_in, const void* v_in,
                                    void* q_state, void* k_state, void* v_state,
                                    const void* q_weight, const void* k_weight,
                                    const void* v_weight, void* q_out, void* k_out, void* v_out,
                                    int64_t batch, int64_t channels, int value_dtype,
                                    int weight_dtype, void* stream);

/* ---- decay, beta and per-head q/k normalisation in one launch:
 *      engine/kernels/kda_prepare.py:630-686 (fused_kda_gates)
 * rows = batch * sequence. raw_decay [rows, H, D] (decay_dtype), dt_bias fp32
 * [H * D], a_log fp32 [H], raw_beta [rows, H] (beta_dtype), q and k
 * [rows, H * D] (qk_dtype); outputs fp32: decay [rows, H, D] =
 * -exp(a_log[h]) * softplus(raw_decay + dt_bias) (softplus(x) = x above 20),
 * beta [rows, H] = sigmoid(raw_beta), q_out / k_out [rows, H, D] = x *
 * rsqrt(sum over the head of x^2 + eps). head_dim <= 1024. */
LK_API int lk_kda_gates(const void* raw_decay, const float* dt_bias, const float* a_log,
                        const void* raw_beta, const void* q, const void* k, float* decay,
                        float* beta, float* q_out, float* k_out, int64_t rows, int64_t heads,
                        int64_t head_dim, float eps, int decay_dtype, int beta_dtype,
                        int qk_dtype, void* stream);

/* ---- a whole KDA decode layer in one launch. No reference counterpart: it
 * runs, for one token per batch row, what engine/klinear/attention.py:193-271
 * runs through fused_short_conv_triple, fused_kda_gates and kda_decode_step
 * (three launches there, plus the bf16 -> fp32 view of v), with one block
 * per (batch row, head). Inputs as lk_kda_short_conv_triple (C = heads *
 * head_dim) and lk_kda_gates (rows = batch, sequence one); state fp32
 * [B, H, D, D] and out fp32 [B, H, D] as lk_kda_decode_step with
 * d_k = d_v = D. Conv states and state are updated in place. q, k, v, decay
 * and beta are bit-identical to the three-launch chain's; the step sums its
 * row groups in another order. head_dim a multiple of 4, at most 128. */
LK_API int lk_kda_decode_layer(const void* q_in, const void* k_in, const void* v_in,
                               void* q_state, void* k_state, void* v_state,
                               const void* q_weight, const void* k_weight,
                               const void* v_weight, const void* raw_decay,
                               const float* dt_bias, const float* a_log, const void* raw_beta,
                               float* state, float* out, int64_t batch, int64_t heads,
                               int64_t head_dim, float eps, float scale, int value_dtype,
                               int weight_dtype, int decay_dtype, int beta_dtype, void* stream);

/* ---- the same layer over several blocks per head (no reference counterpart)
 * Arguments as lk_kda_decode_layer, except that the convolution states are
 * read from q/k/v_state and the shifted states written to q/k/v_state_out
 * (distinct buffers; callers alternate the two from call to call), which lets
 * a head's value columns be split over blocks of 16 without a block reading a
 * state another block already shifted. The recurrent state is updated in
 * place. q, k, v, decay and beta are bit-identical to lk_kda_decode_layer's;
 * the step sums its rows in another grouping. head_dim a multiple of 4, at
 * most 128. */
LK_API int lk_kda_decode_layer_split(const void* q_in, const void* k_in, const void* v_in,
                                     const void* q_state, const void* k_state,
                                     const void* v_state, void* q_state_out, void* k_state_out,
                                     void* v_state_out, const void* q_weight,
                                     const void* k_weight, const void* v_weight,
                                     const void* raw_decay, const float* dt_bias,
                                     const float* a_log, const void* raw_beta, float* state,
                                     float* out, int64_t batch, int64_t heads, int64_t head_dim,
                                     float eps, float scale, int value_dtype, int weight_dtype,
                                     int decay_dtype, int beta_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LK_KDA_H */
