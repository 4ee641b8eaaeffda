/*
 * C ABI of the decode-step normalisation kernels around the MoE and KDA
 * blocks: RMSNorm, the residual add fused with the RMSNorm that follows it,
 * and the gated RMSNorm of the KDA output.
 *
 * Same conventions as lk_w4a16.h: device pointers, element counts, a
 * hipStream_t passed as void*, LK_OK or an error code (message from
 * lk_last_error()); nothing allocates or synchronises, so every call can be
 * captured in a HIP graph. Rows are dense and row-major. Dtype codes are
 * those of lk_kda.h: LK_DTYPE_F32 = 0, LK_DTYPE_F16 = 1, LK_DTYPE_BF16 = 2.
 *
 * Row widths: a multiple of 8 up to 8192. Each row's mean square is an fp32
 * sum in a fixed order (lane-sequential, then a butterfly), so reruns are
 * bit-identical.
 */
#ifndef LK_NORM_H
#define LK_NORM_H

#include "lk_kda.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- RMSNorm: engine/klinear/norm.py:9-13 (rms_norm)
 * x [rows, hidden] (x_dtype), weight [hidden] (weight_dtype); per row
 *   n = to_x_dtype(fp32(x) * rsqrt(mean(fp32(x)^2) + eps))
 *   y = weight * n  in torch's promoted dtype: x_dtype when weight_dtype ==
 *   x_dtype (the product rounded once from fp32), else fp32.
 * y may not alias x. */
LK_API int lk_rms_norm(const void* x, const void* weight, void* y, int64_t rows, int64_t hidden,
                       float eps, int x_dtype, int weight_dtype, void* stream);

/* ---- residual add + RMSNorm: engine/klinear/layer.py:156-160 (hidden =
 *      residual + attended; post_attention_layernorm(hidden)) and :170 with
 *      the next layer's input_layernorm (layer.py:152-153)
 * residual, delta [rows, hidden] (x_dtype): sum = to_x_dtype(fp32(residual) +
 * fp32(delta)) is written to sum_out, and y = rms_norm(sum) as lk_rms_norm.
 * sum_out may alias residual or delta (each element is read and written by
 * the same lane); y may alias neither. */
LK_API int lk_add_rms_norm(const void* residual, const void* delta, const void* weight,
                           void* sum_out, void* y, int64_t rows, int64_t hidden, float eps,
                           int x_dtype, int weight_dtype, void* stream);

/* ---- gated RMSNorm: engine/klinear/norm.py:33-52 (RMSGatedNorm.forward),
 *      the KDA output norm of engine/klinear/attention.py:324-329
 * values [rows, dim] (values_dtype) are first rounded to input_dtype (the
 * reference's .to(hidden_states.dtype) before o_norm; a no-op when the two
 * match); gate [rows, dim] (gate_dtype); weight [dim] (weight_dtype); per row
 *   v = fp32(values);  n = v * rsqrt(mean(v^2) + eps)
 *   y = to_input_dtype(n * fp32(weight) * sigmoid(fp32(gate))).
 * y [rows, dim] in input_dtype; it may not alias values or gate. */
LK_API int lk_rms_gated_norm(const void* values, const void* gate, const void* weight, void* y,
                             int64_t rows, int64_t dim, float eps, int values_dtype,
                             int input_dtype, int gate_dtype, int weight_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LK_NORM_H */
