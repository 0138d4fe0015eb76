/*
 * crane_layer.h -- C ABI of the row kernels that sit either side of the
 * attention block in a decoder layer (gfx950).
 *
 * One Qwen3 / Qwen2.5 / Hunyuan decoder layer (qwen3/modeling.rs:655-673) is
 *   h = x + attn(input_layernorm(x));  out = h + mlp(post_attention_layernorm(h))
 * with mlp = down(silu(gate) * up).  These launchers replace the candle ops
 * around the GEMMs:
 *
 *   crane_hip_rms_norm       candle_nn::RmsNorm::forward on a contiguous
 *       [rows, cols] tensor (input_layernorm, post_attention_layernorm, the
 *       final norm): the fused candle ops::rms_norm, f32 sum of squares,
 *       m = sqrt(sum/cols + eps) rounded to T, y = x / m * w with each op
 *       rounded to T.  The sum's f32 order depends on the row count: calls
 *       of fewer than 1024 rows run a workgroup per row, larger ones a wave
 *       per row, so a row's m (and then its output) can differ in the last
 *       bit between such calls.  crane_hip_add_rms_norm likewise.
 *   crane_hip_add_rms_norm   `residual + hidden` followed by the next RmsNorm
 *       (qwen3/modeling.rs:666-669, and the next layer's input_layernorm).
 *       Crane's FusedAddRmsNorm (crane-core/src/fused_ops/cuda_impl.rs:200-258)
 *       runs exactly that candle pair: the sum is rounded to T and written
 *       back to `residual`, and the norm is taken of the rounded sum.  Here
 *       both happen in one pass over HBM.
 *   crane_hip_silu_mul       Crane's fused_silu_mul (fused_ops.cu:104-126,
 *       cuda_impl.rs:31-186, called at qwen3/modeling.rs:573-585): over
 *       gate_up [rows, 2*inter] (gate || up), out = T(silu(g) * u) with
 *       silu(g) = g / (1 + exp(-g)) in f32.
 *   crane_hip_residual_add   fused_residual_add (fused_ops.cu:382-393):
 *       residual = T(residual + hidden), in place.
 *
 * Conventions are those of crane_hip.h (status codes, host-side checks,
 * stream order, no allocation, no state).  dtype is CRANE_HIP_F32 or
 * CRANE_HIP_BF16 for every tensor of a call; arithmetic is f32.  Rows are
 * contiguous with `cols` (or 2*inter) elements; pointers are 16-byte aligned
 * and cols (inter) is a multiple of 8 for bf16 and of 4 for f32.
 */
#ifndef CRANE_LAYER_H
#define CRANE_LAYER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest row the norm kernels take (every supported model's hidden size fits). */
#define CRANE_LAYER_MAX_COLS 8192

/* out[r, :] = RmsNorm(x[r, :]) * w  (w [cols], or NULL for weight 1). */
int crane_hip_rms_norm(const void* x, const void* w, void* out, int64_t rows, int cols, float eps, int dtype,
                       void* stream);

/* residual[r, :] = T(residual[r, :] + hidden[r, :]) (in place), then
 * out[r, :] = RmsNorm(residual[r, :]) * w.  out may not alias residual or hidden. */
int crane_hip_add_rms_norm(void* residual, const void* hidden, const void* w, void* out, int64_t rows, int cols,
                           float eps, int dtype, void* stream);

/* out [rows, inter] = T(silu(gate_up[r, i]) * gate_up[r, inter + i]). */
int crane_hip_silu_mul(const void* gate_up, void* out, int64_t rows, int inter, int dtype, void* stream);

/* residual[i] = T(residual[i] + hidden[i]) for i < n (n a multiple of 8). */
int crane_hip_residual_add(void* residual, const void* hidden, int64_t n, int dtype, void* stream);

/* crane_hip_add_rms_norm with hidden = T(sum_s parts[s]): parts are the f32
 * split-K partial products [n_parts, rows, cols] of crane_gemm_linear_split,
 * summed in split order and rounded once to T (as the whole product's output
 * would be), then added to residual and normed as there.  Same rounding
 * points as the projection followed by crane_hip_add_rms_norm (the
 * projection's f32 summation order aside).  1 <= n_parts <= 64; out may not
 * alias residual or parts. */
int crane_hip_add_rms_norm_parts(void* residual, const float* parts, int n_parts, const void* w, void* out,
                                 int64_t rows, int cols, float eps, int dtype, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_LAYER_H */
