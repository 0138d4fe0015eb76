/*
 * crane_sampling.h -- C ABI of the token-selection kernels the engine runs on
 * the logits after every decode step (gfx950).
 *
 *   crane_hip_argmax  replaces gpu_argmax (crane-core/src/fused_ops/cuda_impl.rs:
 *       266-356, kernels/fused_ops.cu:244-375), Crane's greedy path
 *       (crane-serve/src/engine/sampling.rs:127-147), for a batch of rows.
 *   crane_hip_topk    replaces topk_indices (cuda_impl.rs:374-545,
 *       fused_ops.cu:404-532), the candidate set of top-k / top-p sampling
 *       (sampling.rs:185-190), k <= 64, for a batch of rows.
 *
 * Order: by value, descending; equal values by index, ascending (candle's
 * CPU argmax returns the first maximum; the top-k order is the reference's
 * descending order with its ties made deterministic).  NaN ranks below every
 * number, -inf included; -0 and +0 are equal.  Conventions as in crane_hip.h; no allocation, no
 * state.  Rows are contiguous, row r at logits + r * n elements.
 */
#ifndef CRANE_SAMPLING_H
#define CRANE_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CRANE_TOPK_MAX 64

/* out_idx[r] = index of the largest logits[r, :] (dtype CRANE_HIP_F32 or
 * CRANE_HIP_BF16); 1 <= n < 2^31. */
int crane_hip_argmax(const void* logits, int64_t rows, int64_t n, int dtype, uint32_t* out_idx, void* stream);

/* out_idx[r, 0..k) = indices of the k largest x[r, :] (f32) in the order
 * above; 1 <= k <= min(n, CRANE_TOPK_MAX), n < 2^31. */
int crane_hip_topk(const float* x, int64_t rows, int64_t n, int k, uint32_t* out_idx, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_SAMPLING_H */
