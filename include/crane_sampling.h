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
 * state (the _ws variants: no state beyond the caller's workspace).  Rows are
 * contiguous, row r at logits + r * n elements.
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

/* The same selections with a workspace, for few rows: with at most 32 rows of
 * at least 32768 entries each row is split over 64..256 workgroups (the
 * reference's gpu_argmax spreads a row over 149 blocks and merges in a second
 * phase, fused_ops.cu:244-375, cuda_impl.rs:296-335; topk_indices merges
 * per-block candidates, fused_ops.cu:404-532) and the result comes from 2
 * (argmax) or 3 (top-k) kernels that meet in the workspace; other shapes run
 * the single-pass kernels above and ignore it.  Same results, bit for bit.
 * crane_hip_select_workspace_bytes(rows, n) is the size both need (0 when no
 * split applies); the workspace is 16-byte aligned, holds nothing between
 * calls and needs no clearing; calls that overlap on one workspace race.
 * Returns CRANE_HIP_E_CAPACITY for a missing or short workspace. */
size_t crane_hip_select_workspace_bytes(int64_t rows, int64_t n);
int crane_hip_argmax_ws(const void* logits, int64_t rows, int64_t n, int dtype, void* workspace, size_t ws_bytes,
                        uint32_t* out_idx, void* stream);
int crane_hip_topk_ws(const float* x, int64_t rows, int64_t n, int k, void* workspace, size_t ws_bytes,
                      uint32_t* out_idx, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_SAMPLING_H */
