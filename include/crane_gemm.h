/*
 * crane_gemm.h -- C ABI of the projections of a decoder layer: the merged QKV
 * projection that feeds crane_hip_qknorm_rope_append, o_proj that consumes
 * the attention output, the MLP projections and the lm_head (gfx950).
 *
 * Crane's projections are candle Linear layers (qwen3/modeling.rs:207-223,
 * 382-387 qkv_proj; :466 and :502 o_proj; the QKV bias of Qwen2.5,
 * qwen25/qwen2.rs:136-138): y = x W^T (+ b) with W stored [N, K] (out
 * features x in features, row-major) and x [M, K] row-major.  The merged qkv
 * output [M, (Hq + 2 Hkv) D] is exactly the `qkv` rows of the fused append,
 * and the attention output [B, S, Hq D] is exactly o_proj's x.
 *
 * The same call serves the MLP projections (gate_up, down) and the lm_head.
 * Products go to hipBLASLt with f32 accumulation, the bias added in the
 * epilogue (one rounding of acc + b, where candle rounds the product and then
 * the sum), except bf16 products with few token rows (M <= 32), which
 * hand-written kernels run with the same accumulation and rounding: a per-wave
 * ring kernel when K <= 8192 splits into its pipelines, by these rules:
 *   N <= 4096:         N a multiple of 16 and K of 2048;
 *   4096 < N <= 8192:  N a multiple of 32 and K of 1024;
 *   N > 8192:          of the configurations of 96 features (K a multiple of
 *                      512), 64 and 48 features (K of 1024) whose N is a
 *                      multiple of the feature count, the one that gives the
 *                      busiest CU the fewest features (the first listed on a
 *                      tie); gate_up + SiLU (crane_gemm_linear_silu_mul) takes
 *                      96 or 64 only
 * (the decode step's qkv_proj, o_proj, gate_up and lm_head), else a streaming
 * kernel for N >= 16384 (N a multiple of 64, K of 128).  The kernel that runs
 * a shape fixes the f32 summation order of its products.  A crane_gemm
 * context holds the hipBLASLt handle,
 * a workspace allocated at creation and the algorithm chosen for each shape
 * (the heuristic query runs once per shape).  Conventions otherwise as in
 * crane_hip.h; crane_gemm_linear does not allocate or synchronise.  Calls on
 * one context from several threads are serialised on the host.  Every call
 * on a context uses its one workspace, so calls whose GPU work may overlap
 * (on different streams) need different contexts.  A context belongs to the
 * device that was current at creation.
 */
#ifndef CRANE_GEMM_H
#define CRANE_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct crane_gemm crane_gemm;

/* A context with `workspace_bytes` of GEMM workspace (0 for the default, 32 MiB). */
int crane_gemm_create(size_t workspace_bytes, crane_gemm** out);
void crane_gemm_destroy(crane_gemm* g);

/* y[M, N] = x[M, K] W[N, K]^T (+ bias[N]) in `dtype` (CRANE_HIP_F32 or
 * CRANE_HIP_BF16), f32 accumulation; bias may be NULL.  Pointers are 16-byte
 * aligned; M, N, K > 0 (M == 0 does nothing). */
int crane_gemm_linear(crane_gemm* g, const void* x, const void* w, const void* bias, void* y, int64_t M, int64_t N,
                      int64_t K, int dtype, void* stream);

/* 1 when crane_gemm_linear_silu_mul takes the shape, else 0: bf16, M <= 32
 * token rows, K <= 8192, inter > 4096, and inter a multiple of 48 with K a
 * multiple of 512 or inter a multiple of 32 with K a multiple of 1024 (the
 * per-wave ring kernel's gated configurations; the Qwen3-8B decode step's
 * gate_up, inter 12288, K 4096, is one).  For other shapes run
 * crane_gemm_linear into a [M, 2 inter] buffer and crane_hip_silu_mul
 * (crane_layer.h). */
int crane_gemm_silu_mul_supported(int64_t M, int64_t inter, int64_t K, int dtype);

/* out[M, inter] = T(silu(g) * u) where [g | u] = T(x[M, K] W[2 inter, K]^T),
 * W the merged gate_up weight (gate rows first): Crane's Mlp gate / up
 * projections followed by fused_silu_mul (qwen3/modeling.rs:573-585), in one
 * launch.  The roundings are those of crane_gemm_linear (no bias) followed by
 * crane_hip_silu_mul: each projection rounded to T, then silu(g) * u in f32
 * rounded once; the projections' f32 summation order is the kernel's own.
 * CRANE_HIP_E_INVALID for a shape crane_gemm_silu_mul_supported rejects. */
int crane_gemm_linear_silu_mul(crane_gemm* g, const void* x, const void* w, void* out, int64_t M, int64_t inter,
                               int64_t K, int dtype, void* stream);

/* 1 when crane_gemm_linear_split takes the shape, else 0: bf16, M <= 32 token
 * rows, N a multiple of 32 or 48, 2 <= splits <= 16, and K a multiple of splits
 * whose share K / splits is at most 32768 and a multiple of 512 (of 256 from
 * 3072 up). */
int crane_gemm_split_supported(int64_t M, int64_t N, int64_t K, int splits, int dtype);

/* The f32 partial products of a projection whose output only feeds a
 * residual add or the fused append: part[s][M][N] = sum over k in
 * [s K / splits, (s + 1) K / splits) of x[M, K] W[N, K]^T, unrounded, no
 * bias.  The sum over s in split order, rounded once to T, is
 * crane_gemm_linear's output up to the f32 summation order;
 * crane_hip_add_rms_norm_parts (crane_layer.h) and
 * crane_hip_qknorm_rope_append_parts (crane_hip.h) consume it.
 * Each workgroup covers 32, 48 or 64 output features over one split of K
 * (the width that spreads the workgroups most evenly over the CUs), so a
 * decode step's narrow products (qkv_proj, o_proj, down_proj) fill the chip
 * and read x splits times less per weight byte than crane_gemm_linear's
 * kernels.  No counterpart in the
 * reference (candle rounds each matmul's output); part is 16-byte aligned
 * and holds splits * M * N floats.  CRANE_HIP_E_INVALID for a shape
 * crane_gemm_split_supported rejects. */
int crane_gemm_linear_split(crane_gemm* g, const void* x, const void* w, float* part, int64_t M, int64_t N, int64_t K,
                            int splits, int dtype, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CRANE_GEMM_H */
