/*
 * oracle.h -- CPU restatement of Crane's candle-CPU attention op chain.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (crane_amd/, include/)
 * links, loads or calls this library.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it, and only as the checker.
 *
 * Every function restates one step of the path as Crane runs it on candle's
 * CPU backend (candle-core / candle-nn 0.10.2, a third-party dependency that
 * is not vendored in the reference):
 *   rope tables ........ crane-core/src/models/qwen3/modeling.rs:117-145,
 *                        hunyuan_dense/modeling.rs:196-231 (NTK alpha),
 *                        qwen25/qwen2.rs:47-64 (tables in the model dtype)
 *   QK-RMSNorm + RoPE .. qwen3/modeling.rs:396-423, hunyuan_dense/modeling.rs:532-555
 *   KV-cache append .... qwen3/modeling.rs:313-370
 *   decode SDPA ........ qwen3/modeling.rs:432-467 (GQA-grouped, q pre-scaled)
 *   prefill SDPA ....... qwen3/modeling.rs:469-502 (expand K/V, post-scaled)
 *   causal mask ........ qwen3/modeling.rs:866-884 (-1e9), qwen2.rs:298-325 (-inf)
 *   batched decode ..... qwen3/modeling.rs:1118-1200 (right-aligned pad + mask)
 *
 * Numeric conventions.  All buffers are `float`.  With dtype = ORC_BF16 every
 * input holds a bf16-representable value and the output of every candle op is
 * rounded to bf16 (round-to-nearest-even, as half::bf16::from_f32 does);
 * element-wise bf16 arithmetic is an f32 operation followed by that rounding
 * (what half's operator impls do).  Reductions (matmul, softmax sum, RMS sum
 * of squares) accumulate in f32 in index order.  Compiled with
 * -ffp-contract=off so a*b-c*d is never fused, as rustc never fuses it.
 *
 * Which of these candle internals are bit-exact cannot be checked here
 * (candle is absent and there is no Rust toolchain); see the header of
 * oracle.c for which checks pin each function.
 */
#ifndef CRANE_ORACLE_H
#define CRANE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1 };
enum { ORC_NORM_THEN_ROPE = 0, ORC_ROPE_THEN_NORM = 1, ORC_ROPE_ONLY = 2 };
enum { ORC_DECODE_GROUPED = 0, ORC_DECODE_STANDARD = 1 };
enum { ORC_MASK_NEG_1E9 = 0, ORC_MASK_NEG_INF = 1 };

/* Round every element to bf16 (RNE) in place. */
void orc_round_bf16(float* x, size_t n);

/* SplitMix64 -> Box-Muller normal generator.  Writes n samples of N(mean, std^2)
 * as float.  Deterministic for a given seed on every platform. */
void orc_gen_normal(uint64_t seed, size_t n, double mean, double std, float* out);
/* Uniform integers in [lo, hi] (inclusive) from SplitMix64. */
void orc_gen_uniform_int(uint64_t seed, size_t n, int lo, int hi, int32_t* out);

/* A1 / A1h: f32 cos/sin tables [max_pos, dim/2].  alpha <= 0 means no NTK scaling. */
void orc_rope_tables(int dim, double theta, double alpha, int max_pos, float* cos_out, float* sin_out);
/* A1q: candle-transformers qwen2 tables built in the model dtype. */
void orc_rope_tables_qwen2(int dim, double theta, int max_pos, int dtype, float* cos_out, float* sin_out);

/* A5: candle_nn::RmsNorm over rows of length d.  contiguous selects the fused
 * ops::rms_norm path (true for a contiguous input) or the LayerNorm fallback. */
void orc_rms_norm(const float* x, float* y, size_t rows, int d, const float* w, float eps,
                  int contiguous, int dtype);
/* The decoder layer's row ops.  Crane's fused SiLU(gate) * up over
 * gate_up [rows, 2*inter] (gate || up): f64 = 0 is the f32 formula of its CUDA
 * kernel, f64 = 1 its cpu_fwd (f64, one conversion to T). */
void orc_silu_mul(const float* gate_up, float* out, size_t rows, int inter, int f64, int dtype);
/* candle's `residual + hidden` in T, in place. */
void orc_residual_add(float* residual, const float* hidden, size_t n, int dtype);
/* candle Linear: y[M,N] = T(T(x[M,K] w[N,K]^T) + bias[N]) (bias may be NULL);
 * the product is accumulated in f64 and converted to T once.  fused = 1:
 * T(x w^T + bias) with one conversion (a GEMM epilogue's rounding). */
void orc_linear(const float* x, const float* w, const float* bias, float* y, int M, int N, int K, int fused,
                int dtype);

/* Sampling (crane_sampling.h order: value descending, index ascending, NaN
 * lowest, -0 == +0): the first maximum per row, and the first k per row. */
void orc_argmax(const float* x, size_t rows, size_t n, uint32_t* out);
void orc_topk(const float* x, size_t rows, size_t n, int k, uint32_t* out);

/* A6: candle_nn::rotary_emb::rope on rows of length d, row r using table row pos[r]. */
void orc_rope(const float* x, float* y, size_t rows, int d, const float* cos, const float* sin,
              const int32_t* pos, int dtype);

/* A3-A7: the merged qkv row [B,S,(Hq+2Hkv)*D] -> q_out [B,Hq,S,D] and cache rows
 * [B,Hkv,cap,D] at [cache_len[b], cache_len[b]+S).  cos/sin are the model-dtype
 * tables [max_pos, D/2]; token s of sequence b uses row positions[b]+s.
 * q_w / k_w may be NULL (weight 1).  Returns 0, or -1 on capacity overflow. */
int orc_qk_norm_rope_append(const float* qkv, int B, int S, int Hq, int Hkv, int D,
                            const float* q_w, const float* k_w, float eps, int order,
                            const float* cos, const float* sin, const int32_t* positions,
                            float* q_out, float* k_cache, float* v_cache, int cap,
                            const int32_t* cache_len, int dtype);

/* A8: decode SDPA over each sequence's own kv_len[b] cache rows.
 * q [B,Hq,D]; caches [B,Hkv,cap,D]; out [B,Hq*D].  variant selects the
 * GQA-grouped path (q pre-scaled) or the standard path (scores post-scaled). */
void orc_attn_decode(const float* q, const float* k_cache, const float* v_cache, int cap,
                     const int32_t* kv_len, int B, int Hq, int Hkv, int D, float scale,
                     float* out, int dtype, int variant, int nthreads);

/* A11: the reference's batched decode: right-aligned padding to max_kv columns
 * plus the -1e9 mask on [0, max_kv - kv_len[b]).  Same arguments as
 * orc_attn_decode; used to show padding+mask equals the varlen form. */
void orc_attn_decode_padded(const float* q, const float* k_cache, const float* v_cache, int cap,
                            const int32_t* kv_len, int B, int Hq, int Hkv, int D, float scale,
                            float* out, int dtype, int nthreads);

/* A9/A10: prefill SDPA.  q [B,Hq,S,D]; caches [B,Hkv,cap,D] hold rows
 * [0, start[b]+S); out [B,S,Hq*D].  causal adds the mask (j > start+i masked).
 * row_lo/row_hi restrict the computed query rows (for bounded samples);
 * pass 0 and S for the full problem.  head_lo/head_hi restrict q heads. */
void orc_attn_prefill(const float* q, const float* k_cache, const float* v_cache, int cap,
                      const int32_t* start, int B, int S, int Hq, int Hkv, int D, float scale,
                      int causal, float* out, int dtype, int mask_kind,
                      int row_lo, int row_hi, int head_lo, int head_hi, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
