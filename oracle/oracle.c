/*
 * oracle.c -- CPU restatement of Crane's candle-CPU attention op chain.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the thing
 * measured or shipped.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * What pins each function (tests/test_oracle.py):
 *   orc_rope_tables ........ closed form in float64 (<= 1 ulp of f32 from the
 *                            f64 value of the same f32 argument), identity row 0,
 *                            and orc_rope_tables_qwen2 in f32 equal to it bit-for-bit
 *   orc_rope_tables_qwen2 .. f32 mode == orc_rope_tables; bf16 mode: positions
 *                            above 256 rounded (checked against the closed form)
 *   orc_rms_norm ........... float64 textbook formula; scale equivariance; RMS of
 *                            the output == 1 - O(eps); transformers Qwen3RMSNorm
 *   orc_rope ............... transformers apply_rotary_pos_emb / rotate_half on the
 *                            same tables; pair-norm preservation; identity at pos 0;
 *                            composition R(p1)R(p2) = R(p1+p2) in float64
 *   orc_qk_norm_rope_append  composition of the two above for all three orders;
 *                            cache rows outside [len, len+S) untouched (canary)
 *   orc_attn_decode ........ float64 brute force softmax(qK^T*scale)V; torch SDPA
 *                            (enable_gqa); equal keys => mean of V; one dominant
 *                            key => its V row; equals the last row of prefill
 *   orc_attn_decode_padded . equals orc_attn_decode (padding + -1e9 == varlen)
 *   orc_attn_prefill ....... float64 brute force; torch SDPA is_causal; causal row 0
 *                            => V[0]; -1e9 and -inf masks give identical f32 output
 * Bit-level agreement with candle's bf16 rounding points (rope per-op rounding,
 * rms_norm path, softmax and gemm accumulation) cannot be checked without candle:
 * those rounding points follow candle 0.10.2 as read from its public source and
 * are "parity unpinned" at the last bit; the tolerances absorb them.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- bf16 -- */

static inline float bf16r(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {      /* inf / nan */
        if (u & 0x007fffffu) u |= 0x00400000u;   /* quiet nan, keep sign */
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);         /* round to nearest even */
        u &= 0xffff0000u;
    }
    float y;
    memcpy(&y, &u, 4);
    return y;
}

/* Round to the op's dtype: identity for f32, bf16 RNE otherwise. */
static inline float rd(float x, int dtype) { return dtype == ORC_BF16 ? bf16r(x) : x; }

void orc_round_bf16(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = bf16r(x[i]);
}

/* ------------------------------------------------------------ generator -- */

static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Uniform double in (0, 1]. */
static inline double unit_open0(uint64_t* s) {
    return (double)((splitmix64(s) >> 11) + 1) * (1.0 / 9007199254740992.0);
}

void orc_gen_normal(uint64_t seed, size_t n, double mean, double std, float* out) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        double u1 = unit_open0(&s), u2 = unit_open0(&s);
        double r = sqrt(-2.0 * log(u1));
        out[i++] = (float)(mean + std * r * cos(two_pi * u2));
        if (i < n) out[i++] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

void orc_gen_uniform_int(uint64_t seed, size_t n, int lo, int hi, int32_t* out) {
    uint64_t s = seed;
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; ++i) out[i] = (int32_t)((int64_t)lo + (int64_t)(splitmix64(&s) % span));
}

/* ----------------------------------------------------------- rope tables -- */

/* qwen3/modeling.rs:117-139 and hunyuan_dense/modeling.rs:196-231:
 * inv[k] = 1.0f32 / (f32)(base^(2k/dim)) with the pow in f64; freqs = p * inv
 * in f32 (a k=1 matmul: one rounding); cos/sin by libm cosf/sinf (what Rust's
 * f32::cos/sin call on Linux).  Hunyuan's NTK alpha raises the base to
 * theta * alpha^(dim/(dim-2)) in f64 (hunyuan_dense/modeling.rs:205). */
void orc_rope_tables(int dim, double theta, double alpha, int max_pos, float* cos_out, float* sin_out) {
    int half = dim / 2;
    double base = theta;
    if (alpha > 0.0) base = theta * pow(alpha, (double)dim / ((double)dim - 2.0));
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    for (int k = 0; k < half; ++k) inv[k] = 1.0f / (float)pow(base, (double)(2 * k) / (double)dim);
    for (int p = 0; p < max_pos; ++p) {
        for (int k = 0; k < half; ++k) {
            float f = (float)p * inv[k];
            cos_out[(size_t)p * half + k] = cosf(f);
            sin_out[(size_t)p * half + k] = sinf(f);
        }
    }
    free(inv);
}

/* qwen25/qwen2.rs:47-64 (copy of candle-transformers qwen2): inv_freq and the
 * u32 positions are cast to the model dtype before the k=1 matmul, whose
 * product is rounded to that dtype, and sin/cos are bf16 unary ops (f32 libm
 * then rounding). */
void orc_rope_tables_qwen2(int dim, double theta, int max_pos, int dtype, float* cos_out, float* sin_out) {
    int half = dim / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    for (int k = 0; k < half; ++k) inv[k] = rd(1.0f / (float)pow(theta, (double)(2 * k) / (double)dim), dtype);
    for (int p = 0; p < max_pos; ++p) {
        float pp = rd((float)(uint32_t)p, dtype);
        for (int k = 0; k < half; ++k) {
            float f = rd(pp * inv[k], dtype);
            cos_out[(size_t)p * half + k] = rd(cosf(f), dtype);
            sin_out[(size_t)p * half + k] = rd(sinf(f), dtype);
        }
    }
    free(inv);
}

/* -------------------------------------------------------------- RmsNorm -- */

static void rms_norm_row(const float* x, float* y, int d, const float* w, float eps, int contiguous, int dtype) {
    if (contiguous) {
        /* candle-nn ops::rms_norm (fused CustomOp2, cpu_fwd): f32 sum of squares,
         * m = sqrt(sum2/d + eps) converted to T, y = x / m * alpha in T. */
        float sum2 = 0.0f;
        for (int i = 0; i < d; ++i) sum2 += x[i] * x[i];
        float m = rd(sqrtf(sum2 / (float)d + eps), dtype);
        for (int i = 0; i < d; ++i) {
            float wi = w ? w[i] : 1.0f;
            y[i] = rd(rd(x[i] / m, dtype) * wi, dtype);
        }
    } else {
        /* candle-nn LayerNorm::forward with remove_mean = false (the RmsNorm
         * fallback for a non-contiguous input): f32 internally,
         * x / sqrt(sum(x^2) * (1/d) + eps), cast to T, then * weight in T. */
        float sum2 = 0.0f;
        for (int i = 0; i < d; ++i) sum2 += x[i] * x[i];
        float denom = sqrtf(sum2 * (float)(1.0 / (double)d) + eps);
        for (int i = 0; i < d; ++i) {
            float wi = w ? w[i] : 1.0f;
            y[i] = rd(rd(x[i] / denom, dtype) * wi, dtype);
        }
    }
}

void orc_rms_norm(const float* x, float* y, size_t rows, int d, const float* w, float eps,
                  int contiguous, int dtype) {
    for (size_t r = 0; r < rows; ++r) rms_norm_row(x + r * d, y + r * d, d, w, eps, contiguous, dtype);
}

/* ----------------------------------------------------------------- rope -- */

/* candle_nn::rotary_emb::rope (non-interleaved, "rotate half"), cpu_fwd in T:
 *   y[i]     = x[i]*c - x[i+d/2]*s
 *   y[i+d/2] = x[i]*s + x[i+d/2]*c          (each product and sum rounded in T) */
static void rope_row(const float* x, float* y, int d, const float* c, const float* s, int dtype) {
    int h = d / 2;
    for (int i = 0; i < h; ++i) {
        float x1 = x[i], x2 = x[i + h];
        float a = rd(x1 * c[i], dtype), b = rd(x2 * s[i], dtype);
        float e = rd(x1 * s[i], dtype), f = rd(x2 * c[i], dtype);
        y[i] = rd(a - b, dtype);
        y[i + h] = rd(e + f, dtype);
    }
}

void orc_rope(const float* x, float* y, size_t rows, int d, const float* cos, const float* sin,
              const int32_t* pos, int dtype) {
    for (size_t r = 0; r < rows; ++r)
        rope_row(x + r * d, y + r * d, d, cos + (size_t)pos[r] * (d / 2), sin + (size_t)pos[r] * (d / 2), dtype);
}

/* -------------------------------------------------- fused append (A3-A7) -- */

/* One head row through Crane's per-head op order:
 *   Qwen3   (qwen3/modeling.rs:410-423):        rope(rms_norm(x))
 *   Hunyuan (hunyuan_dense/modeling.rs:541-555): rms_norm(rope(x))
 *   Qwen2.5 (qwen2.rs:75-76):                   rope(x)
 * In Qwen3 the norm sees the transposed [B,H,S,D] view, which is contiguous
 * only when S == 1; Hunyuan norms the contiguous rope output. */
static void head_chain(const float* x, float* y, int D, const float* w, float eps, int order,
                       const float* c, const float* s, int S, int dtype, float* tmp) {
    switch (order) {
    case ORC_NORM_THEN_ROPE:
        rms_norm_row(x, tmp, D, w, eps, S == 1, dtype);
        rope_row(tmp, y, D, c, s, dtype);
        break;
    case ORC_ROPE_THEN_NORM:
        rope_row(x, tmp, D, c, s, dtype);
        rms_norm_row(tmp, y, D, w, eps, 1, dtype);
        break;
    default:
        rope_row(x, y, D, c, s, dtype);
        break;
    }
}

int orc_qk_norm_rope_append(const float* qkv, int B, int S, int Hq, int Hkv, int D,
                            const float* q_w, const float* k_w, float eps, int order,
                            const float* cos, const float* sin, const int32_t* positions,
                            float* q_out, float* k_cache, float* v_cache, int cap,
                            const int32_t* cache_len, int dtype) {
    const size_t W = (size_t)(Hq + 2 * Hkv) * D;
    const int half = D / 2;
    for (int b = 0; b < B; ++b)
        if (cache_len[b] < 0 || cache_len[b] + S > cap) return -1;
    float* tmp = (float*)malloc(sizeof(float) * (size_t)D);
    for (int b = 0; b < B; ++b) {
        for (int s = 0; s < S; ++s) {
            const float* row = qkv + ((size_t)b * S + s) * W;
            const int p = positions[b] + s;
            const float* c = cos + (size_t)p * half;
            const float* sn = sin + (size_t)p * half;
            for (int h = 0; h < Hq; ++h) {
                float* dst = q_out + (((size_t)b * Hq + h) * S + s) * D;
                head_chain(row + (size_t)h * D, dst, D, q_w, eps, order, c, sn, S, dtype, tmp);
            }
            const size_t r = (size_t)cache_len[b] + s;
            for (int h = 0; h < Hkv; ++h) {
                float* kd = k_cache + (((size_t)b * Hkv + h) * cap + r) * D;
                float* vd = v_cache + (((size_t)b * Hkv + h) * cap + r) * D;
                head_chain(row + (size_t)(Hq + h) * D, kd, D, k_w, eps, order, c, sn, S, dtype, tmp);
                memcpy(vd, row + (size_t)(Hq + Hkv + h) * D, sizeof(float) * (size_t)D);
            }
        }
    }
    free(tmp);
    return 0;
}

/* ------------------------------------------------------- softmax (A8/A9) -- */

/* candle-nn ops::softmax_last_dim, cpu_fwd in T: max in T, e = exp(s - max)
 * with the subtraction and the exp rounded to T, sum of e accumulated in f32
 * then converted to T (vec_reduce_sum), p = e / sum in T. */
static void softmax_row(float* s, int n, int dtype) {
    float mx = -INFINITY;
    for (int j = 0; j < n; ++j) mx = s[j] > mx ? s[j] : mx;
    float sum = 0.0f;
    for (int j = 0; j < n; ++j) {
        s[j] = rd(expf(rd(s[j] - mx, dtype)), dtype);
        sum += s[j];
    }
    sum = rd(sum, dtype);
    for (int j = 0; j < n; ++j) s[j] = rd(s[j] / sum, dtype);
}

/* ---------------------------------------------------------- decode (A8) -- */

static void decode_head(const float* qh, const float* K, const float* V, int L, int D, float scale,
                        float* o, int dtype, int variant, float* sc, float* qs) {
    /* Grouped path (qwen3/modeling.rs:440-457): q_g = q * scale via affine in T
     * (scale converted to T first), scores = q_g @ K^T.  Standard path
     * (qwen2.rs:196-201, qwen3 n_rep == 1): scores = (q @ K^T) * scale. */
    const float sc_t = rd(scale, dtype);
    for (int d = 0; d < D; ++d) qs[d] = variant == ORC_DECODE_GROUPED ? rd(qh[d] * sc_t, dtype) : qh[d];
    for (int j = 0; j < L; ++j) {
        const float* k = K + (size_t)j * D;
        float acc = 0.0f;
        for (int d = 0; d < D; ++d) acc += qs[d] * k[d];
        acc = rd(acc, dtype);
        if (variant != ORC_DECODE_GROUPED) acc = rd(acc * sc_t, dtype);
        sc[j] = acc;
    }
    softmax_row(sc, L, dtype);
    for (int d = 0; d < D; ++d) o[d] = 0.0f;
    for (int j = 0; j < L; ++j) {
        const float* v = V + (size_t)j * D;
        const float p = sc[j];
        for (int d = 0; d < D; ++d) o[d] += p * v[d];
    }
    for (int d = 0; d < D; ++d) o[d] = rd(o[d], dtype);
}

void orc_attn_decode(const float* q, const float* k_cache, const float* v_cache, int cap,
                     const int32_t* kv_len, int B, int Hq, int Hkv, int D, float scale,
                     float* out, int dtype, int variant, int nthreads) {
    const int n_rep = Hq / Hkv;
    int maxL = 0;
    for (int b = 0; b < B; ++b) maxL = kv_len[b] > maxL ? kv_len[b] : maxL;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)(maxL > 0 ? maxL : 1));
        float* qs = (float*)malloc(sizeof(float) * (size_t)D);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int bh = 0; bh < B * Hq; ++bh) {
            const int b = bh / Hq, h = bh % Hq, g = h / n_rep;
            const float* K = k_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            const float* V = v_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            decode_head(q + (size_t)bh * D, K, V, kv_len[b], D, scale, out + (size_t)bh * D, dtype, variant, sc, qs);
        }
        free(sc);
        free(qs);
    }
}

/* qwen3/modeling.rs:1141-1200 (pad_and_stack_kv_caches) and 1118-1138
 * (build_batch_decode_mask): every sequence is right-aligned into max_kv
 * columns with zero rows in front, and -1e9 (in T) is added on the padding
 * columns before softmax_last_dim.  The decode SDPA is the grouped path. */
void orc_attn_decode_padded(const float* q, const float* k_cache, const float* v_cache, int cap,
                            const int32_t* kv_len, int B, int Hq, int Hkv, int D, float scale,
                            float* out, int dtype, int nthreads) {
    const int n_rep = Hq / Hkv;
    int W = 0;
    for (int b = 0; b < B; ++b) W = kv_len[b] > W ? kv_len[b] : W;
    const float mval = rd(-1e9f, dtype);
    int all_equal = 1;
    for (int b = 0; b < B; ++b) all_equal &= (kv_len[b] == W);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)(W > 0 ? W : 1));
        float* qs = (float*)malloc(sizeof(float) * (size_t)D);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int bh = 0; bh < B * Hq; ++bh) {
            const int b = bh / Hq, h = bh % Hq, g = h / n_rep;
            const int pad = W - kv_len[b];
            const float* K = k_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            const float* V = v_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            const float sc_t = rd(scale, dtype);
            for (int d = 0; d < D; ++d) qs[d] = rd(q[(size_t)bh * D + d] * sc_t, dtype);
            for (int j = 0; j < W; ++j) {
                float acc = 0.0f;
                if (j >= pad) {
                    const float* k = K + (size_t)(j - pad) * D;
                    for (int d = 0; d < D; ++d) acc += qs[d] * k[d];
                } /* a zero pad row scores exactly 0 */
                acc = rd(acc, dtype);
                /* the mask is None when every length equals max_kv (:1125-1127) */
                if (!all_equal) acc = rd(acc + (j < pad ? mval : -0.0f), dtype);
                sc[j] = acc;
            }
            softmax_row(sc, W, dtype);
            float* o = out + (size_t)bh * D;
            for (int d = 0; d < D; ++d) o[d] = 0.0f;
            for (int j = 0; j < W; ++j) {
                const float p = sc[j];
                if (j < pad) {               /* zero rows contribute p * 0 */
                    for (int d = 0; d < D; ++d) o[d] += p * 0.0f;
                    continue;
                }
                const float* v = V + (size_t)(j - pad) * D;
                for (int d = 0; d < D; ++d) o[d] += p * v[d];
            }
            for (int d = 0; d < D; ++d) o[d] = rd(o[d], dtype);
        }
        free(sc);
        free(qs);
    }
}

/* --------------------------------------------------------- prefill (A9) -- */

/* qwen3/modeling.rs:469-502 (and hunyuan_dense 610-645, qwen2.rs 191-211):
 * K/V expanded to Hq heads (head h reads kv head h / n_rep), scores =
 * (q @ K^T) rounded to T then * scale in T, + mask in T, softmax_last_dim,
 * @ V, transposed to [B,S,Hq*D].  The mask (qwen3/modeling.rs:866-884) is
 * (allowed ? 0 : 1) * -1e9 in T; qwen2.rs:298-325 uses 0 / -inf.  The full
 * score row over all start+S keys is materialised, masked columns included,
 * as candle does. */
void orc_attn_prefill(const float* q, const float* k_cache, const float* v_cache, int cap,
                      const int32_t* start, int B, int S, int Hq, int Hkv, int D, float scale,
                      int causal, float* out, int dtype, int mask_kind,
                      int row_lo, int row_hi, int head_lo, int head_hi, int nthreads) {
    const int n_rep = Hq / Hkv;
    int maxL = 0;
    for (int b = 0; b < B; ++b) maxL = start[b] + S > maxL ? start[b] + S : maxL;
    if (row_lo < 0) row_lo = 0;
    if (row_hi > S) row_hi = S;
    if (head_lo < 0) head_lo = 0;
    if (head_hi > Hq) head_hi = Hq;
    const int nrows = row_hi - row_lo, nheads = head_hi - head_lo;
    if (nrows <= 0 || nheads <= 0) return;
    const float sc_t = rd(scale, dtype);
    const float mval = mask_kind == ORC_MASK_NEG_INF ? -INFINITY : rd(-1e9f, dtype);
    const long total = (long)B * nheads * nrows;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)(maxL > 0 ? maxL : 1));
        float* o = (float*)malloc(sizeof(float) * (size_t)D);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (long t = 0; t < total; ++t) {
            const int b = (int)(t / ((long)nheads * nrows));
            const int h = head_lo + (int)((t / nrows) % nheads);
            const int i = row_lo + (int)(t % nrows);
            const int g = h / n_rep;
            const int L = start[b] + S;
            const float* qi = q + (((size_t)b * Hq + h) * S + i) * D;
            const float* K = k_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            const float* V = v_cache + ((size_t)b * Hkv + g) * (size_t)cap * D;
            for (int j = 0; j < L; ++j) {
                const float* k = K + (size_t)j * D;
                float acc = 0.0f;
                for (int d = 0; d < D; ++d) acc += qi[d] * k[d];
                acc = rd(rd(acc, dtype) * sc_t, dtype);
                if (causal) {
                    const int masked = j > start[b] + i;
                    if (mask_kind == ORC_MASK_NEG_INF) acc = masked ? -INFINITY : acc;
                    else acc = rd(acc + (masked ? mval : -0.0f), dtype);
                }
                sc[j] = acc;
            }
            softmax_row(sc, L, dtype);
            for (int d = 0; d < D; ++d) o[d] = 0.0f;
            for (int j = 0; j < L; ++j) {
                const float* v = V + (size_t)j * D;
                const float p = sc[j];
                for (int d = 0; d < D; ++d) o[d] += p * v[d];
            }
            float* dst = out + (((size_t)b * S + i) * Hq + h) * D;
            for (int d = 0; d < D; ++d) dst[d] = rd(o[d], dtype);
        }
        free(sc);
        free(o);
    }
}

/* ------------------------------------------------- layer row operations -- */

/* f64 -> bf16 with one round-to-nearest-even, as half::bf16::from_f64 (no
 * intermediate f32 rounding).  Finite inputs in f32 range. */
static float bf16_from_double(double x) {
    if (x == 0.0 || !isfinite(x)) return (float)x;
    int e;
    frexp(x, &e);                               /* |x| in [2^(e-1), 2^e) */
    if (e - 1 < -126) e = -126 + 1;             /* bf16 subnormals share f32's exponent floor */
    const double ulp = ldexp(1.0, e - 1 - 7);   /* 8 significant bits */
    return (float)(rint(x / ulp) * ulp);        /* x / ulp is exact; rint rounds to even */
}

void orc_silu_mul(const float* gate_up, float* out, size_t rows, int inter, int f64, int dtype) {
    for (size_t r = 0; r < rows; ++r) {
        const float* g = gate_up + r * 2 * (size_t)inter;
        const float* u = g + inter;
        float* o = out + r * (size_t)inter;
        for (int i = 0; i < inter; ++i) {
            if (f64) {
                /* FusedSiluMul::cpu_fwd (cuda_impl.rs:65-76): f64 silu and product,
                 * one conversion to T. */
                const double gd = g[i];
                const double s = gd / (1.0 + exp(-gd));
                o[i] = dtype == ORC_BF16 ? bf16_from_double(s * (double)u[i]) : (float)(s * (double)u[i]);
            } else {
                /* fused_silu_mul_{bf16,f32} (fused_ops.cu:104-126, 163-182):
                 * f32 g / (1 + expf(-g)) * u, one conversion to T. */
                const float s = g[i] / (1.0f + expf(-g[i]));
                o[i] = rd(s * u[i], dtype);
            }
        }
    }
}

void orc_residual_add(float* residual, const float* hidden, size_t n, int dtype) {
    for (size_t i = 0; i < n; ++i) residual[i] = rd(residual[i] + hidden[i], dtype);
}

/* candle Linear::forward (x.matmul(w.t()) then broadcast_add(bias), the merged
 * qkv_proj of qwen3/modeling.rs:382-387 and o_proj): the product accumulated
 * in f64 and converted to T once, then the bias added in T.  fused = 1 rounds
 * product + bias once instead (a GEMM epilogue's semantics). */
void orc_linear(const float* x, const float* w, const float* bias, float* y, int M, int N, int K, int fused,
                int dtype) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const float* xr = x + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const float* wr = w + (size_t)n * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
            float p;
            if (bias && fused) {
                acc += (double)bias[n];
                p = dtype == ORC_BF16 ? bf16_from_double(acc) : (float)acc;
            } else {
                p = dtype == ORC_BF16 ? bf16_from_double(acc) : (float)acc;
                if (bias) p = rd(p + bias[n], dtype);
            }
            y[(size_t)m * N + n] = p;
        }
    }
}

/* --------------------------------------------------------------- sampling -- */

/* Order of crane_sampling.h: value descending, then index ascending; NaN
 * below every number, -0 equal to +0. */
static inline uint32_t order_key(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static int before(float a, uint32_t ia, float b, uint32_t ib) {
    const uint32_t ka = order_key(a), kb = order_key(b);
    return ka != kb ? ka > kb : ia < ib;
}

/* gpu_argmax / candle argmax (first maximum) per row. */
void orc_argmax(const float* x, size_t rows, size_t n, uint32_t* out) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * n;
        uint32_t best = 0;
        for (size_t i = 1; i < n; ++i)
            if (before(xr[i], (uint32_t)i, xr[best], best)) best = (uint32_t)i;
        out[r] = best;
    }
}

/* topk_indices per row: the first k elements in that order (a full sort of
 * (key, index) pairs, k <= 64). */
typedef struct {
    uint32_t key, idx;
} orc_pair;

static int pair_cmp(const void* a, const void* b) {
    const orc_pair* p = (const orc_pair*)a;
    const orc_pair* q = (const orc_pair*)b;
    if (p->key != q->key) return p->key > q->key ? -1 : 1;
    return p->idx < q->idx ? -1 : (p->idx > q->idx ? 1 : 0);
}

void orc_topk(const float* x, size_t rows, size_t n, int k, uint32_t* out) {
    orc_pair* pairs = (orc_pair*)malloc(n * sizeof(orc_pair));
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * n;
        for (size_t i = 0; i < n; ++i) {
            pairs[i].key = order_key(xr[i]);
            pairs[i].idx = (uint32_t)i;
        }
        qsort(pairs, n, sizeof(orc_pair), pair_cmp);
        for (int j = 0; j < k; ++j) out[r * k + j] = pairs[j].idx;
    }
    free(pairs);
}
