// append.hip -- fused per-head QK-RMSNorm + RoPE + KV-cache append (gfx950).
//
// One pass over Crane's merged qkv rows replaces, per layer,
//   qwen3/modeling.rs:382-404  qkv narrow + reshape/transpose(+contiguous copies)
//   qwen3/modeling.rs:410-419  q_norm / k_norm (candle_nn::RmsNorm over D)
//   qwen3/modeling.rs:422-423  candle_nn::rotary_emb::rope on q and k (rotate-half)
//   qwen3/modeling.rs:313-332  update_kv_cache: slice_set of k and v at cache_seq_len
// with the Hunyuan order (rope, then norm: hunyuan_dense/modeling.rs:541-555) and
// the Qwen2.5 order (rope only: qwen2.rs:75-76) selected by `order`.
//
// Work item = one head row (128 elements) of one token: Hq query rows, Hkv key
// rows and Hkv value rows per token.  8 lanes own an item; lane l holds dims
// [8l, 8l+8) and their rotate-half partners [64+8l, 64+8l+8) as two 16-byte
// pieces, so the rotation is lane-local and the RMS sum is an 8-lane DPP
// butterfly.  The arithmetic is f32 with the result of every candle op
// rounded to the storage type, as Crane's candle op chain rounds it (the
// kernel is HBM-bound, so this is free).  Every cache row is written exactly
// once; q lands in [B,Hq,S,D] for the attention kernels.
// HBM traffic per token: (Hq+2Hkv)*D elements read, the same written.
#include "common.h"

namespace crane {
namespace {

constexpr int kItemsPerBlock = 32;  // 256 threads / 8 lanes per item

// Sum over the 8 lanes of a DPP half-row; every lane gets the total.
__device__ __forceinline__ float group8_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror
    return x;
}

// candle_nn RmsNorm over the 128 dims held by 8 lanes.  `contiguous` selects
// candle's fused ops::rms_norm (m = sqrt(mean(x^2)+eps) converted to T, then
// x / m * w in T) or the LayerNorm fallback used for a non-contiguous input
// (x / sqrt(mean(x^2)+eps) in f32, converted to T, then * w in T).  The sum of
// squares accumulates in f32.
// w1, w2: this lane's 16 weights (the caller loads them with the row).
template <typename T>
__device__ __forceinline__ void rms_norm8(float (&x1)[8], float (&x2)[8], const float (&w1)[8],
                                          const float (&w2)[8], float eps, bool contiguous) {
    // explicit FMAs: the sum's bits do not depend on how the compiler
    // contracts it in each instantiation of the kernel
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ss = __builtin_fmaf(x1[i], x1[i], ss);
        ss = __builtin_fmaf(x2[i], x2[i], ss);
    }
    ss = group8_sum(ss);
    float m = sqrtf(ss * (1.0f / kHeadDim) + eps);
    if (contiguous) m = rt<T>(m);
    // x / m from one reciprocal per row (div_by) when every row of the wave has
    // a normal, moderate m (m >= sqrt(eps) is never 0 for eps > 0); the
    // division otherwise (an infinite or NaN input, a zero eps)
    if (__all(m >= 0x1p-60f && m <= 0x1p60f)) {
        const float r = 1.0f / m;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x1[i] = rt<T>(rt<T>(div_by(x1[i], m, r)) * w1[i]);
            x2[i] = rt<T>(rt<T>(div_by(x2[i], m, r)) * w2[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x1[i] = rt<T>(rt<T>(x1[i] / m) * w1[i]);
            x2[i] = rt<T>(rt<T>(x2[i] / m) * w2[i]);
        }
    }
}

// candle_nn::rotary_emb::rope (rotate-half): every product and sum rounded in T.
template <typename T>
__device__ __forceinline__ void rope8(float (&x1)[8], float (&x2)[8], const float (&c)[8], const float (&s)[8]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = x1[i], b = x2[i];
        x1[i] = rt<T>(rt<T>(a * c[i]) - rt<T>(b * s[i]));
        x2[i] = rt<T>(rt<T>(a * s[i]) + rt<T>(b * c[i]));
    }
}

// Where a head row comes from.  QkvRows: the merged projection's output
// rows (row r at qkv + r * stride elements).  QkvParts: the f32 split-K
// partial products of that projection [NP][rows][n] (crane_gemm_linear_split),
// summed in split order, plus the bias when there is one, and rounded once
// to T -- the rounding point of the whole product's output.  Both put the
// lane's 16 values (dims 8 l.. and 64 + 8 l..) in x1, x2 and issue every load
// before the first use.
template <typename T>
struct QkvRows {
    const T* qkv;
    int64_t stride;
    __device__ __forceinline__ void load(int64_t tok, int head, int l, float (&x1)[8], float (&x2)[8]) const {
        const T* src = qkv + tok * stride + (int64_t)head * kHeadDim;
        load8(src + 8 * l, x1);
        load8(src + 64 + 8 * l, x2);
    }
};

template <typename T, int NP>
struct QkvParts {
    const float* parts;
    int64_t plane;  // elements per split: rows * n
    int64_t n;      // elements per row: (Hq + 2 Hkv) D
    const T* bias;  // [n] or null
    __device__ __forceinline__ void load(int64_t tok, int head, int l, float (&x1)[8], float (&x2)[8]) const {
        const float* src = parts + tok * n + (int64_t)head * kHeadDim;
        float p1[NP][8], p2[NP][8], b1[8], b2[8];
#pragma unroll
        for (int sp = 0; sp < NP; ++sp) {
            load8(src + sp * plane + 8 * l, p1[sp]);
            load8(src + sp * plane + 64 + 8 * l, p2[sp]);
        }
        if (bias) {
            load8(bias + (int64_t)head * kHeadDim + 8 * l, b1);
            load8(bias + (int64_t)head * kHeadDim + 64 + 8 * l, b2);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) b1[i] = b2[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float a = 0.f, c = 0.f;
#pragma unroll
            for (int sp = 0; sp < NP; ++sp) {
                a += p1[sp][i];
                c += p2[sp][i];
            }
            x1[i] = rt<T>(a + b1[i]);
            x2[i] = rt<T>(c + b2[i]);
        }
    }
};

template <typename T, class ROWS, class SRC>
__global__ __launch_bounds__(256) void qknorm_rope_append_kernel(
    SRC src_rows, const T* __restrict__ qw, const T* __restrict__ kw,
    float eps, int order, const T* __restrict__ cos_t, const T* __restrict__ sin_t, int64_t cs_stride,
    int64_t table_rows, const int32_t* __restrict__ positions, T* __restrict__ q_out, T* __restrict__ k_cache,
    T* __restrict__ v_cache, ROWS rows, const int32_t* __restrict__ cache_len, int S, int Hq, int Hkv,
    int64_t n_items) {
    const int64_t item = (int64_t)blockIdx.x * kItemsPerBlock + (threadIdx.x >> 3);
    const int l = threadIdx.x & 7;
    if (item >= n_items) return;  // whole 8-lane groups leave together
    const int H = Hq + 2 * Hkv;
    const int head = (int)(item % H);
    const int64_t tok = item / H;
    const int s = (int)(tok % S);
    const int b = (int)(tok / S);

    const bool is_q = head < Hq, is_v = head >= Hq + Hkv;
    // Every load that does not wait on another is issued first: the row, the
    // lengths and the norm weights; only the cos / sin rows wait on the
    // position.  Only k and v heads read cache_len, which the q-only entry
    // point (crane_hip_qnorm_rope) does not pass: q heads read positions in
    // its place (a load with no branch around it, so nothing waits for it).
    const int32_t cl_raw = (is_q ? positions : cache_len)[b];
    const int32_t cl = is_q ? 0 : cl_raw;
    const int32_t pb = positions[b];
    float x1[8], x2[8];
    src_rows.load(tok, head, l, x1, x2);
    const T* w = is_q ? qw : kw;
    float w1[8], w2[8];
    if (!is_v && w) {
        load8(w + 8 * l, w1);
        load8(w + 64 + 8 * l, w2);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w1[i] = w2[i] = 1.f;
    }

    if (is_v) {  // value row: straight into the cache
        const int64_t off = rows.offset(b, Hkv, head - Hq - Hkv, (int64_t)cl + s);
        if (off < 0) return;  // past the capacity (or on an invalid page): not written
        T* dst = v_cache + off;
        store8(dst + 8 * l, x1);
        store8(dst + 64 + 8 * l, x2);
        return;
    }
    T* dst;
    if (is_q) {
        dst = q_out + (((int64_t)b * Hq + head) * S + s) * kHeadDim;
    } else {
        const int64_t off = rows.offset(b, Hkv, head - Hq, (int64_t)cl + s);
        if (off < 0) return;
        dst = k_cache + off;
    }
    const int64_t p = (int64_t)pb + s;
    if (p < 0 || p >= table_rows) return;  // no table row for this position: nothing is written
    float c[8], sn[8];
    load8(cos_t + p * cs_stride + 8 * l, c);
    load8(sin_t + p * cs_stride + 8 * l, sn);

    // Qwen3 norms the transposed [B,H,S,D] view, contiguous only when S == 1;
    // Hunyuan norms the contiguous rope output.
    if (order == CRANE_HIP_NORM_THEN_ROPE) rms_norm8<T>(x1, x2, w1, w2, eps, S == 1);
    rope8<T>(x1, x2, c, sn);
    if (order == CRANE_HIP_ROPE_THEN_NORM) rms_norm8<T>(x1, x2, w1, w2, eps, true);

    store8(dst + 8 * l, x1);
    store8(dst + 64 + 8 * l, x2);
}

// The rows an append reads: the projection's output rows (qkv, row stride
// in elements) or its f32 split-K partial products (parts [n_parts][B S][n],
// n_parts 2 or 4, and the projection's bias or null).
struct RowSource {
    const void* qkv = nullptr;
    int64_t stride = 0;
    const float* parts = nullptr;
    int n_parts = 0;
    const void* bias = nullptr;
};

template <typename T, class ROWS, class SRC>
void launch_append(const SRC& src, int64_t blocks, const void* q_norm_w, const void* k_norm_w, float eps, int order,
                   const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows, const int32_t* positions,
                   void* q_out, void* k_cache, void* v_cache, const ROWS& rows, const int32_t* cache_len, int S, int Hq,
                   int Hkv, int64_t n_items, hipStream_t st) {
    hipLaunchKernelGGL((qknorm_rope_append_kernel<T, ROWS, SRC>), dim3((unsigned)blocks), dim3(256), 0, st, src,
                       (const T*)q_norm_w, (const T*)k_norm_w, eps, order, (const T*)cos, (const T*)sin, cs_stride,
                       table_rows, positions, (T*)q_out, (T*)k_cache, (T*)v_cache, rows, cache_len, S, Hq, Hkv,
                       n_items);
}

template <typename T, class ROWS>
void launch_append_src(const RowSource& src, int64_t blocks, const void* q_norm_w, const void* k_norm_w, float eps,
                       int order, const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                       const int32_t* positions, void* q_out, void* k_cache, void* v_cache, const ROWS& rows,
                       const int32_t* cache_len, int B, int S, int Hq, int Hkv, int64_t n_items, hipStream_t st) {
    const int64_t n = (int64_t)(Hq + 2 * Hkv) * kHeadDim;
    if (!src.parts) {
        const QkvRows<T> r{(const T*)src.qkv, src.stride};
        launch_append<T>(r, blocks, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows, positions, q_out,
                         k_cache, v_cache, rows, cache_len, S, Hq, Hkv, n_items, st);
    } else if (src.n_parts == 2) {
        const QkvParts<T, 2> r{src.parts, (int64_t)B * S * n, n, (const T*)src.bias};
        launch_append<T>(r, blocks, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows, positions, q_out,
                         k_cache, v_cache, rows, cache_len, S, Hq, Hkv, n_items, st);
    } else {
        const QkvParts<T, 4> r{src.parts, (int64_t)B * S * n, n, (const T*)src.bias};
        launch_append<T>(r, blocks, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows, positions, q_out,
                         k_cache, v_cache, rows, cache_len, S, Hq, Hkv, n_items, st);
    }
}

// Checks shared by both layouts and both row sources, then the launch; `rows`
// addresses the cache.
template <class ROWS>
int qknorm_rope_append(const RowSource& src, const void* q_norm_w, const void* k_norm_w, float eps, int order,
                       const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                       const int32_t* positions, void* q_out, void* k_cache, void* v_cache, const ROWS& rows,
                       const int32_t* cache_len, int B, int S, int Hq, int Hkv, int D, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || S < 0 || Hq <= 0 || Hkv <= 0) return CRANE_HIP_E_INVALID;
    if (Hq % Hkv != 0) return CRANE_HIP_E_GQA;
    if (order < CRANE_HIP_NORM_THEN_ROPE || order > CRANE_HIP_ROPE_ONLY) return CRANE_HIP_E_INVALID;
    if (!(eps >= 0.0f)) return CRANE_HIP_E_INVALID;
    if (src.parts && src.n_parts != 2 && src.n_parts != 4) return CRANE_HIP_E_INVALID;
    if (B == 0 || S == 0) return CRANE_HIP_OK;
    if ((!src.parts && !src.qkv) || !cos || !sin || !positions || !q_out || !k_cache || !v_cache || !cache_len)
        return CRANE_HIP_E_INVALID;
    if (cs_stride < D / 2 || table_rows <= 0) return CRANE_HIP_E_INVALID;
    if (!src.parts && src.stride < (int64_t)(Hq + 2 * Hkv) * D) return CRANE_HIP_E_INVALID;
    const int64_t per16 = dtype == CRANE_HIP_BF16 ? 8 : 4;  // elements per 16 bytes
    if ((!src.parts && src.stride % per16 != 0) || cs_stride % per16 != 0) return CRANE_HIP_E_ALIGN;
    if (!aligned16(src.parts ? (const void*)src.parts : src.qkv) || (src.bias && !aligned16(src.bias)) ||
        !aligned16(cos) || !aligned16(sin) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
        (q_norm_w && !aligned16(q_norm_w)) || (k_norm_w && !aligned16(k_norm_w)))
        return CRANE_HIP_E_ALIGN;

    const int64_t n_items = (int64_t)B * S * (Hq + 2 * Hkv);
    const int64_t blocks = (n_items + kItemsPerBlock - 1) / kItemsPerBlock;
    if (blocks > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        launch_append_src<float>(src, blocks, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows,
                                 positions, q_out, k_cache, v_cache, rows, cache_len, B, S, Hq, Hkv, n_items, st);
    else
        launch_append_src<bf16_t>(src, blocks, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows,
                                  positions, q_out, k_cache, v_cache, rows, cache_len, B, S, Hq, Hkv, n_items, st);
    return launch_status(hipGetLastError());
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" int crane_hip_qknorm_rope_append(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                            const void* k_norm_w, float eps, int order, const void* cos,
                                            const void* sin, int64_t cs_stride, int64_t table_rows,
                                            const int32_t* positions,
                                            void* q_out, void* k_cache, void* v_cache, int64_t cache_cap,
                                            const int32_t* cache_len, int64_t max_rows, int B, int S, int Hq,
                                            int Hkv, int D, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (cache_cap <= 0 || max_rows < 0 || max_rows > cache_cap) return CRANE_HIP_E_CAPACITY;
    if ((int64_t)S > max_rows) return CRANE_HIP_E_CAPACITY;
    RowSource src;
    src.qkv = qkv;
    src.stride = qkv_row_stride;
    return qknorm_rope_append(src, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows, positions, q_out,
                              k_cache, v_cache, DenseRows{cache_cap}, cache_len, B, S, Hq, Hkv, D, dtype, stream);
}

// The same append reading the projection's split-K partial products: the
// decode step's qkv_proj as crane_gemm_linear_split, its reduction (and bias)
// folded into this pass.
extern "C" int crane_hip_qknorm_rope_append_parts(const float* parts, int n_parts, const void* qkv_bias,
                                                  const void* q_norm_w, const void* k_norm_w, float eps, int order,
                                                  const void* cos, const void* sin, int64_t cs_stride,
                                                  int64_t table_rows, const int32_t* positions, void* q_out,
                                                  void* k_cache, void* v_cache, int64_t cache_cap,
                                                  const int32_t* cache_len, int64_t max_rows, int B, int S, int Hq,
                                                  int Hkv, int D, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (cache_cap <= 0 || max_rows < 0 || max_rows > cache_cap) return CRANE_HIP_E_CAPACITY;
    if ((int64_t)S > max_rows) return CRANE_HIP_E_CAPACITY;
    RowSource src;  // null parts: no rows at all (CRANE_HIP_E_INVALID unless nothing is to be done)
    src.parts = parts;
    src.n_parts = n_parts;
    src.bias = qkv_bias;
    return qknorm_rope_append(src, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows, positions, q_out,
                              k_cache, v_cache, DenseRows{cache_cap}, cache_len, B, S, Hq, Hkv, D, dtype, stream);
}

// The Hunyuan CLA layer (hunyuan_dense/modeling.rs:502-514) projects only q and
// attends over the anchor layer's cache: the same kernel over Hq head rows per
// token with no key or value heads, so no cache is addressed or written.
extern "C" int crane_hip_qnorm_rope(const void* q, int64_t q_row_stride, const void* q_norm_w, float eps, int order,
                                    const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                                    const int32_t* positions, void* q_out, int B, int S, int Hq, int D, int dtype,
                                    void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || S < 0 || Hq <= 0) return CRANE_HIP_E_INVALID;
    if (order < CRANE_HIP_NORM_THEN_ROPE || order > CRANE_HIP_ROPE_ONLY) return CRANE_HIP_E_INVALID;
    if (!(eps >= 0.0f)) return CRANE_HIP_E_INVALID;
    if (B == 0 || S == 0) return CRANE_HIP_OK;
    if (!q || !cos || !sin || !positions || !q_out) return CRANE_HIP_E_INVALID;
    if (q_row_stride < (int64_t)Hq * D || cs_stride < D / 2 || table_rows <= 0) return CRANE_HIP_E_INVALID;
    const int64_t per16 = dtype == CRANE_HIP_BF16 ? 8 : 4;  // elements per 16 bytes
    if (q_row_stride % per16 != 0 || cs_stride % per16 != 0) return CRANE_HIP_E_ALIGN;
    if (!aligned16(q) || !aligned16(cos) || !aligned16(sin) || !aligned16(q_out) || (q_norm_w && !aligned16(q_norm_w)))
        return CRANE_HIP_E_ALIGN;
    const int64_t n_items = (int64_t)B * S * Hq;
    const int64_t blocks = (n_items + kItemsPerBlock - 1) / kItemsPerBlock;
    if (blocks > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    const DenseRows none{1};  // never consulted: every item is a q head
    if (dtype == CRANE_HIP_F32)
        launch_append<float>(QkvRows<float>{(const float*)q, q_row_stride}, blocks, q_norm_w, nullptr, eps, order, cos,
                             sin, cs_stride, table_rows, positions, q_out, nullptr, nullptr, none, nullptr, S, Hq, 0,
                             n_items, st);
    else
        launch_append<bf16_t>(QkvRows<bf16_t>{(const bf16_t*)q, q_row_stride}, blocks, q_norm_w, nullptr, eps, order,
                              cos, sin, cs_stride, table_rows, positions, q_out, nullptr, nullptr, none, nullptr, S, Hq,
                              0, n_items, st);
    return launch_status(hipGetLastError());
}

extern "C" int crane_hip_qknorm_rope_append_paged(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                                  const void* k_norm_w, float eps, int order, const void* cos,
                                                  const void* sin, int64_t cs_stride, int64_t table_rows,
                                                  const int32_t* positions, void* q_out, void* k_pool, void* v_pool,
                                                  int64_t n_pages, int page_rows, const int32_t* block_table,
                                                  int64_t table_stride, const int32_t* cache_len, int B, int S, int Hq,
                                                  int Hkv, int D, int dtype, void* stream) {
    const int rc = check_paged(n_pages, page_rows, block_table, table_stride, Hkv);
    if (rc) return rc;
    if ((int64_t)S > table_stride * page_rows) return CRANE_HIP_E_CAPACITY;
    RowSource src;
    src.qkv = qkv;
    src.stride = qkv_row_stride;
    return qknorm_rope_append(src, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows,
                              positions, q_out, k_pool, v_pool,
                              PagedRows{block_table, table_stride, n_pages, page_rows}, cache_len, B, S, Hq, Hkv, D,
                              dtype, stream);
}
