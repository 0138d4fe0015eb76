// decode.hip -- batched split-KV (flash-decoding) attention for one new token
// per sequence over Crane's [B, Hkv, cap, D] KV cache (gfx950).
//
// Replaces the GQA-grouped decode SDPA of qwen3/modeling.rs:432-467 (and
// hunyuan_dense/modeling.rs:575-608, qwen2.rs:185-206) together with the
// batched-decode right-aligned padding + -1e9 mask of qwen3/modeling.rs:1118-1200:
// sequence b reads exactly its own kv_len[b] rows, which gives the same
// softmax as padding with masked columns (exp(-1e9 - m) == 0 in f32).
//
// One kernel (decode_split_kernel): one workgroup per (chunk of kChunk keys,
// kv head, sequence).  The G query heads that share the kv head are processed together,
// so every K/V row is read from HBM once for the whole GQA group.  A row is
// read by 16 lanes with one 16-byte load each (bf16: 8 dims per lane), and a
// wave covers 4 rows per load instruction.  Scores go to LDS, the chunk's
// softmax statistics (max m, sum l, in the log2 domain) are computed once per
// (head, key), and P@V accumulates in f32.  A sequence that fits one chunk is
// normalised and written directly.  Otherwise each chunk writes its
// unnormalised f32 output and (m, l) to the workspace and bumps a per-(sequence,
// head group) counter; the chunk that arrives last combines all partials with
// the log-sum-exp rule, writes the normalised rows and re-arms the counter, so
// no second launch is needed.  The counters must be zero before the first
// call on a workspace and are zero again after every call.
#include "common.h"

namespace crane {
namespace {

constexpr int kChunk = 256;     // keys per workgroup in pass 1
constexpr int kThreads = 256;   // 4 waves
constexpr int kMaxGroup = 8;    // q heads handled per workgroup

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// grid: (nsplit, Hkv * (n_rep / G), B).  ws_o: [B, Hq, nsplit, D] f32;
// ws_ml: [B, Hq, nsplit, 2] f32 (max, sum) in the log2 domain;
// counters: [B, gridDim.y] int32, zero between calls.
template <typename T, int G>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t cap,
    const int32_t* __restrict__ kv_len, int max_kv, int Hq, int Hkv, int n_rep, float scale_log2, int nsplit,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int* __restrict__ counters, T* __restrict__ out) {
    const int c = blockIdx.x;
    const int sub_per_kv = n_rep / G;
    const int kvh = blockIdx.y / sub_per_kv;
    const int h0 = kvh * n_rep + (blockIdx.y % sub_per_kv) * G;  // first q head of this group
    const int b = blockIdx.z;
    const int L = min(kv_len[b], max_kv);  // never read past the rows the host vouched for
    const int j0 = c * kChunk;
    const int tid = threadIdx.x;
    if (j0 >= L) {  // uniform over the workgroup
        if (c == 0)  // an empty sequence attends to nothing: its rows are zero
            for (int e = tid; e < G * kHeadDim; e += kThreads)
                Elem<T>::store(out + ((int64_t)b * Hq + h0) * kHeadDim + e, 0.f);
        return;
    }
    const int n = min(kChunk, L - j0);

    const int lane = tid & 63, wave = tid >> 6, grp = lane >> 4, l16 = lane & 15;

    __shared__ float s_lds[kChunk][G];
    __shared__ float red[4][G][kHeadDim];
    __shared__ float ml[G][2];

    float qf[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        load8(q + ((int64_t)b * Hq + h0 + h) * kHeadDim + 8 * l16, qf[h]);
#pragma unroll
        for (int d = 0; d < 8; ++d) qf[h][d] *= scale_log2;
    }
    const int64_t base = (((int64_t)b * Hkv + kvh) * cap + j0) * kHeadDim + 8 * l16;
    const T* K = kc + base;
    const T* V = vc + base;

    // Phase A: scores (log2 domain) of this chunk.
    for (int it = 0; it < kChunk / 16; ++it) {
        const int j = it * 16 + wave * 4 + grp;
        if (j < n) {  // uniform within a 16-lane group
            float kf[8];
            load8(K + (int64_t)j * kHeadDim, kf);
            float acc[G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float a = 0.f;
#pragma unroll
                for (int d = 0; d < 8; ++d) a += qf[h][d] * kf[d];
                acc[h] = a;
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                acc[h] += __shfl_xor(acc[h], 1, 16);
                acc[h] += __shfl_xor(acc[h], 2, 16);
                acc[h] += __shfl_xor(acc[h], 4, 16);
                acc[h] += __shfl_xor(acc[h], 8, 16);
            }
#pragma unroll
            for (int h = 0; h < G; ++h)
                if (l16 == h) s_lds[j][h] = acc[h];
        }
    }
    __syncthreads();

    // Phase B: per-head chunk max and exp-sum; scores become probabilities.
    for (int h = wave; h < G; h += 4) {
        float m = -INFINITY;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, s_lds[j][h]);
        m = wave_max(m);
        float l = 0.f;
        for (int j = lane; j < n; j += 64) {
            const float p = fast_exp2(s_lds[j][h] - m);
            s_lds[j][h] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            ml[h][0] = m;
            ml[h][1] = l;
        }
    }
    __syncthreads();

    // Phase C: unnormalised P @ V.
    float o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) o[h][d] = 0.f;
    for (int it = 0; it < kChunk / 16; ++it) {
        const int j = it * 16 + wave * 4 + grp;
        if (j < n) {
            float vf[8];
            load8(V + (int64_t)j * kHeadDim, vf);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = s_lds[j][h];
#pragma unroll
                for (int d = 0; d < 8; ++d) o[h][d] += p * vf[d];
            }
        }
    }
    // Sum the 4 row groups of the wave, then the 4 waves through LDS.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            o[h][d] += __shfl_xor(o[h][d], 16);
            o[h][d] += __shfl_xor(o[h][d], 32);
        }
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int d = 0; d < 8; ++d) red[wave][h][8 * l16 + d] = o[h][d];
    }
    __syncthreads();

    const int n_chunks = (L + kChunk - 1) / kChunk;
    if (n_chunks == 1) {  // the whole sequence fits one chunk: normalise and finish here
        for (int e = tid; e < G * kHeadDim; e += kThreads) {
            const int h = e / kHeadDim, d = e % kHeadDim;
            const float v = red[0][h][d] + red[1][h][d] + red[2][h][d] + red[3][h][d];
            Elem<T>::store(out + ((int64_t)b * Hq + h0 + h) * kHeadDim + d, v / ml[h][1]);
        }
        return;
    }
    for (int e = tid; e < G * kHeadDim; e += kThreads) {
        const int h = e / kHeadDim, d = e % kHeadDim;
        const float v = red[0][h][d] + red[1][h][d] + red[2][h][d] + red[3][h][d];
        ws_o[(((int64_t)b * Hq + h0 + h) * nsplit + c) * kHeadDim + d] = v;
    }
    if (tid < G) {
        float* dst = ws_ml + (((int64_t)b * Hq + h0 + tid) * nsplit + c) * 2;
        dst[0] = ml[tid][0];
        dst[1] = ml[tid][1];
    }
    // The last chunk of this (sequence, head group) to finish merges all
    // partials (log-sum-exp rule) and re-arms the counter for the next call.
    __threadfence();
    __syncthreads();
    __shared__ int is_last;
    int* counter = counters + (int64_t)b * gridDim.y + blockIdx.y;
    if (tid == 0) is_last = atomicAdd(counter, 1) == n_chunks - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int e = tid; e < G * kHeadDim; e += kThreads) {
        const int h = e / kHeadDim, d = e % kHeadDim;
        const int64_t bh = (int64_t)b * Hq + h0 + h;
        const float* pm = ws_ml + bh * nsplit * 2;
        const float* po = ws_o + bh * nsplit * kHeadDim + d;
        float M = -INFINITY;
        for (int cc = 0; cc < n_chunks; ++cc) M = fmaxf(M, __builtin_nontemporal_load(pm + 2 * cc));
        float num = 0.f, den = 0.f;
        for (int cc = 0; cc < n_chunks; ++cc) {
            const float w = fast_exp2(__builtin_nontemporal_load(pm + 2 * cc) - M);
            den += w * __builtin_nontemporal_load(pm + 2 * cc + 1);
            num += w * __builtin_nontemporal_load(po + (int64_t)cc * kHeadDim);
        }
        Elem<T>::store(out + bh * kHeadDim + d, num / den);
    }
    if (tid == 0) *counter = 0;
}

int pick_group(int n_rep) {
    for (int g = kMaxGroup; g >= 1; --g)
        if (n_rep % g == 0) return g;
    return 1;
}

template <typename T>
int launch_decode(const T* q, const T* kc, const T* vc, int64_t cap, const int32_t* kv_len, int max_kv, int nsplit,
                  int B, int Hq, int Hkv, float scale, float* ws_o, float* ws_ml, int* counters, T* out,
                  hipStream_t st) {
    const int n_rep = Hq / Hkv;
    const int G = pick_group(n_rep);
    const dim3 grid((unsigned)nsplit, (unsigned)(Hkv * (n_rep / G)), (unsigned)B);
    const float sl = scale * kLog2e;
#define CRANE_DECODE_CASE(g)                                                                                 \
    case g:                                                                                                  \
        hipLaunchKernelGGL((decode_split_kernel<T, g>), grid, dim3(kThreads), 0, st, q, kc, vc, cap, kv_len, \
                           max_kv, Hq, Hkv, n_rep, sl, nsplit, ws_o, ws_ml, counters, out);                 \
        break;
    switch (G) {
        CRANE_DECODE_CASE(1)
        CRANE_DECODE_CASE(2)
        CRANE_DECODE_CASE(3)
        CRANE_DECODE_CASE(4)
        CRANE_DECODE_CASE(5)
        CRANE_DECODE_CASE(6)
        CRANE_DECODE_CASE(7)
        CRANE_DECODE_CASE(8)
        default: return CRANE_HIP_E_GQA;
    }
#undef CRANE_DECODE_CASE
    return launch_status(hipGetLastError());
}

int64_t n_splits(int64_t max_kv) { return (max_kv + kChunk - 1) / kChunk; }

struct WsLayout {
    size_t o_off, ml_off, cnt_off, total;
};

WsLayout ws_layout(int B, int Hq, int Hkv, int64_t ns) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout w;
    const size_t o_bytes = (size_t)B * Hq * ns * kHeadDim * sizeof(float);
    const size_t ml_bytes = (size_t)B * Hq * ns * 2 * sizeof(float);
    const size_t cnt_bytes = (size_t)B * Hq * sizeof(int);  // >= B * Hkv * (n_rep / G)
    (void)Hkv;
    w.o_off = 0;
    w.ml_off = up(o_bytes);
    w.cnt_off = w.ml_off + up(ml_bytes);
    w.total = w.cnt_off + up(cnt_bytes);
    return w;
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" size_t crane_hip_attn_decode_workspace(int B, int Hq, int Hkv, int D, int64_t max_kv, int dtype) {
    (void)dtype;
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || D != kHeadDim || max_kv <= 0) return 0;
    return ws_layout(B, Hq, Hkv, n_splits(max_kv)).total;
}

extern "C" int crane_hip_attn_decode(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                     const int32_t* kv_len, int64_t max_kv, int B, int Hq, int Hkv, int D,
                                     float scale, void* workspace, size_t ws_bytes, void* out, int dtype,
                                     void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || Hq <= 0 || Hkv <= 0) return CRANE_HIP_E_INVALID;
    if (Hq % Hkv != 0) return CRANE_HIP_E_GQA;
    if (cache_cap <= 0 || max_kv > cache_cap) return CRANE_HIP_E_CAPACITY;
    if (max_kv <= 0) return CRANE_HIP_E_INVALID;
    if (!(scale > 0.0f) || !__builtin_isfinite(scale)) return CRANE_HIP_E_INVALID;
    if (B == 0) return CRANE_HIP_OK;
    if (!q || !k_cache || !v_cache || !kv_len || !out) return CRANE_HIP_E_INVALID;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return CRANE_HIP_E_ALIGN;
    const size_t need = crane_hip_attn_decode_workspace(B, Hq, Hkv, D, max_kv, dtype);
    if (!workspace || ws_bytes < need || !aligned16(workspace)) return CRANE_HIP_E_WORKSPACE;
    const int64_t ns = n_splits(max_kv);
    if (max_kv > 0x7fffffffLL || ns > 0x7fffffffLL || (int64_t)B * Hq > 0x7fffffffLL || B > 65535)
        return CRANE_HIP_E_INVALID;
    const WsLayout w = ws_layout(B, Hq, Hkv, ns);
    float* ws_o = (float*)((char*)workspace + w.o_off);
    float* ws_ml = (float*)((char*)workspace + w.ml_off);
    int* counters = (int*)((char*)workspace + w.cnt_off);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        return launch_decode<float>((const float*)q, (const float*)k_cache, (const float*)v_cache, cache_cap, kv_len,
                                    (int)max_kv, (int)ns, B, Hq, Hkv, scale, ws_o, ws_ml, counters, (float*)out, st);
    return launch_decode<bf16_t>((const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, cache_cap,
                                 kv_len, (int)max_kv, (int)ns, B, Hq, Hkv, scale, ws_o, ws_ml, counters,
                                 (bf16_t*)out, st);
}
