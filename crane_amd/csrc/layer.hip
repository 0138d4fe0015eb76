// layer.hip -- the row kernels either side of the attention block of a decoder
// layer (gfx950); C ABI in include/crane_layer.h.
//
// RmsNorm (input_layernorm / post_attention_layernorm / final norm,
// qwen3/modeling.rs:655-673 via candle_nn::RmsNorm), residual add + RmsNorm (the
// candle pair Crane's FusedAddRmsNorm runs, crane-core/src/fused_ops/
// cuda_impl.rs:200-258), SiLU(gate) * up (fused_ops.cu:104-126) and the plain
// residual add (fused_ops.cu:382-393).
//
// All four are HBM-bound.  The norms give one wave a whole row: the row is
// loaded once into registers (16-byte chunks, up to CRANE_LAYER_MAX_COLS
// elements), the sum of squares is a DPP wave reduction, and the normalised
// row is written from the registers, so every tensor crosses HBM exactly once
// (add + norm: residual and hidden read, residual and out written).  With few
// rows (a decode step) one wave per row leaves most of the chip idle and the
// call is latency-bound; there a workgroup of 4 waves takes each row.  Rounding
// follows candle's ops: the sum r + h is rounded to T before it is stored and
// squared; m = sqrt(sum/cols + eps) is rounded to T; then x / m and the
// product with the weight are each rounded to T.  SiLU * up is the f32
// formula of Crane's kernel, g / (1 + exp(-g)) * u, rounded once to T.
#include "common.h"
#include "../../include/crane_layer.h"

namespace crane {
namespace {

template <typename T> struct Vec;
template <> struct Vec<float> {
    static constexpr int N = 4;
    static __device__ __forceinline__ void unpack(const uint4& u, float (&v)[4]) {
        v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y);
        v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
    }
    static __device__ __forceinline__ uint4 pack(const float (&v)[4]) {
        return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    }
};
template <> struct Vec<bf16_t> {
    static constexpr int N = 8;
    static __device__ __forceinline__ void unpack(const uint4& u, float (&v)[8]) {
        v[0] = bf16_lo(u.x); v[1] = bf16_hi(u.x); v[2] = bf16_lo(u.y); v[3] = bf16_hi(u.y);
        v[4] = bf16_lo(u.z); v[5] = bf16_hi(u.z); v[6] = bf16_lo(u.w); v[7] = bf16_hi(u.w);
    }
    static __device__ __forceinline__ uint4 pack(const float (&v)[8]) {
        return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                          pack_bf16x2(v[6], v[7]));
    }
};

// 16-byte loads and stores; NT selects the non-temporal (streaming) policy.
// Which kernel streams what was measured at config 4's prefill rows with the
// tensors rotated through 3 copies (so the 256 MB Infinity Cache cannot
// serve a call from the one before): rms_norm 6% faster with non-temporal
// stores, add + rms_norm and the residual add 8% faster with both,
// silu_mul fastest with neither.
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));
template <bool NT, typename T>
__device__ __forceinline__ uint4 ld16(const T* p) {
    if constexpr (NT) {
        const u32x4_v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}
template <bool NT, typename T>
__device__ __forceinline__ void st16(T* p, const uint4& u) {
    if constexpr (NT) {
        const u32x4_v v = {u.x, u.y, u.z, u.w};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_v*>(p));
    } else {
        *reinterpret_cast<uint4*>(p) = u;
    }
}

constexpr int kRowsPerBlock = 4;  // one wave per row

// One wave per row; CH 16-byte chunks per lane hold the row (CH * 64 * N >= cols).
template <typename T, bool ADD, int CH>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rms_norm_kernel(T* __restrict__ x, const T* __restrict__ hidden,
                                                                     const T* __restrict__ w, T* __restrict__ out,
                                                                     int64_t rows, int cols, float eps) {
    constexpr int N = Vec<T>::N;
    constexpr bool kNtLoad = ADD;  // the rows are streamed; the weight is shared by all rows
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves
    const int nch = cols / N;
    T* xr = x + row * cols;
    uint4 c[CH];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * 64 + lane;
        if (idx < nch) {
            uint4 a = ld16<kNtLoad>(xr + idx * N);
            if constexpr (ADD) {  // residual = T(residual + hidden), stored, and normed as rounded
                float va[N], vh[N];
                Vec<T>::unpack(a, va);
                Vec<T>::unpack(ld16<kNtLoad>(hidden + row * cols + idx * N), vh);
#pragma unroll
                for (int e = 0; e < N; ++e) va[e] += vh[e];
                a = Vec<T>::pack(va);
                st16<true>(xr + idx * N, a);
            }
            c[i] = a;
            float v[N];
            Vec<T>::unpack(a, v);
#pragma unroll
            for (int e = 0; e < N; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
        }
    }
    ss = wave_sum(ss);
    const float m = rt<T>(sqrtf(ss / (float)cols + eps));
    const bool fast = m >= 0x1p-60f && m <= 0x1p60f;  // a normal, moderate divisor (div_by); else the division
    const float rm = 1.0f / m;
    T* orow = out + row * cols;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * 64 + lane;
        if (idx < nch) {
            float v[N], wv[N];
            Vec<T>::unpack(c[i], v);
            if (w) {
                Vec<T>::unpack(ld16<false>(w + idx * N), wv);
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) wv[e] = 1.f;
            }
            if (fast) {  // uniform: x / m from the row's reciprocal (div_by)
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(div_by(v[e], m, rm)) * wv[e];
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(v[e] / m) * wv[e];
            }
            st16<true>(orow + idx * N, Vec<T>::pack(v));  // the pack rounds the product to T
        }
    }
}

// Few rows (a decode step's B rows): one workgroup of 256 threads per row, so
// the row's chunks are spread over 4 waves instead of one.  Thread t holds
// chunks t, t + 256, ...; the weight chunks are loaded with the row (one round
// trip to memory); the sum of squares is reduced per wave (DPP) and across the
// 4 waves through LDS in a fixed order.  Same rounding points as
// rms_norm_kernel.
constexpr int kRowThreads = 256;

template <typename T, bool ADD, int CH>
__global__ __launch_bounds__(kRowThreads) void rms_norm_row_kernel(T* __restrict__ x, const T* __restrict__ hidden,
                                                                   const T* __restrict__ w, T* __restrict__ out,
                                                                   int cols, float eps) {
    constexpr int N = Vec<T>::N;
    __shared__ float part[kRowThreads / 64];
    const int64_t row = blockIdx.x;
    const int nch = cols / N;
    T* xr = x + row * cols;
    uint4 c[CH], wc[CH], hc[ADD ? CH : 1];
    // every load of the row is issued before the first store
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            c[i] = ld16<ADD>(xr + idx * N);
            if (w) wc[i] = ld16<false>(w + idx * N);
            if constexpr (ADD) hc[i] = ld16<true>(hidden + row * cols + idx * N);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            uint4 a = c[i];
            if constexpr (ADD) {  // residual = T(residual + hidden), stored, and normed as rounded
                float va[N], vh[N];
                Vec<T>::unpack(a, va);
                Vec<T>::unpack(hc[i], vh);
#pragma unroll
                for (int e = 0; e < N; ++e) va[e] += vh[e];
                a = Vec<T>::pack(va);
                st16<true>(xr + idx * N, a);
            }
            c[i] = a;
            float v[N];
            Vec<T>::unpack(a, v);
#pragma unroll
            for (int e = 0; e < N; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = part[0];
#pragma unroll
    for (int v = 1; v < kRowThreads / 64; ++v) total += part[v];
    const float m = rt<T>(sqrtf(total / (float)cols + eps));
    const bool fast = m >= 0x1p-60f && m <= 0x1p60f;  // a normal, moderate divisor (div_by); else the division
    const float rm = 1.0f / m;
    T* orow = out + row * cols;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            float v[N], wv[N];
            Vec<T>::unpack(c[i], v);
            if (w) {
                Vec<T>::unpack(wc[i], wv);
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) wv[e] = 1.f;
            }
            if (fast) {  // uniform: x / m from the row's reciprocal (div_by)
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(div_by(v[e], m, rm)) * wv[e];
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(v[e] / m) * wv[e];
            }
            st16<true>(orow + idx * N, Vec<T>::pack(v));
        }
    }
}

// residual = T(residual + T(sum_s parts[s])), then the norm of the sum, as
// rms_norm_row_kernel<T, true> with hidden = T(sum_s parts[s]): parts holds
// the f32 split-K partial sums [n_parts][rows][cols] of the projection whose
// output is added here (crane_gemm_linear_split), summed in split order and
// rounded once, as the whole product's output would be.  NP (2 or 4, or 0 for
// any count) is n_parts known at compile time: then every load of the row --
// residual, weight and all the partials -- is issued before the first use,
// one memory round trip in all (with a run-time count each split's loads
// waited for the previous split's).
template <typename T, int CH, int NP>
__global__ __launch_bounds__(kRowThreads) void add_parts_rms_norm_row_kernel(T* __restrict__ x,
                                                                             const float* __restrict__ parts,
                                                                             int n_parts, const T* __restrict__ w,
                                                                             T* __restrict__ out, int64_t rows,
                                                                             int cols, float eps) {
    constexpr int N = Vec<T>::N;
    constexpr bool kHold = NP > 0 && CH * NP * N <= 128;  // partials held in registers
    constexpr int NH = kHold ? NP : 1;
    __shared__ float part[kRowThreads / 64];
    const int64_t row = blockIdx.x;
    const int nch = cols / N;
    T* xr = x + row * cols;
    uint4 c[CH], wc[CH];
    float4 pq[kHold ? CH : 1][NH][N / 4];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            c[i] = ld16<true>(xr + idx * N);
            if (w) wc[i] = ld16<false>(w + idx * N);
            if constexpr (kHold) {
#pragma unroll
                for (int sp = 0; sp < NP; ++sp) {
                    const float* pp = parts + ((int64_t)sp * rows + row) * cols + (int64_t)idx * N;
#pragma unroll
                    for (int e = 0; e < N; e += 4) pq[i][sp][e / 4] = *reinterpret_cast<const float4*>(pp + e);
                }
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            float va[N], vh[N];
#pragma unroll
            for (int e = 0; e < N; ++e) vh[e] = 0.f;
            auto add4 = [&](int e, const float4 q) __attribute__((always_inline)) {
                vh[e] += q.x;
                vh[e + 1] += q.y;
                vh[e + 2] += q.z;
                vh[e + 3] += q.w;
            };
            if constexpr (kHold) {
#pragma unroll
                for (int sp = 0; sp < NP; ++sp)
#pragma unroll
                    for (int e = 0; e < N; e += 4) add4(e, pq[i][sp][e / 4]);
            } else {
                for (int sp = 0; sp < n_parts; ++sp) {
                    const float* pp = parts + ((int64_t)sp * rows + row) * cols + (int64_t)idx * N;
#pragma unroll
                    for (int e = 0; e < N; e += 4) add4(e, *reinterpret_cast<const float4*>(pp + e));
                }
            }
            Vec<T>::unpack(c[i], va);
#pragma unroll
            for (int e = 0; e < N; ++e) va[e] += rt<T>(vh[e]);
            const uint4 a = Vec<T>::pack(va);
            st16<true>(xr + idx * N, a);
            c[i] = a;
            float v[N];
            Vec<T>::unpack(a, v);
#pragma unroll
            for (int e = 0; e < N; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = part[0];
#pragma unroll
    for (int v = 1; v < kRowThreads / 64; ++v) total += part[v];
    const float m = rt<T>(sqrtf(total / (float)cols + eps));
    const bool fast = m >= 0x1p-60f && m <= 0x1p60f;  // a normal, moderate divisor (div_by); else the division
    const float rm = 1.0f / m;
    T* orow = out + row * cols;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int idx = i * kRowThreads + (int)threadIdx.x;
        if (idx < nch) {
            float v[N], wv[N];
            Vec<T>::unpack(c[i], v);
            if (w) {
                Vec<T>::unpack(wc[i], wv);
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) wv[e] = 1.f;
            }
            if (fast) {
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(div_by(v[e], m, rm)) * wv[e];
            } else {
#pragma unroll
                for (int e = 0; e < N; ++e) v[e] = rt<T>(v[e] / m) * wv[e];
            }
            st16<true>(orow + idx * N, Vec<T>::pack(v));
        }
    }
}

template <typename T>
int launch_add_parts_norm(T* x, const float* parts, int n_parts, const T* w, T* out, int64_t rows, int cols,
                          float eps, hipStream_t st) {
    const int per_thread = (cols / Vec<T>::N + kRowThreads - 1) / kRowThreads;
#define CRANE_PARTS_CASE(ch)                                                                                      \
    if (per_thread <= ch) {                                                                                       \
        if (n_parts == 4)                                                                                         \
            hipLaunchKernelGGL((add_parts_rms_norm_row_kernel<T, ch, 4>), dim3((unsigned)rows), dim3(kRowThreads), \
                               0, st, x, parts, n_parts, w, out, rows, cols, eps);                                \
        else if (n_parts == 2)                                                                                    \
            hipLaunchKernelGGL((add_parts_rms_norm_row_kernel<T, ch, 2>), dim3((unsigned)rows), dim3(kRowThreads), \
                               0, st, x, parts, n_parts, w, out, rows, cols, eps);                                \
        else                                                                                                      \
            hipLaunchKernelGGL((add_parts_rms_norm_row_kernel<T, ch, 0>), dim3((unsigned)rows), dim3(kRowThreads), \
                               0, st, x, parts, n_parts, w, out, rows, cols, eps);                                \
        return launch_status(hipGetLastError());                                                                  \
    }
    CRANE_PARTS_CASE(1)
    CRANE_PARTS_CASE(2)
    CRANE_PARTS_CASE(4)
    CRANE_PARTS_CASE(8)
#undef CRANE_PARTS_CASE
    return CRANE_HIP_E_INVALID;
}

// Row counts below this take rms_norm_row_kernel (a workgroup per row).
constexpr int64_t kFewRows = 1024;

// grid (ceil(chunks per row / 256), row slots): thread x of workgroup
// (bx, by) owns chunk 256 bx + x of rows by, by + gridDim.y, ...  A flat
// chunk index needed a 64-bit division per chunk, which made the kernel
// compute-bound (config 4 rows: 773.6 -> 670.4 us, 60.2% -> 69.4% of HBM).
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* __restrict__ gu, T* __restrict__ out, int inter,
                                                       int64_t rows) {
    constexpr int N = Vec<T>::N;
    const int cpr = inter / N;  // chunks per output row
    const int j = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (j >= cpr) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const T* g = gu + r * 2 * inter + (int64_t)j * N;
        float gv[N], uv[N];
        Vec<T>::unpack(ld16<false>(g), gv);
        Vec<T>::unpack(ld16<false>(g + inter), uv);
#pragma unroll
        for (int e = 0; e < N; ++e) gv[e] = silu(gv[e]) * uv[e];
        st16<false>(out + r * inter + (int64_t)j * N, Vec<T>::pack(gv));
    }
}

template <typename T>
__global__ __launch_bounds__(256) void residual_add_kernel(T* __restrict__ res, const T* __restrict__ hid,
                                                           int64_t n_chunks) {
    constexpr int N = Vec<T>::N;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < n_chunks;
         c += (int64_t)gridDim.x * blockDim.x) {
        float a[N], h[N];
        Vec<T>::unpack(ld16<true>(res + c * N), a);
        Vec<T>::unpack(ld16<true>(hid + c * N), h);
#pragma unroll
        for (int e = 0; e < N; ++e) a[e] += h[e];
        st16<true>(res + c * N, Vec<T>::pack(a));
    }
}

// Grid of a grid-stride elementwise kernel: enough workgroups to fill the
// chip several times over, no more.
unsigned stride_grid(int64_t n_chunks) {
    const int64_t want = (n_chunks + 255) / 256;
    return (unsigned)(want < 8192 ? (want > 0 ? want : 1) : 8192);
}

template <typename T, bool ADD>
int launch_norm(T* x, const T* hidden, const T* w, T* out, int64_t rows, int cols, float eps, hipStream_t st) {
    if (rows < kFewRows) {
        const int per_thread = (cols / Vec<T>::N + kRowThreads - 1) / kRowThreads;
#define CRANE_ROW_CASE(ch)                                                                                       \
        if (per_thread <= ch) {                                                                                  \
            hipLaunchKernelGGL((rms_norm_row_kernel<T, ADD, ch>), dim3((unsigned)rows), dim3(kRowThreads), 0, st, \
                               x, hidden, w, out, cols, eps);                                                    \
            return launch_status(hipGetLastError());                                                             \
        }
        CRANE_ROW_CASE(1)
        CRANE_ROW_CASE(2)
        CRANE_ROW_CASE(4)
        CRANE_ROW_CASE(8)
#undef CRANE_ROW_CASE
        return CRANE_HIP_E_INVALID;
    }
    const int per_lane = (cols / Vec<T>::N + 63) / 64;
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)), block(64 * kRowsPerBlock);
#define CRANE_NORM_CASE(ch)                                                                                   \
    if (per_lane <= ch) {                                                                                     \
        hipLaunchKernelGGL((rms_norm_kernel<T, ADD, ch>), grid, block, 0, st, x, hidden, w, out, rows, cols, eps); \
        return launch_status(hipGetLastError());                                                              \
    }
    CRANE_NORM_CASE(2)
    CRANE_NORM_CASE(4)
    CRANE_NORM_CASE(8)
    CRANE_NORM_CASE(16)
    CRANE_NORM_CASE(32)
#undef CRANE_NORM_CASE
    return CRANE_HIP_E_INVALID;
}

int check_rows(int dtype, const void* a, const void* b, const void* c, int64_t rows, int cols) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (rows < 0 || cols <= 0 || cols > CRANE_LAYER_MAX_COLS) return CRANE_HIP_E_INVALID;
    if (cols % (dtype == CRANE_HIP_F32 ? 4 : 8) != 0) return CRANE_HIP_E_ALIGN;
    if (rows == 0) return CRANE_HIP_OK;
    if (!a || !b || !c) return CRANE_HIP_E_INVALID;
    if (!aligned16(a) || !aligned16(b) || !aligned16(c)) return CRANE_HIP_E_ALIGN;
    if ((rows + kRowsPerBlock - 1) / kRowsPerBlock > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    return -1;  // go on
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" int crane_hip_rms_norm(const void* x, const void* w, void* out, int64_t rows, int cols, float eps,
                                  int dtype, void* stream) {
    int rc = check_rows(dtype, x, out, out, rows, cols);
    if (rc >= 0) return rc;
    if (!(eps >= 0.0f) || (w && !aligned16(w))) return w && !aligned16(w) ? CRANE_HIP_E_ALIGN : CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        return launch_norm<float, false>((float*)const_cast<void*>(x), nullptr, (const float*)w, (float*)out, rows,
                                         cols, eps, st);
    return launch_norm<bf16_t, false>((bf16_t*)const_cast<void*>(x), nullptr, (const bf16_t*)w, (bf16_t*)out, rows,
                                      cols, eps, st);
}

extern "C" int crane_hip_add_rms_norm(void* residual, const void* hidden, const void* w, void* out, int64_t rows,
                                      int cols, float eps, int dtype, void* stream) {
    int rc = check_rows(dtype, residual, hidden, out, rows, cols);
    if (rc >= 0) return rc;
    if (!(eps >= 0.0f)) return CRANE_HIP_E_INVALID;
    if (w && !aligned16(w)) return CRANE_HIP_E_ALIGN;
    if (out == residual || out == hidden) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        return launch_norm<float, true>((float*)residual, (const float*)hidden, (const float*)w, (float*)out, rows,
                                        cols, eps, st);
    return launch_norm<bf16_t, true>((bf16_t*)residual, (const bf16_t*)hidden, (const bf16_t*)w, (bf16_t*)out, rows,
                                     cols, eps, st);
}

extern "C" int crane_hip_silu_mul(const void* gate_up, void* out, int64_t rows, int inter, int dtype,
                                  void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (rows < 0 || inter <= 0) return CRANE_HIP_E_INVALID;
    const int N = dtype == CRANE_HIP_F32 ? 4 : 8;
    if (inter % N != 0) return CRANE_HIP_E_ALIGN;
    if (rows == 0) return CRANE_HIP_OK;
    if (!gate_up || !out) return CRANE_HIP_E_INVALID;
    if (!aligned16(gate_up) || !aligned16(out)) return CRANE_HIP_E_ALIGN;
    const dim3 grid((unsigned)((inter / N + 255) / 256), (unsigned)(rows < 16384 ? rows : 16384));
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        hipLaunchKernelGGL(silu_mul_kernel<float>, grid, dim3(256), 0, st, (const float*)gate_up, (float*)out, inter,
                           rows);
    else
        hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, grid, dim3(256), 0, st, (const bf16_t*)gate_up, (bf16_t*)out,
                           inter, rows);
    return launch_status(hipGetLastError());
}

extern "C" int crane_hip_residual_add(void* residual, const void* hidden, int64_t n, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (n < 0) return CRANE_HIP_E_INVALID;
    const int N = dtype == CRANE_HIP_F32 ? 4 : 8;
    if (n % N != 0) return CRANE_HIP_E_ALIGN;
    if (n == 0) return CRANE_HIP_OK;
    if (!residual || !hidden) return CRANE_HIP_E_INVALID;
    if (!aligned16(residual) || !aligned16(hidden)) return CRANE_HIP_E_ALIGN;
    const int64_t n_chunks = n / N;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        hipLaunchKernelGGL(residual_add_kernel<float>, dim3(stride_grid(n_chunks)), dim3(256), 0, st,
                           (float*)residual, (const float*)hidden, n_chunks);
    else
        hipLaunchKernelGGL(residual_add_kernel<bf16_t>, dim3(stride_grid(n_chunks)), dim3(256), 0, st,
                           (bf16_t*)residual, (const bf16_t*)hidden, n_chunks);
    return launch_status(hipGetLastError());
}

extern "C" int crane_hip_add_rms_norm_parts(void* residual, const float* parts, int n_parts, const void* w, void* out,
                                            int64_t rows, int cols, float eps, int dtype, void* stream) {
    int rc = check_rows(dtype, residual, parts, out, rows, cols);
    if (rc >= 0) return rc;
    if (!(eps >= 0.0f) || n_parts < 1 || n_parts > 64 || rows > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (w && !aligned16(w)) return CRANE_HIP_E_ALIGN;
    if (out == residual || (const void*)out == (const void*)parts) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        return launch_add_parts_norm<float>((float*)residual, parts, n_parts, (const float*)w, (float*)out, rows, cols,
                                            eps, st);
    return launch_add_parts_norm<bf16_t>((bf16_t*)residual, parts, n_parts, (const bf16_t*)w, (bf16_t*)out, rows,
                                         cols, eps, st);
}
