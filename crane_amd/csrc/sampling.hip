// sampling.hip -- argmax and top-k over logits rows (gfx950); C ABI in
// include/crane_sampling.h.
//
// Both kernels give one 1024-thread workgroup a row (a vocabulary of ~152k
// logits is 0.3-0.6 MB, one L2's worth) and order elements by a 32-bit key that
// is monotone in the float value (NaN mapped to 0, below -inf).
//   argmax: each thread keeps the largest (key << 32 | ~index) of its
//     16-byte chunks, so a 64-bit max is the largest value with the lowest
//     index; wave and workgroup max with shuffles and LDS.
//   top-k: pass 0 takes each thread's largest key; the k-th largest of those
//     1024 keys (a radix select in LDS) is a lower bound t of the answer.
//     Pass 1 collects the keys >= t -- a few hundred for real logits -- into
//     LDS and a bitonic sort orders them (key descending, index ascending).
//     When more than 2048 keys reach t (a row of equal values, say), an exact
//     radix select of the k-th largest key runs over the row (8 bits per pass,
//     4 passes, per-wave LDS histograms), then one gather: keys above it in
//     any order, keys equal to it in index order when the tie straddles k
//     (ballot prefixes over coalesced tiles), sorted by a 64-lane bitonic
//     network.  The first pass reads HBM; the rest hit L2.
#include "common.h"
#include "../../include/crane_sampling.h"

namespace crane {
namespace {

constexpr int kThreads = 1024;
constexpr int kWavesT = kThreads / 64;

__device__ __forceinline__ uint32_t fkey(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;  // NaN ranks lowest
    if (u == 0x80000000u) u = 0u;                      // -0 equals +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t ikey(float v, uint32_t i) { return ((uint64_t)fkey(v) << 32) | (uint32_t)~i; }

template <typename T> __device__ __forceinline__ float elem(const T* p);
template <> __device__ __forceinline__ float elem<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float elem<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const T* __restrict__ x, int64_t n, uint32_t* __restrict__ out) {
    constexpr int N = 16 / sizeof(T);  // elements per 16-byte chunk
    const T* xr = x + (int64_t)blockIdx.x * n;
    const int tid = threadIdx.x;
    uint64_t best = 0;
    const bool vec = (n % N) == 0 && (((uintptr_t)xr) & 15) == 0;
    const int64_t nvec = vec ? n / N : 0;
    constexpr int U = 8;  // 16-byte loads in flight per thread
    for (int64_t c0 = tid; c0 < nvec; c0 += (int64_t)kThreads * U) {
        uint4 u[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t c = c0 + (int64_t)j * kThreads;
            u[j] = c < nvec ? *reinterpret_cast<const uint4*>(xr + c * N) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t c = c0 + (int64_t)j * kThreads;
            if (c >= nvec) break;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(&u[j]);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                float v;
                if constexpr (sizeof(T) == 4) v = __uint_as_float(w[e]);
                else v = (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
                const uint64_t k = ikey(v, (uint32_t)(c * N + e));
                best = k > best ? k : best;
            }
        }
    }
    for (int64_t i = nvec * N + tid; i < n; i += kThreads) {  // no vector path, or none needed
        const uint64_t k = ikey(elem(xr + i), (uint32_t)i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor64(best, m);
        best = o > best ? o : best;
    }
    __shared__ uint64_t wbest[kWavesT];
    if ((tid & 63) == 0) wbest[tid >> 6] = best;
    __syncthreads();
    if (tid < 64) {
        best = tid < kWavesT ? wbest[tid] : 0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint64_t o = shfl_xor64(best, m);
            best = o > best ? o : best;
        }
        if (tid == 0) out[blockIdx.x] = ~(uint32_t)best;
    }
}

// The bin of an 8-bit digit histogram (256 counts in `tot`) where the count
// from the top reaches krem; run by one wave.  Writes the digit, the count in
// higher bins and the count in the bin.
__device__ __forceinline__ void crossing_bin(const uint32_t* tot, uint32_t krem, int lane, uint32_t* s_digit,
                                             uint32_t* s_above, uint32_t* s_eq) {
    uint32_t c[4], local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        c[j] = tot[255 - (4 * lane + j)];
        local += c[j];
    }
    uint32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
    }
    const uint64_t hit = __ballot(incl >= krem);
    if (lane == __ffsll((unsigned long long)hit) - 1) {
        uint32_t cum = incl - local;
        int j = 0;
        while (j < 3 && cum + c[j] < krem) cum += c[j++];
        *s_digit = 255u - (uint32_t)(4 * lane + j);
        *s_above = cum;
        *s_eq = c[j];
    }
}

constexpr int kCand = 2048;  // candidates sorted in LDS on the fast path

__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ x, int64_t n, int k,
                                                        uint32_t* __restrict__ out) {
    const float* xr = x + (int64_t)blockIdx.x * n;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ uint32_t hist[kWavesT][256];
    __shared__ uint32_t tot[256];
    __shared__ uint32_t tkey[kThreads];
    __shared__ uint64_t cand[kCand];
    __shared__ uint32_t s_digit, s_above, s_eq, s_count, s_base;
    __shared__ uint32_t wsum[kWavesT];
    const bool vec = (n % 4) == 0 && (((uintptr_t)xr) & 15) == 0;
    const int64_t nvec = vec ? n / 4 : 0;

    // Visit every element of the row as (key, index): 16-byte loads, 4 in
    // flight per thread, then a scalar tail.
    auto for_each = [&](auto&& f) __attribute__((always_inline)) {
        constexpr int U = 4;
        for (int64_t c0 = tid; c0 < nvec; c0 += (int64_t)kThreads * U) {
            float4 v[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t c = c0 + (int64_t)j * kThreads;
                v[j] = c < nvec ? *reinterpret_cast<const float4*>(xr + c * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t c = c0 + (int64_t)j * kThreads;
                if (c >= nvec) break;
                f(fkey(v[j].x), (uint32_t)(c * 4));
                f(fkey(v[j].y), (uint32_t)(c * 4 + 1));
                f(fkey(v[j].z), (uint32_t)(c * 4 + 2));
                f(fkey(v[j].w), (uint32_t)(c * 4 + 3));
            }
        }
        for (int64_t i = nvec * 4 + tid; i < n; i += kThreads) f(fkey(xr[i]), (uint32_t)i);
    };

    // Exact radix select of the k-th largest key among the keys `visit`
    // enumerates (4 passes of 8 bits; per-wave LDS histograms).  Returns it;
    // *above = keys above it, *eq = keys equal to it.
    auto select = [&](auto&& visit, uint32_t want, uint32_t* above, uint32_t* eq) __attribute__((always_inline)) {
        uint32_t prefix = 0, mask = 0, krem = want, n_above = 0;
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            for (int j = tid; j < kWavesT * 256; j += kThreads) (&hist[0][0])[j] = 0;
            __syncthreads();
            visit([&](uint32_t key, uint32_t) {
                if ((key & mask) == prefix) atomicAdd(&hist[wave][(key >> shift) & 255u], 1u);
            });
            __syncthreads();
            if (tid < 256) {
                uint32_t t = 0;
#pragma unroll
                for (int w = 0; w < kWavesT; ++w) t += hist[w][tid];
                tot[tid] = t;
            }
            __syncthreads();
            if (wave == 0) crossing_bin(tot, krem, lane, &s_digit, &s_above, &s_eq);
            __syncthreads();
            prefix |= s_digit << shift;
            mask |= 255u << shift;
            krem -= s_above;
            n_above += s_above;
        }
        *above = n_above;
        *eq = s_eq;
        return prefix;
    };

    // Pass 0: the largest key of each thread.  The k-th largest of these 1024
    // keys is a lower bound of the row's k-th largest (they are k distinct
    // elements), so every answer has a key >= t.
    uint32_t mine = 0;
    for_each([&](uint32_t key, uint32_t) { mine = key > mine ? key : mine; });
    tkey[tid] = mine;
    __syncthreads();
    uint32_t dummy_above, dummy_eq;
    const uint32_t t = select([&](auto&& f) { f(tkey[tid], 0u); }, (uint32_t)min(k, kThreads), &dummy_above, &dummy_eq);

    // Pass 1: the candidates (key >= t) into LDS.
    if (tid == 0) s_count = 0;
    __syncthreads();
    for_each([&](uint32_t key, uint32_t i) {
        if (key >= t) {
            const uint32_t slot = atomicAdd(&s_count, 1u);
            if (slot < kCand) cand[slot] = ((uint64_t)key << 32) | ~i;
        }
    });
    __syncthreads();
    const uint32_t count = s_count;
    if (count <= kCand) {
        // Fast path: sort the candidates, key descending then index ascending
        // (bitonic over the next power of two, padded with the lowest key).
        uint32_t P = 64;
        while (P < count) P <<= 1;
        for (uint32_t i = count + tid; i < P; i += kThreads) cand[i] = 0;
        __syncthreads();
        for (uint32_t size = 2; size <= P; size <<= 1)
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t p = tid; p < P / 2; p += kThreads) {
                    const uint32_t a = 2 * stride * (p / stride) + (p % stride), b = a + stride;
                    const bool desc = (a & size) == 0;
                    const uint64_t va = cand[a], vb = cand[b];
                    if ((va < vb) == desc) {
                        cand[a] = vb;
                        cand[b] = va;
                    }
                }
                __syncthreads();
            }
        if (tid < k) out[(int64_t)blockIdx.x * k + tid] = ~(uint32_t)cand[tid];
        return;
    }

    // Many keys >= t (e.g. a row of equal values): exact radix select of the
    // k-th largest over the row, then one gather.
    uint32_t n_above, n_eq;
    const uint32_t kth = select(for_each, (uint32_t)k, &n_above, &n_eq);
    const uint32_t krem = (uint32_t)k - n_above;  // keys equal to kth that are taken
    if (tid == 0) s_count = 0;
    __syncthreads();
    for_each([&](uint32_t key, uint32_t i) {
        if (key > kth || (key == kth && n_eq == krem)) cand[atomicAdd(&s_count, 1u)] = ((uint64_t)key << 32) | ~i;
    });
    if (n_eq > krem) {  // the tie straddles k: equal keys in index order, tile by tile
        if (tid == 0) s_base = 0;
        __syncthreads();
        for (int64_t t0 = 0; t0 < n; t0 += kThreads) {
            const int64_t i = t0 + tid;
            const bool eq = i < n && fkey(xr[i]) == kth;
            const uint64_t b = __ballot(eq);
            if (lane == 0) wsum[wave] = (uint32_t)__popcll(b);
            __syncthreads();
            uint32_t before = s_base;
            for (int w = 0; w < wave; ++w) before += wsum[w];
            before += (uint32_t)__popcll(b & ((1ull << lane) - 1ull));
            if (eq && before < krem) cand[n_above + before] = ((uint64_t)kth << 32) | ~(uint32_t)i;
            __syncthreads();
            if (tid == 0) {
                uint32_t sum = s_base;
                for (int w = 0; w < kWavesT; ++w) sum += wsum[w];
                s_base = sum;
            }
            __syncthreads();
            if (s_base >= krem) break;  // uniform: read after the barrier
        }
    }
    __syncthreads();
    if (wave == 0) {  // sort the k candidates: key descending, then index ascending
        uint64_t v = lane < k ? cand[lane] : 0;
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const uint64_t o = shfl_xor64(v, stride);
                const bool desc = (lane & size) == 0, low = (lane & stride) == 0;
                v = (low == desc) ? (o > v ? o : v) : (o < v ? o : v);
            }
        if (lane < k) out[(int64_t)blockIdx.x * k + lane] = ~(uint32_t)v;
    }
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" int crane_hip_argmax(const void* logits, int64_t rows, int64_t n, int dtype, uint32_t* out_idx,
                                void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (rows < 0 || n <= 0 || n > 0x7fffffffLL || rows > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (rows == 0) return CRANE_HIP_OK;
    if (!logits || !out_idx) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_F32)
        hipLaunchKernelGGL(argmax_kernel<float>, dim3((unsigned)rows), dim3(kThreads), 0, st, (const float*)logits, n,
                           out_idx);
    else
        hipLaunchKernelGGL(argmax_kernel<bf16_t>, dim3((unsigned)rows), dim3(kThreads), 0, st, (const bf16_t*)logits,
                           n, out_idx);
    return launch_status(hipGetLastError());
}

extern "C" int crane_hip_topk(const float* x, int64_t rows, int64_t n, int k, uint32_t* out_idx, void* stream) {
    if (rows < 0 || n <= 0 || n > 0x7fffffffLL || rows > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (k < 1 || k > CRANE_TOPK_MAX || (int64_t)k > n) return CRANE_HIP_E_INVALID;
    if (rows == 0) return CRANE_HIP_OK;
    if (!x || !out_idx) return CRANE_HIP_E_INVALID;
    hipLaunchKernelGGL(topk_kernel, dim3((unsigned)rows), dim3(kThreads), 0, (hipStream_t)stream, x, n, k, out_idx);
    return launch_status(hipGetLastError());
}
