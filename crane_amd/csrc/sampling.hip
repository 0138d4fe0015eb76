// sampling.hip -- argmax and top-k over logits rows (gfx950); C ABI in
// include/crane_sampling.h.
//
// The single-pass kernels give one 1024-thread workgroup a row (a vocabulary
// of ~152k logits is 0.3-0.6 MB, one L2's worth); with few rows the _ws entry
// points split each row over many workgroups (see "split rows" below).  All
// order elements by a 32-bit key that is monotone in the float value (NaN
// mapped to 0, below -inf).
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

// Sort `count` <= kCand candidates (key << 32 | ~index) held in LDS, key
// descending then index ascending (bitonic over the next power of two, padded
// with the lowest key), and write the first k indices; the whole workgroup
// calls it.
__device__ void sort_candidates(uint64_t* cand, uint32_t count, int k, uint32_t* __restrict__ out_row) {
    const int tid = threadIdx.x;
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
    if (tid < k) out_row[tid] = ~(uint32_t)cand[tid];
}

// The exact top-k of one row by one workgroup of kThreads threads.
__device__ void topk_block(const float* __restrict__ xr, int64_t n, int k, uint32_t* __restrict__ out_row) {
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
    if (count <= kCand) {  // fast path: sort the candidates
        sort_candidates(cand, count, k, out_row);
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
        if (lane < k) out_row[lane] = ~(uint32_t)v;
    }
}

__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ x, int64_t n, int k,
                                                        uint32_t* __restrict__ out) {
    topk_block(x + (int64_t)blockIdx.x * n, n, k, out + (int64_t)blockIdx.x * k);
}

// ------------------------------------------------------------------ split rows
//
// Few rows: one workgroup per row would leave most of the chip idle (a
// 152k-entry row is 0.3-0.6 MB), so each row is cut into P slices of L
// elements (P >= 64 workgroups per row) and the work goes in phases, each a
// kernel, that meet in the caller's workspace (a kernel boundary is the only
// synchronisation: nothing to clear, no counters, no fences):
//   argmax:  (1) each slice's largest (key << 32 | ~index);  (2) the largest of
//            the P of a row.
//   top-k:   (1) each slice's largest key, and slice 0 zeroes the row's
//            candidate count;  (2) every workgroup of a row computes t, the
//            k-th largest of the P slice maxima -- k elements of distinct
//            slices are >= t, so t is a lower bound of the row's k-th largest
//            and every answer has a key >= t (t is taken a little lower
//            still, to the 24-bit prefix) -- and appends its slice's keys
//            >= t to the row's candidate list (wave-aggregated atomics);
//            (3) one workgroup per row ranks the candidates (a few hundred for
//            real logits; a thread's rank is the count of larger candidates)
//            or sorts them (more than 1024) and writes the first k, or, when
//            more than kCand reached t (long runs of equal values), runs the
//            exact one-workgroup path over the row.
// (Merging the phases into one kernel, the last workgroup of a row to arrive
// doing the merge, needs an agent-scope release / acquire per workgroup; at
// these sizes those fences cost more than the launches they save.)
constexpr int kSplitThreads = 256;
constexpr int kSplitMinParts = CRANE_TOPK_MAX;  // P >= k, so the slice-max bound holds
constexpr int kSplitMaxParts = 256;
constexpr int64_t kSplitMinN = 32768;
constexpr int64_t kSplitMaxRows = 32;

// Slice [p L, min(n, p L + L)) of row xr as (key, index) pairs.
template <typename T, typename F>
__device__ __forceinline__ void for_slice(const T* __restrict__ xr, int64_t n, int64_t L, int p, F&& f) {
    constexpr int N = 16 / sizeof(T);
    const int64_t i0 = (int64_t)p * L, i1 = min(n, i0 + L);
    const bool vec = (i0 % N) == 0 && (((uintptr_t)(xr + i0)) & 15) == 0;
    int64_t i = i0;
    if (vec) {
        const int64_t nv = (i1 - i0) / N;
        for (int64_t c = threadIdx.x; c < nv; c += kSplitThreads) {
            const uint4 u = *reinterpret_cast<const uint4*>(xr + i0 + c * N);
            const uint32_t* w = reinterpret_cast<const uint32_t*>(&u);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                float v;
                if constexpr (sizeof(T) == 4) v = __uint_as_float(w[e]);
                else v = (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
                f(fkey(v), (uint32_t)(i0 + c * N + e));
            }
        }
        i = i0 + nv * N;
    }
    for (int64_t j = i + threadIdx.x; j < i1; j += kSplitThreads) f(fkey(elem(xr + j)), (uint32_t)j);
}

// Largest of v over the workgroup (kSplitThreads threads); every thread gets it.
__device__ __forceinline__ uint64_t block_max64(uint64_t v) {
    __shared__ uint64_t wmax[kSplitThreads / 64];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor64(v, m);
        v = o > v ? o : v;
    }
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t r = wmax[0];
#pragma unroll
    for (int w = 1; w < kSplitThreads / 64; ++w) r = wmax[w] > r ? wmax[w] : r;
    return r;
}

template <typename T>
__global__ __launch_bounds__(kSplitThreads) void argmax_part_kernel(const T* __restrict__ x, int64_t n, int64_t L,
                                                                    uint64_t* __restrict__ part) {
    const int p = blockIdx.x, row = blockIdx.y;
    uint64_t best = 0;
    for_slice<T>(x + (int64_t)row * n, n, L, p, [&](uint32_t key, uint32_t i) {
        const uint64_t kk = ((uint64_t)key << 32) | (uint32_t)~i;
        best = kk > best ? kk : best;
    });
    best = block_max64(best);
    if (threadIdx.x == 0) part[(int64_t)row * gridDim.x + p] = best;
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t* __restrict__ part, int P,
                                                          uint32_t* __restrict__ out) {
    // P <= kSplitMaxParts: every load is issued before the first compare
    const uint64_t* pr = part + (int64_t)blockIdx.x * P;
    uint64_t v[kSplitMaxParts / 64];
#pragma unroll
    for (int j = 0; j < kSplitMaxParts / 64; ++j) v[j] = 64 * j + (int)threadIdx.x < P ? pr[64 * j + threadIdx.x] : 0;
    uint64_t best = v[0];
#pragma unroll
    for (int j = 1; j < kSplitMaxParts / 64; ++j) best = v[j] > best ? v[j] : best;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor64(best, m);
        best = o > best ? o : best;
    }
    if (threadIdx.x == 0) out[blockIdx.x] = ~(uint32_t)best;
}

// Per-row block of the top-k workspace: the candidate count, the P slice
// maxima, then kCand candidates (8-byte aligned).
__host__ __device__ __forceinline__ int64_t topk_cand_offset(int P) { return ((4 + 4 * (int64_t)P + 7) / 8) * 8; }
__host__ __device__ __forceinline__ int64_t topk_row_bytes(int P) { return topk_cand_offset(P) + 8 * (int64_t)kCand; }

__global__ __launch_bounds__(kSplitThreads) void topk_max_kernel(const float* __restrict__ x, int64_t n, int64_t L,
                                                                 uint8_t* __restrict__ ws) {
    const int p = blockIdx.x, P = gridDim.x, row = blockIdx.y;
    uint32_t* hdr = reinterpret_cast<uint32_t*>(ws + (int64_t)row * topk_row_bytes(P));
    uint64_t best = 0;
    for_slice<float>(x + (int64_t)row * n, n, L, p, [&](uint32_t key, uint32_t) {
        best = key > best ? key : best;
    });
    best = block_max64(best);
    if (threadIdx.x == 0) {
        hdr[1 + p] = (uint32_t)best;
        if (p == 0) hdr[0] = 0u;  // the candidate count, for the next kernel
    }
}

// A lower bound of the k-th largest of the P (<= kSplitMaxParts) keys
// m[0..P), by one wave: the largest t with at least k keys >= t, bit by bit
// over the top 24 bits only (t's low 8 bits are 0).  It lies within the k-th
// largest key's 24-bit prefix (2^-15 of its value), so it admits at most the
// few extra keys that share that prefix (none for logits widened from bf16),
// in three quarters of the steps of the exact search.  (A 16-bit prefix,
// 2^-7 of the value, takes the same time here but lets a row whose values
// crowd near the k-th overflow the candidate list.)
__device__ __forceinline__ uint32_t kth_largest_wave(const uint32_t* m, int P, int k, int lane) {
    uint32_t v[kSplitMaxParts / 64];
#pragma unroll
    for (int j = 0; j < kSplitMaxParts / 64; ++j) v[j] = 64 * j + lane < P ? m[64 * j + lane] : 0u;
    uint32_t t = 0;
    for (int bit = 31; bit >= 8; --bit) {
        const uint32_t c = t | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kSplitMaxParts / 64; ++j) cnt += __popcll(__ballot(v[j] >= c));
        if (cnt >= k) t = c;
    }
    return t;
}

__global__ __launch_bounds__(kSplitThreads) void topk_collect_kernel(const float* __restrict__ x, int64_t n, int64_t L,
                                                                     int k, uint8_t* __restrict__ ws) {
    const int p = blockIdx.x, P = gridDim.x, row = blockIdx.y;
    const int lane = threadIdx.x & 63;
    uint8_t* rb = ws + (int64_t)row * topk_row_bytes(P);
    uint32_t* hdr = reinterpret_cast<uint32_t*>(rb);
    uint64_t* cand = reinterpret_cast<uint64_t*>(rb + topk_cand_offset(P));
    const float* xr = x + (int64_t)row * n;
    const int64_t i0 = (int64_t)p * L, i1 = min(n, i0 + L);
    const bool vec = (i0 % 4) == 0 && (((uintptr_t)(xr + i0)) & 15) == 0;
    const int64_t nv = vec ? (i1 - i0) / 4 : 0;
    // this thread's first 16 bytes of the slice, in flight while t is computed
    const int64_t c0 = threadIdx.x;
    const float4 first = c0 < nv ? *reinterpret_cast<const float4*>(xr + i0 + 4 * c0) : make_float4(0.f, 0.f, 0.f, 0.f);
    __shared__ uint32_t s_t;
    if (threadIdx.x < 64) {
        const uint32_t tw = kth_largest_wave(hdr + 1, P, k, lane);
        if (lane == 0) s_t = tw;
    }
    __syncthreads();
    const uint32_t t = s_t;
    auto take = [&](uint32_t key, uint32_t i) __attribute__((always_inline)) {
        const bool tk = key >= t;
        const uint64_t b = __ballot(tk);
        if (b == 0) return;  // uniform per wave
        uint32_t base = 0;
        const int leader = __ffsll((unsigned long long)b) - 1;
        if (lane == leader) base = atomicAdd(&hdr[0], (uint32_t)__popcll(b));
        base = __shfl(base, leader);
        const uint32_t slot = base + (uint32_t)__popcll(b & ((1ull << lane) - 1ull));
        if (tk && slot < (uint32_t)kCand) cand[slot] = ((uint64_t)key << 32) | (uint32_t)~i;
    };
    for (int64_t c = c0; c < nv; c += kSplitThreads) {
        const float4 v = c == c0 ? first : *reinterpret_cast<const float4*>(xr + i0 + 4 * c);
        const uint32_t i = (uint32_t)(i0 + 4 * c);
        take(fkey(v.x), i);
        take(fkey(v.y), i + 1);
        take(fkey(v.z), i + 2);
        take(fkey(v.w), i + 3);
    }
    for (int64_t j = i0 + 4 * nv + threadIdx.x; j < i1; j += kSplitThreads) take(fkey(xr[j]), (uint32_t)j);
}

__global__ __launch_bounds__(kThreads) void topk_final_kernel(const float* __restrict__ x, int64_t n, int k, int P,
                                                              const uint8_t* __restrict__ ws,
                                                              uint32_t* __restrict__ out) {
    static_assert(kThreads <= kCand, "one candidate slot per thread");
    const int row = blockIdx.x;
    const uint8_t* rb = ws + (int64_t)row * topk_row_bytes(P);
    const uint64_t* src = reinterpret_cast<const uint64_t*>(rb + topk_cand_offset(P));
    // this thread's first slot is loaded beside the count, not after it (the
    // slots past the count hold stale keys and are dropped)
    const uint64_t first = src[threadIdx.x];
    const uint32_t count = *reinterpret_cast<const uint32_t*>(rb);
    uint32_t* out_row = out + (int64_t)row * k;
    if (count > (uint32_t)kCand) {  // uniform: long runs of equal values
        topk_block(x + (int64_t)row * n, n, k, out_row);
        return;
    }
    __shared__ uint64_t cand[kCand];
    // the list padded to a multiple of 8 with 0, which is below every
    // candidate (the low word ~index is never 0)
    const uint32_t count8 = (count + 7u) & ~7u;
    if (threadIdx.x < count) cand[threadIdx.x] = first;
    else if (threadIdx.x < count8) cand[threadIdx.x] = 0;
    for (uint32_t i = threadIdx.x + kThreads; i < count; i += kThreads) cand[i] = src[i];
    __syncthreads();
    if (count <= (uint32_t)kThreads) {
        // Up to one candidate per thread: its rank is the number of larger
        // candidates (the keys are distinct: the index is part of them), read
        // back from LDS as broadcasts, 8 loads in flight, by the waves that
        // hold candidates only; ranks below k are the answer, in order.
        if (threadIdx.x < count) {
            uint32_t rank = 0;
            for (uint32_t q = 0; q < count8; q += 8) {
                uint64_t w[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) w[e] = cand[q + e];
#pragma unroll
                for (int e = 0; e < 8; ++e) rank += w[e] > first ? 1u : 0u;
            }
            if (rank < (uint32_t)k) out_row[rank] = ~(uint32_t)first;
        }
    } else {
        sort_candidates(cand, count, k, out_row);
    }
}

// Slices of a row for the split path: P workgroups of L elements (L a whole
// number of 16-byte chunks), P = 0 when the row is taken whole.
struct Split {
    int P;
    int64_t L;
};

// Slices per row: one row takes every CU (256 slices); more rows share the
// chip, argmax about 2048 workgroups in all, top-k about 4096 with at least
// 128 slices a row (the k-th largest slice max is the candidate bound, and with
// P close to k it falls to the row's smallest slice maxima: the candidates
// overflow).  Slices hold at least 512 entries.  Graph replay, 151936 entries:
// argmax 1 row 4.98 us at 148 slices or 256, 32 rows 9.76 -> 7.22 us at 64;
// top-64 1 row 11.49 -> 10.29 us at 256, 32 rows 21.85 us at 148, 21.26 at 74.
Split split_of(int64_t rows, int64_t n, bool topk) {
    if (rows > kSplitMaxRows || n < kSplitMinN) return {0, 0};
    int64_t P = (topk ? 4096 : 2048) / rows;
    if (topk && P < 2 * kSplitMinParts) P = 2 * kSplitMinParts;
    if (P > n / 512) P = n / 512;
    P = P < kSplitMinParts ? kSplitMinParts : (P > kSplitMaxParts ? kSplitMaxParts : P);
    int64_t L = (n + P - 1) / P;
    L = (L + 7) / 8 * 8;
    const int64_t used = (n + L - 1) / L;  // non-empty slices
    if (used < kSplitMinParts) return {0, 0};
    return {(int)used, L};
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

extern "C" size_t crane_hip_select_workspace_bytes(int64_t rows, int64_t n) {
    if (rows <= 0 || n <= 0) return 0;
    // the larger of the two plans' needs (either may run the single pass)
    const Split sa = split_of(rows, n, false), st = split_of(rows, n, true);
    const int64_t arg = sa.P ? rows * sa.P * 8 : 0, top = st.P ? rows * topk_row_bytes(st.P) : 0;
    return (size_t)(arg > top ? arg : top);
}

extern "C" int crane_hip_argmax_ws(const void* logits, int64_t rows, int64_t n, int dtype, void* workspace,
                                   size_t ws_bytes, uint32_t* out_idx, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (rows < 0 || n <= 0 || n > 0x7fffffffLL || rows > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (rows == 0) return CRANE_HIP_OK;
    const Split sp = split_of(rows, n, false);
    if (sp.P == 0) return crane_hip_argmax(logits, rows, n, dtype, out_idx, stream);
    if (!logits || !out_idx) return CRANE_HIP_E_INVALID;
    if (!workspace || ws_bytes < crane_hip_select_workspace_bytes(rows, n) || ((uintptr_t)workspace & 15))
        return CRANE_HIP_E_CAPACITY;
    hipStream_t st = (hipStream_t)stream;
    uint64_t* part = (uint64_t*)workspace;
    const dim3 grid((unsigned)sp.P, (unsigned)rows);
    if (dtype == CRANE_HIP_F32)
        hipLaunchKernelGGL(argmax_part_kernel<float>, grid, dim3(kSplitThreads), 0, st, (const float*)logits, n, sp.L,
                           part);
    else
        hipLaunchKernelGGL(argmax_part_kernel<bf16_t>, grid, dim3(kSplitThreads), 0, st, (const bf16_t*)logits, n,
                           sp.L, part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(64), 0, st, part, sp.P, out_idx);
    return launch_status(hipGetLastError());
}

extern "C" int crane_hip_topk_ws(const float* x, int64_t rows, int64_t n, int k, void* workspace, size_t ws_bytes,
                                 uint32_t* out_idx, void* stream) {
    if (rows < 0 || n <= 0 || n > 0x7fffffffLL || rows > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (k < 1 || k > CRANE_TOPK_MAX || (int64_t)k > n) return CRANE_HIP_E_INVALID;
    if (rows == 0) return CRANE_HIP_OK;
    const Split sp = split_of(rows, n, true);
    if (sp.P == 0) return crane_hip_topk(x, rows, n, k, out_idx, stream);
    if (!x || !out_idx) return CRANE_HIP_E_INVALID;
    if (!workspace || ws_bytes < crane_hip_select_workspace_bytes(rows, n) || ((uintptr_t)workspace & 15))
        return CRANE_HIP_E_CAPACITY;
    hipStream_t st = (hipStream_t)stream;
    uint8_t* ws = (uint8_t*)workspace;
    const dim3 grid((unsigned)sp.P, (unsigned)rows);
    hipLaunchKernelGGL(topk_max_kernel, grid, dim3(kSplitThreads), 0, st, x, n, sp.L, ws);
    hipLaunchKernelGGL(topk_collect_kernel, grid, dim3(kSplitThreads), 0, st, x, n, sp.L, k, ws);
    hipLaunchKernelGGL(topk_final_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, x, n, k, sp.P,
                       (const uint8_t*)ws, out_idx);
    return launch_status(hipGetLastError());
}
