// common.h -- shared device helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/crane_hip.h"

namespace crane {

constexpr int kHeadDim = 128;

typedef uint16_t bf16_t;  // raw bf16 bits in memory

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_v;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_v;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_v;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_v;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(bf16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even f32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    __bf16 b = (__bf16)f;
    return __builtin_bit_cast(bf16_t, b);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_v v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// Crane's SiLU, g / (1 + exp(-g)) in f32 (fused_ops.cu:104-126): one
// definition for the row kernel and the gated GEMM epilogue, so both round
// the same value.
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Element type traits: f32 and bf16 storage, f32 arithmetic.
template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float load(const float* p) { return *p; }
    static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
    static __device__ __forceinline__ float load(const bf16_t* p) { return bf16_to_f32(*p); }
    static __device__ __forceinline__ void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// Load / store 4 consecutive elements as float.
__device__ __forceinline__ void load4(const float* p, float (&v)[4]) {
    float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ __forceinline__ void load4(const bf16_t* p, float (&v)[4]) {
    uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_lo(t.x); v[1] = bf16_hi(t.x); v[2] = bf16_lo(t.y); v[3] = bf16_hi(t.y);
}
__device__ __forceinline__ void store4(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store4(bf16_t* p, const float (&v)[4]) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

// Load 8 consecutive elements as float.
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    float4 a = *reinterpret_cast<const float4*>(p);
    float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load8(const bf16_t* p, float (&v)[8]) {
    uint4 t = *reinterpret_cast<const uint4*>(p);
    v[0] = bf16_lo(t.x); v[1] = bf16_hi(t.x); v[2] = bf16_lo(t.y); v[3] = bf16_hi(t.y);
    v[4] = bf16_lo(t.z); v[5] = bf16_hi(t.z); v[6] = bf16_lo(t.w); v[7] = bf16_hi(t.w);
}

// Store 8 consecutive elements.
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void store8(bf16_t* p, const float (&v)[8]) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
}

// Rounding to the storage type after a candle op: identity for f32,
// round-to-nearest-even bf16 for bf16 (half::bf16 arithmetic rounds every op).
template <typename T> __device__ __forceinline__ float rt(float x);
template <> __device__ __forceinline__ float rt<float>(float x) { return x; }
// bf16: v_cvt_pk_bf16_f32 with a zero low half leaves the rounded value in the
// high half, i.e. already an f32 (one VALU instruction; the compiler's own
// form rounds into the low half and shifts it up).  The compiler does not
// insert wait states for an instruction written as inline assembly: after a
// transcendental (v_exp_f32, v_sqrt_f32, ...) a VALU read of its result needs
// one, so the s_nop 0 is part of the form.
template <> __device__ __forceinline__ float rt<bf16_t>(float x) {
    float r;
    asm("s_nop 0\n\tv_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
    return r;
}

// x / d rounded to nearest as IEEE division rounds it, from r = 1 / d (one
// correctly rounded reciprocal per divisor): q0 = x r, the remainder
// e = x - q0 d is exact in one FMA, and q0 + e r rounded is the correctly
// rounded quotient (Markstein's theorem for round-to-nearest binary
// arithmetic) while d is finite and nonzero and nothing over- or underflows.
// Three instructions instead of the division's ten; callers keep the division
// for divisors outside that range.
__device__ __forceinline__ float div_by(float x, float d, float r) {
    const float q0 = x * r;
    const float e = __builtin_fmaf(-q0, d, x);
    return __builtin_fmaf(e, r, q0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// ---- wave64 reductions with DPP (no LDS)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a DPP row; every lane gets the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x124>(x);  // row_ror:4
    x += dpp<0x128>(x);  // row_ror:8
    return x;
}


// Whole-wave max / sum with DPP: reduce each 16-lane row, fold the rows with
// row_bcast:15 / row_bcast:31 into lane 63, and broadcast it with readlane.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float x, float identity) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, identity),
                                                                 __builtin_bit_cast(int, x), CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x128>(v));
    v = fmaxf(v, dpp_rows<0x142, 0xa>(v, -INFINITY));  // row_bcast:15 into rows 1, 3
    v = fmaxf(v, dpp_rows<0x143, 0xc>(v, -INFINITY));  // row_bcast:31 into rows 2, 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += dpp_rows<0x142, 0xa>(v, 0.f);
    v += dpp_rows<0x143, 0xc>(v, 0.f);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Where row j of (sequence b, kv head kvh) of the K or V cache lives.
// offset() is the element offset of the row inside its buffer, or -1 when the
// row is past the sequence's capacity or its page id is outside the pool
// (such a row is never read or written).
//
// Dense: Crane's contiguous [B, Hkv, cap, D] buffers.
struct DenseRows {
    static constexpr bool kPaged = false;
    int64_t cap;
    __device__ __forceinline__ int64_t offset(int b, int Hkv, int kvh, int64_t j) const {
        if (j < 0 || j >= cap) return -1;
        return (((int64_t)b * Hkv + kvh) * cap + j) * kHeadDim;
    }
};
// Paged: pools [n_pages, Hkv, page_rows, D]; row j of sequence b is row
// j % page_rows of page table[b * stride + j / page_rows].
struct PagedRows {
    static constexpr bool kPaged = true;
    const int32_t* table;
    int64_t stride;
    int64_t n_pages;
    int page_rows;
    __device__ __forceinline__ int64_t offset(int b, int Hkv, int kvh, int64_t j) const {
        if (j < 0 || j >= stride * page_rows) return -1;
        // The table is read-only for the kernel's lifetime: read it through
        // the constant address space, so a wave-uniform lookup is a scalar load.
        typedef const __attribute__((address_space(4))) int32_t* table_t;
        const int64_t page = ((table_t)table)[b * stride + j / page_rows];
        if (page < 0 || page >= n_pages) return -1;
        return ((page * Hkv + kvh) * page_rows + j % page_rows) * kHeadDim;
    }
};

}  // namespace crane

// Host-side helpers shared by the launchers.
namespace crane {
inline int launch_status(hipError_t e) { return e == hipSuccess ? CRANE_HIP_OK : CRANE_HIP_E_LAUNCH; }
// The device a launch on `stream` runs on: the stream's own device, or the
// current device for the null stream.  -1 when the runtime cannot tell.
inline int stream_device(hipStream_t stream) {
    int dev = -1;
    if (stream) {
        if (hipStreamGetDevice(stream, &dev) != hipSuccess) return -1;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return -1;
    }
    return dev;
}
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline int elem_size(int dtype) { return dtype == CRANE_HIP_F32 ? 4 : 2; }
inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
// Round-to-nearest-even f32 -> bf16 value (finite inputs), as half::bf16::from_f32.
inline float host_round_bf16(float f) {
    const uint32_t u = f32_bits(f);
    return bits_f32((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
}
// Host checks of a paged cache description: pools [n_pages, Hkv, page_rows, D]
// and a block table of `stride` page ids per sequence.
inline int check_paged(int64_t n_pages, int page_rows, const int32_t* table, int64_t stride, int Hkv) {
    if (n_pages <= 0 || page_rows <= 0 || page_rows % CRANE_HIP_PAGE_ALIGN != 0 || stride <= 0 || !table)
        return CRANE_HIP_E_INVALID;
    if (n_pages > 0x7fffffffLL || stride > 0x7fffffffLL / page_rows) return CRANE_HIP_E_INVALID;
    if (Hkv > 0 && n_pages > ((int64_t)1 << 62) / ((int64_t)Hkv * page_rows * kHeadDim)) return CRANE_HIP_E_INVALID;
    return CRANE_HIP_OK;
}
}  // namespace crane
