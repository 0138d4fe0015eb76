// rope.hip -- host-side builders of the RoPE cos/sin tables the fused append
// reads (built once per model, as Crane builds them at load).
//
// The arithmetic follows the reference step by step, on the host CPU, so the
// tables are bit-identical to Crane's:
//   qwen3/modeling.rs:117-139 (RotaryEmbedding::new): inv_freq[i] =
//     1.0f32 / (base^(2i/dim) computed in f64, converted to f32); positions as
//     f32; freqs = positions x inv_freq, a k=1 matmul (one f32 product per
//     entry); cos/sin of the f32 angle (Rust's f32::cos/sin call the C
//     library's cosf/sinf on Linux);
//   hunyuan_dense/modeling.rs:202-219: the NTK-alpha base
//     theta * alpha^(dim/(dim-2)) in f64, then the same steps;
//   qwen3/modeling.rs:857-864: the f32 tables cast to the model dtype
//     (bf16: round to nearest even);
//   qwen25/qwen2.rs:47-64 (candle-transformers qwen2): inv_freq and the
//     positions cast to the model dtype before the product, the product
//     rounded to it, cos/sin computed in f32 and rounded to it.
#include <math.h>
#include <string.h>

#include "common.h"

namespace crane {
namespace {

// Round-to-nearest-even f32 -> bf16 bits (finite values), as half::bf16::from_f32.
inline uint16_t bf16_bits(float f) { return (uint16_t)(f32_bits(host_round_bf16(f)) >> 16); }

inline void put(void* dst, size_t i, float v, int dtype) {
    if (dtype == CRANE_HIP_BF16)
        static_cast<uint16_t*>(dst)[i] = bf16_bits(v);
    else
        static_cast<float*>(dst)[i] = v;
}

inline float in_dtype(float v, int dtype) { return dtype == CRANE_HIP_BF16 ? host_round_bf16(v) : v; }

int check_tables(int dim, int64_t max_pos, int dtype, const void* c, const void* s) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (dim <= 0 || dim % 2 != 0 || max_pos < 0 || max_pos > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    if (max_pos > 0 && (!c || !s)) return CRANE_HIP_E_INVALID;
    return CRANE_HIP_OK;
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" int crane_hip_rope_tables(int dim, double theta, double alpha, int64_t max_pos, int dtype, void* cos_out,
                                     void* sin_out) {
    int rc = check_tables(dim, max_pos, dtype, cos_out, sin_out);
    if (rc) return rc;
    if (!(theta > 0.0) || !isfinite(theta) || !(alpha >= 0.0) || !isfinite(alpha)) return CRANE_HIP_E_INVALID;
    const int half = dim / 2;
    const double base = alpha > 0.0 ? theta * pow(alpha, (double)dim / ((double)dim - 2.0)) : theta;
    float inv[512];
    if (half > 512) return CRANE_HIP_E_INVALID;
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / (float)pow(base, (double)(2 * i) / (double)dim);
    for (int64_t p = 0; p < max_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float f = (float)p * inv[i];
            put(cos_out, (size_t)p * half + i, in_dtype(cosf(f), dtype), dtype);
            put(sin_out, (size_t)p * half + i, in_dtype(sinf(f), dtype), dtype);
        }
    return CRANE_HIP_OK;
}

extern "C" int crane_hip_rope_tables_qwen2(int dim, double theta, int64_t max_pos, int dtype, void* cos_out,
                                           void* sin_out) {
    int rc = check_tables(dim, max_pos, dtype, cos_out, sin_out);
    if (rc) return rc;
    if (!(theta > 0.0) || !isfinite(theta)) return CRANE_HIP_E_INVALID;
    const int half = dim / 2;
    float inv[512];
    if (half > 512) return CRANE_HIP_E_INVALID;
    for (int i = 0; i < half; ++i) inv[i] = in_dtype(1.0f / (float)pow(theta, (double)(2 * i) / (double)dim), dtype);
    for (int64_t p = 0; p < max_pos; ++p) {
        const float pp = in_dtype((float)(uint32_t)p, dtype);
        for (int i = 0; i < half; ++i) {
            const float f = in_dtype(pp * inv[i], dtype);
            put(cos_out, (size_t)p * half + i, in_dtype(cosf(f), dtype), dtype);
            put(sin_out, (size_t)p * half + i, in_dtype(sinf(f), dtype), dtype);
        }
    }
    return CRANE_HIP_OK;
}
