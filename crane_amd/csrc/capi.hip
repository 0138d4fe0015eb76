// capi.hip -- status strings and build identification for the C ABI.
#include "common.h"

extern "C" const char* crane_hip_strerror(int code) {
    switch (code) {
        case CRANE_HIP_OK: return "ok";
        case CRANE_HIP_E_INVALID: return "invalid argument (size, stride or null pointer)";
        case CRANE_HIP_E_DTYPE: return "unsupported dtype (expected f32 or bf16)";
        case CRANE_HIP_E_HEAD_DIM: return "unsupported head_dim (expected 128)";
        case CRANE_HIP_E_GQA: return "num_heads is not a multiple of num_kv_heads";
        case CRANE_HIP_E_CAPACITY: return "KV cache capacity exceeded";
        case CRANE_HIP_E_WORKSPACE: return "workspace missing, misaligned or too small";
        case CRANE_HIP_E_LAUNCH: return "HIP kernel launch failed";
        case CRANE_HIP_E_ALIGN: return "pointer or stride not 16-byte aligned";
        default: return "unknown crane_hip status";
    }
}

extern "C" const char* crane_hip_version(void) { return "crane_hip 2 gfx950"; }
