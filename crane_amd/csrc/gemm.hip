// gemm.hip -- the QKV / o_proj projections (candle Linear, y = x W^T + b) on
// hipBLASLt; C ABI in include/crane_gemm.h.
//
// Row-major y[M, N] = x[M, K] W[N, K]^T is, in hipBLASLt's column-major
// terms, D[N, M] = op(A) B with A = W viewed as [K, N] (transposed: N x K),
// B = x viewed as [K, M], D = y viewed as [N, M]; the bias vector (one value
// per row of D, i.e. per output feature) is the BIAS epilogue.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <new>
#include <tuple>

#include "common.h"
#include "../../include/crane_gemm.h"

namespace crane {
namespace {

constexpr size_t kDefaultWorkspace = 32u << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

void free_plan(Plan& p) {
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) (void)hipblasLtMatrixLayoutDestroy(p.d);
    p = Plan();
}

}  // namespace

class Gemm {
  public:
    ~Gemm() {
        for (auto& kv : plans_) free_plan(kv.second);
        if (ws_) (void)hipFree(ws_);
        if (handle_) (void)hipblasLtDestroy(handle_);
    }

    int init(size_t ws_bytes) {
        ws_bytes_ = ws_bytes ? ws_bytes : kDefaultWorkspace;
        if (hipblasLtCreate(&handle_) != HIPBLAS_STATUS_SUCCESS) {
            handle_ = nullptr;
            return CRANE_HIP_E_LAUNCH;
        }
        if (hipMalloc(&ws_, ws_bytes_) != hipSuccess) {
            ws_ = nullptr;
            return CRANE_HIP_E_LAUNCH;
        }
        return CRANE_HIP_OK;
    }

    // Serialised per context: the plan map, and the bias pointer set on a
    // shared descriptor just before the call that reads it.
    int linear(const void* x, const void* w, const void* bias, void* y, int64_t M, int64_t N, int64_t K, int dtype,
               hipStream_t st) {
        std::lock_guard<std::mutex> lock(mu_);
        Plan* p = nullptr;
        int rc = plan(M, N, K, dtype, bias != nullptr, &p);
        if (rc) return rc;
        if (bias && hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                                    sizeof(bias)) != HIPBLAS_STATUS_SUCCESS)
            return CRANE_HIP_E_LAUNCH;
        const float alpha = 1.0f, beta = 0.0f;
        const hipblasStatus_t s = hipblasLtMatmul(handle_, p->desc, &alpha, w, p->a, x, p->b, &beta, y, p->d, y, p->d,
                                                  &p->algo, ws_, ws_bytes_, st);
        return s == HIPBLAS_STATUS_SUCCESS ? CRANE_HIP_OK : CRANE_HIP_E_LAUNCH;
    }

  private:
    // The descriptors and the heuristic's algorithm for one shape, built once.
    int plan(int64_t M, int64_t N, int64_t K, int dtype, bool has_bias, Plan** out) {
        const auto key = std::make_tuple(M, N, K, dtype, has_bias);
        auto it = plans_.find(key);
        if (it != plans_.end()) {
            *out = &it->second;
            return CRANE_HIP_OK;
        }
        Plan p;
        const hipDataType t = dtype == CRANE_HIP_F32 ? HIP_R_32F : HIP_R_16BF;
        const hipblasOperation_t opA = HIPBLAS_OP_T, opB = HIPBLAS_OP_N;
        const hipblasLtEpilogue_t epi = has_bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
        bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opA, sizeof(opA)) ==
                       HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opB, sizeof(opB)) ==
                       HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ==
                       HIPBLAS_STATUS_SUCCESS;
        if (ok && has_bias) {
            const int32_t bt = t;
            ok = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) ==
                 HIPBLAS_STATUS_SUCCESS;
        }
        ok = ok && hipblasLtMatrixLayoutCreate(&p.a, t, K, N, K) == HIPBLAS_STATUS_SUCCESS;  // W as [K, N], ld K
        ok = ok && hipblasLtMatrixLayoutCreate(&p.b, t, K, M, K) == HIPBLAS_STATUS_SUCCESS;  // x as [K, M], ld K
        ok = ok && hipblasLtMatrixLayoutCreate(&p.d, t, N, M, N) == HIPBLAS_STATUS_SUCCESS;  // y as [N, M], ld N
        hipblasLtMatmulPreference_t pref = nullptr;
        ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
        const uint64_t wsb = ws_bytes_;
        ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                         sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulHeuristicResult_t res{};
        int found = 0;
        ok = ok && hipblasLtMatmulAlgoGetHeuristic(handle_, p.desc, p.a, p.b, p.d, p.d, pref, 1, &res, &found) ==
                       HIPBLAS_STATUS_SUCCESS;
        if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
        if (!ok || found < 1 || res.state != HIPBLAS_STATUS_SUCCESS) {
            free_plan(p);
            return CRANE_HIP_E_INVALID;  // no algorithm for this shape / dtype
        }
        p.algo = res.algo;
        auto ins = plans_.emplace(key, p);
        *out = &ins.first->second;
        return CRANE_HIP_OK;
    }

    std::mutex mu_;
    hipblasLtHandle_t handle_ = nullptr;
    void* ws_ = nullptr;
    size_t ws_bytes_ = 0;
    std::map<std::tuple<int64_t, int64_t, int64_t, int, bool>, Plan> plans_;
};

}  // namespace crane

struct crane_gemm {
    crane::Gemm impl;
};

extern "C" int crane_gemm_create(size_t workspace_bytes, crane_gemm** out) {
    if (!out) return CRANE_HIP_E_INVALID;
    *out = nullptr;
    crane_gemm* g = new (std::nothrow) crane_gemm();
    if (!g) return CRANE_HIP_E_INVALID;
    const int rc = g->impl.init(workspace_bytes);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return CRANE_HIP_OK;
}

extern "C" void crane_gemm_destroy(crane_gemm* g) { delete g; }

extern "C" int crane_gemm_linear(crane_gemm* g, const void* x, const void* w, const void* bias, void* y, int64_t M,
                                 int64_t N, int64_t K, int dtype, void* stream) {
    if (!g) return CRANE_HIP_E_INVALID;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (M < 0 || N <= 0 || K <= 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
        return CRANE_HIP_E_INVALID;
    if (M == 0) return CRANE_HIP_OK;
    if (!x || !w || !y) return CRANE_HIP_E_INVALID;
    if (!crane::aligned16(x) || !crane::aligned16(w) || !crane::aligned16(y) || (bias && !crane::aligned16(bias)))
        return CRANE_HIP_E_ALIGN;
    return g->impl.linear(x, w, bias, y, M, N, K, dtype, (hipStream_t)stream);
}
