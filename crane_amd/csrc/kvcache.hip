// kvcache.hip -- host-side KV-cache manager (one layer's K/V pair) over the
// attention launchers; the C ABI is include/crane_kv.h.
//
// Mirrors Attention::update_kv_cache (qwen3/modeling.rs:313-370): rows are
// written in place while they fit; the first use allocates S + 256 rows and a
// full buffer is reallocated to (rows needed) + 256 with the valid rows copied
// over.  The batched-decode set-up and tear-down (setup_batch_decode /
// pad_and_stack_kv_caches :973-1030,1141-1200 and extract_batch_kv
// :1066-1102) become a stack of single-sequence caches into one batch cache
// with a length per sequence, and a copy of one sequence's rows back out: no
// padding, no mask, and the decode kernel reads each sequence's rows in place.
#include <algorithm>
#include <new>
#include <vector>

#include "common.h"
#include "../../include/crane_kv.h"

namespace crane {
namespace {

__global__ void add_lengths_kernel(int32_t* len, int B, int S) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) len[i] += S;
}

__global__ void starts_from_lengths_kernel(const int32_t* len, int32_t* start, int B, int S) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) start[i] = len[i] - S;
}

int hip_status(hipError_t e) { return e == hipSuccess ? CRANE_HIP_OK : CRANE_HIP_E_LAUNCH; }

}  // namespace

// One layer's cache: K and V buffers [B, Hkv, cap, D] and the valid rows of
// every sequence (host copy `len`, device copy `dev_len`).
class KvCache {
  public:
    KvCache(int B, int Hkv, int D, int dtype)
        : B_(B), Hkv_(Hkv), D_(D), dtype_(dtype), es_(elem_size(dtype)), len_(B, 0) {}
    ~KvCache() { release(); }
    KvCache(const KvCache&) = delete;
    KvCache& operator=(const KvCache&) = delete;

    int B() const { return B_; }
    int Hkv() const { return Hkv_; }
    int D() const { return D_; }
    int dtype() const { return dtype_; }
    int64_t cap() const { return cap_; }
    void* k() const { return k_; }
    void* v() const { return v_; }
    const int32_t* dev_len() const { return dev_len_; }
    const std::vector<int64_t>& len() const { return len_; }
    int64_t max_len() const { return len_.empty() ? 0 : *std::max_element(len_.begin(), len_.end()); }
    size_t row_bytes() const { return (size_t)D_ * es_; }
    uint64_t bytes() const { return k_ ? 2ull * (uint64_t)B_ * Hkv_ * cap_ * row_bytes() : 0; }

    bool same_shape(const KvCache& o) const { return Hkv_ == o.Hkv_ && D_ == o.D_ && dtype_ == o.dtype_; }

    // Device array of lengths, created on first need.
    int ensure_dev_len(hipStream_t st) {
        if (dev_len_) return CRANE_HIP_OK;
        if (hipMalloc(&dev_len_, sizeof(int32_t) * (size_t)std::max(B_, 1)) != hipSuccess) {
            dev_len_ = nullptr;
            return CRANE_HIP_E_LAUNCH;
        }
        return upload_lengths(st);
    }

    int upload_lengths(hipStream_t st) {
        std::vector<int32_t> h(len_.begin(), len_.end());
        if (h.empty()) return CRANE_HIP_OK;
        const int rc = hip_status(hipMemcpyAsync(dev_len_, h.data(), sizeof(int32_t) * h.size(),
                                                 hipMemcpyHostToDevice, st));
        if (rc) return rc;
        return hip_status(hipStreamSynchronize(st));  // h is a local staging buffer
    }

    // Replace the buffers by ones of `new_cap` rows, keeping the first `keep`
    // rows of every (sequence, head).
    int reallocate(int64_t new_cap, int64_t keep, hipStream_t st) {
        void *nk = nullptr, *nv = nullptr;
        const size_t bytes = (size_t)B_ * Hkv_ * new_cap * row_bytes();
        if (bytes > 0) {
            if (hipMalloc(&nk, bytes) != hipSuccess) return CRANE_HIP_E_LAUNCH;
            if (hipMalloc(&nv, bytes) != hipSuccess) {
                (void)hipFree(nk);
                return CRANE_HIP_E_LAUNCH;
            }
        }
        if (k_ && keep > 0 && B_ * Hkv_ > 0) {
            const size_t w = (size_t)keep * row_bytes();
            int rc = hip_status(hipMemcpy2DAsync(nk, new_cap * row_bytes(), k_, cap_ * row_bytes(), w,
                                                 (size_t)B_ * Hkv_, hipMemcpyDeviceToDevice, st));
            if (!rc)
                rc = hip_status(hipMemcpy2DAsync(nv, new_cap * row_bytes(), v_, cap_ * row_bytes(), w,
                                                 (size_t)B_ * Hkv_, hipMemcpyDeviceToDevice, st));
            if (!rc) rc = hip_status(hipStreamSynchronize(st));  // the old buffers are freed next
            if (rc) {
                (void)hipFree(nk);
                (void)hipFree(nv);
                return rc;
            }
        }
        free_buffers();
        k_ = nk;
        v_ = nv;
        cap_ = new_cap;
        return CRANE_HIP_OK;
    }

    int reserve(int64_t add, hipStream_t st) {
        if (add < 0) return CRANE_HIP_E_INVALID;
        const int64_t needed = max_len() + add;
        const int64_t new_cap = crane_kv_grown_capacity(cap_, needed);
        if (new_cap > 0x7fffffffLL) return CRANE_HIP_E_CAPACITY;
        if (new_cap == cap_ && (k_ || new_cap == 0)) return CRANE_HIP_OK;
        return reallocate(new_cap, max_len(), st);
    }

    // Lengths grow by S on the host and on the device.
    int grow_lengths(int S, hipStream_t st) {
        for (auto& l : len_) l += S;
        if (!dev_len_ || B_ == 0) return CRANE_HIP_OK;
        hipLaunchKernelGGL(add_lengths_kernel, dim3((B_ + 255) / 256), dim3(256), 0, st, dev_len_, B_, S);
        return launch_status(hipGetLastError());
    }

    int set_lengths(const int64_t* host_len, hipStream_t st) {
        for (int b = 0; b < B_; ++b)
            if (host_len[b] < 0 || host_len[b] > cap_) return CRANE_HIP_E_CAPACITY;
        len_.assign(host_len, host_len + B_);
        if (!dev_len_) return CRANE_HIP_OK;
        return upload_lengths(st);
    }

    // start[b] = len[b] - S on the device (prefill chunk starts).
    int chunk_starts(int S, hipStream_t st, const int32_t** out) {
        if (!dev_start_ && hipMalloc(&dev_start_, sizeof(int32_t) * (size_t)std::max(B_, 1)) != hipSuccess) {
            dev_start_ = nullptr;
            return CRANE_HIP_E_LAUNCH;
        }
        hipLaunchKernelGGL(starts_from_lengths_kernel, dim3((B_ + 255) / 256), dim3(256), 0, st, dev_len_, dev_start_,
                           B_, S);
        *out = dev_start_;
        return launch_status(hipGetLastError());
    }

    void release() {
        free_buffers();
        if (dev_len_) (void)hipFree(dev_len_);
        if (dev_start_) (void)hipFree(dev_start_);
        dev_len_ = nullptr;
        dev_start_ = nullptr;
    }

  private:
    void free_buffers() {
        if (k_) (void)hipFree(k_);
        if (v_) (void)hipFree(v_);
        k_ = v_ = nullptr;
        cap_ = 0;
    }

    int B_, Hkv_, D_, dtype_;
    size_t es_;
    int64_t cap_ = 0;
    void* k_ = nullptr;
    void* v_ = nullptr;
    int32_t* dev_len_ = nullptr;
    int32_t* dev_start_ = nullptr;
    std::vector<int64_t> len_;
};

}  // namespace crane

using crane::KvCache;

struct crane_kv {
    KvCache impl;
    crane_kv(int B, int Hkv, int D, int dtype) : impl(B, Hkv, D, dtype) {}
};

extern "C" int64_t crane_kv_grown_capacity(int64_t cap, int64_t needed) {
    if (cap < 0 || needed < 0) return -1;
    return needed <= cap ? cap : needed + CRANE_KV_ROOM;
}

extern "C" int crane_kv_create(int B, int Hkv, int D, int dtype, crane_kv** out) {
    if (!out) return CRANE_HIP_E_INVALID;
    *out = nullptr;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != crane::kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || B > 65535 || Hkv <= 0 || Hkv > 65535) return CRANE_HIP_E_INVALID;
    crane_kv* kv = new (std::nothrow) crane_kv(B, Hkv, D, dtype);
    if (!kv) return CRANE_HIP_E_INVALID;
    *out = kv;
    return CRANE_HIP_OK;
}

extern "C" void crane_kv_destroy(crane_kv* kv) { delete kv; }

extern "C" int crane_kv_reserve(crane_kv* kv, int64_t add_rows, void* stream) {
    if (!kv) return CRANE_HIP_E_INVALID;
    const hipStream_t st = (hipStream_t)stream;
    int rc = kv->impl.ensure_dev_len(st);
    return rc ? rc : kv->impl.reserve(add_rows, st);
}

extern "C" int crane_kv_update(crane_kv* kv, const void* k, const void* v, int S, void* stream) {
    if (!kv || S < 0) return CRANE_HIP_E_INVALID;
    KvCache& c = kv->impl;
    if (S == 0 || c.B() == 0) return CRANE_HIP_OK;
    if (!k || !v) return CRANE_HIP_E_INVALID;
    const hipStream_t st = (hipStream_t)stream;
    int rc = c.ensure_dev_len(st);
    if (!rc) rc = c.reserve(S, st);
    if (rc) return rc;
    const size_t rb = c.row_bytes(), w = (size_t)S * rb;
    for (int b = 0; b < c.B() && !rc; ++b) {
        const size_t dst = ((size_t)b * c.Hkv() * c.cap() + (size_t)c.len()[b]) * rb;
        const size_t src = (size_t)b * c.Hkv() * S * rb;
        rc = crane::hip_status(hipMemcpy2DAsync((uint8_t*)c.k() + dst, c.cap() * rb, (const uint8_t*)k + src, w, w,
                                                (size_t)c.Hkv(), hipMemcpyDeviceToDevice, st));
        if (!rc)
            rc = crane::hip_status(hipMemcpy2DAsync((uint8_t*)c.v() + dst, c.cap() * rb, (const uint8_t*)v + src, w,
                                                    w, (size_t)c.Hkv(), hipMemcpyDeviceToDevice, st));
    }
    return rc ? rc : c.grow_lengths(S, st);
}

extern "C" int crane_kv_append_qkv(crane_kv* kv, const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                   const void* k_norm_w, float eps, int order, const void* cos, const void* sin,
                                   int64_t cs_stride, int64_t table_rows, const int32_t* positions, void* q_out, int S,
                                   int Hq, void* stream) {
    if (!kv || S < 0 || Hq <= 0) return CRANE_HIP_E_INVALID;
    KvCache& c = kv->impl;
    if (S == 0 || c.B() == 0) return CRANE_HIP_OK;
    const hipStream_t st = (hipStream_t)stream;
    int rc = c.ensure_dev_len(st);
    if (!rc) rc = c.reserve(S, st);
    if (rc) return rc;
    rc = crane_hip_qknorm_rope_append(qkv, qkv_row_stride, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride,
                                      table_rows, positions, q_out, c.k(), c.v(), c.cap(), c.dev_len(),
                                      c.max_len() + S, c.B(), S, Hq, c.Hkv(), c.D(), c.dtype(), stream);
    return rc ? rc : c.grow_lengths(S, st);
}

extern "C" int crane_kv_decode(const crane_kv* kv, const void* q, int Hq, float scale, int score_mode, void* workspace,
                               size_t ws_bytes, void* out, void* stream) {
    if (!kv) return CRANE_HIP_E_INVALID;
    const KvCache& c = kv->impl;
    if (c.B() == 0) return CRANE_HIP_OK;
    if (!c.k() || !c.dev_len() || c.max_len() == 0) return CRANE_HIP_E_INVALID;
    return crane_hip_attn_decode(q, c.k(), c.v(), c.cap(), c.dev_len(), c.max_len(), c.B(), Hq, c.Hkv(), c.D(), scale,
                                 score_mode, workspace, ws_bytes, out, c.dtype(), stream);
}

extern "C" int crane_kv_prefill(const crane_kv* kv, const void* q, int Hq, int S, float scale, int flags, void* out,
                                void* stream) {
    if (!kv || S < 0) return CRANE_HIP_E_INVALID;
    KvCache& c = const_cast<crane_kv*>(kv)->impl;  // only the scratch start array is written
    if (c.B() == 0 || S == 0) return CRANE_HIP_OK;
    if (!c.k() || !c.dev_len()) return CRANE_HIP_E_INVALID;
    for (int64_t l : c.len())
        if (l < S) return CRANE_HIP_E_INVALID;  // every sequence must hold its S new rows
    const int32_t* start = nullptr;
    int rc = c.chunk_starts(S, (hipStream_t)stream, &start);
    if (rc) return rc;
    return crane_hip_attn_prefill(q, c.k(), c.v(), c.cap(), start, c.max_len() - S, c.B(), S, Hq, c.Hkv(), c.D(),
                                  scale, flags, out, c.dtype(), stream);
}

extern "C" int crane_kv_views(const crane_kv* kv, void** k, void** v, int64_t* cap, const int32_t** dev_len,
                              int64_t* host_len) {
    if (!kv) return CRANE_HIP_E_INVALID;
    const KvCache& c = kv->impl;
    if (k) *k = c.k();
    if (v) *v = c.v();
    if (cap) *cap = c.cap();
    if (dev_len) *dev_len = c.dev_len();
    if (host_len) std::copy(c.len().begin(), c.len().end(), host_len);
    return CRANE_HIP_OK;
}

extern "C" int crane_kv_set_lengths(crane_kv* kv, const int64_t* host_len, void* stream) {
    if (!kv || (!host_len && kv->impl.B() > 0)) return CRANE_HIP_E_INVALID;
    return kv->impl.set_lengths(host_len, (hipStream_t)stream);
}

extern "C" uint64_t crane_kv_bytes(const crane_kv* kv) { return kv ? kv->impl.bytes() : 0; }

extern "C" int crane_kv_stack(crane_kv* dst, const crane_kv* const* srcs, int n, int64_t extra_room, void* stream) {
    if (!dst || n < 0 || extra_room < 0 || (n > 0 && !srcs)) return CRANE_HIP_E_INVALID;
    KvCache& d = dst->impl;
    if (d.B() != n) return CRANE_HIP_E_INVALID;
    int64_t max_len = 0;
    for (int i = 0; i < n; ++i) {
        // dst is reallocated before the copies: a source that is dst itself would be lost
        if (!srcs[i] || srcs[i] == dst || srcs[i]->impl.B() != 1 || !d.same_shape(srcs[i]->impl))
            return CRANE_HIP_E_INVALID;
        max_len = std::max(max_len, srcs[i]->impl.len()[0]);
    }
    const hipStream_t st = (hipStream_t)stream;
    int rc = d.ensure_dev_len(st);
    if (!rc) rc = d.reallocate(std::max<int64_t>(max_len + extra_room, 1), 0, st);
    if (rc) return rc;
    const size_t rb = d.row_bytes();
    std::vector<int64_t> lens(n);
    for (int i = 0; i < n && !rc; ++i) {
        const KvCache& s = srcs[i]->impl;
        lens[i] = s.len()[0];
        if (lens[i] == 0) continue;
        const size_t dst_off = (size_t)i * d.Hkv() * d.cap() * rb;
        rc = crane::hip_status(hipMemcpy2DAsync((uint8_t*)d.k() + dst_off, d.cap() * rb, s.k(), s.cap() * rb,
                                                lens[i] * rb, (size_t)d.Hkv(), hipMemcpyDeviceToDevice, st));
        if (!rc)
            rc = crane::hip_status(hipMemcpy2DAsync((uint8_t*)d.v() + dst_off, d.cap() * rb, s.v(), s.cap() * rb,
                                                    lens[i] * rb, (size_t)d.Hkv(), hipMemcpyDeviceToDevice, st));
    }
    return rc ? rc : d.set_lengths(lens.data(), st);
}

extern "C" int crane_kv_extract(const crane_kv* batch, int i, crane_kv* dst, void* stream) {
    if (!batch || !dst || dst == batch) return CRANE_HIP_E_INVALID;
    const KvCache& s = batch->impl;
    KvCache& d = dst->impl;
    if (i < 0 || i >= s.B() || d.B() != 1 || !d.same_shape(s)) return CRANE_HIP_E_INVALID;
    const int64_t n = s.len()[i];
    const hipStream_t st = (hipStream_t)stream;
    int rc = d.ensure_dev_len(st);
    if (rc) return rc;
    if (d.cap() < n || !d.k()) {
        // extract_batch_kv hands back exactly the valid rows; the next append
        // then grows the buffer by the usual policy.
        rc = d.reallocate(std::max<int64_t>(n, 1), 0, st);
        if (rc) return rc;
    }
    if (n > 0) {
        const size_t rb = s.row_bytes();
        const size_t src_off = (size_t)i * s.Hkv() * s.cap() * rb;
        rc = crane::hip_status(hipMemcpy2DAsync(d.k(), d.cap() * rb, (const uint8_t*)s.k() + src_off, s.cap() * rb,
                                                n * rb, (size_t)s.Hkv(), hipMemcpyDeviceToDevice, st));
        if (!rc)
            rc = crane::hip_status(hipMemcpy2DAsync(d.v(), d.cap() * rb, (const uint8_t*)s.v() + src_off, s.cap() * rb,
                                                    n * rb, (size_t)s.Hkv(), hipMemcpyDeviceToDevice, st));
        if (rc) return rc;
    }
    const int64_t len = n;
    return d.set_lengths(&len, st);
}
