// pagedkv.hip -- paged KV-cache manager (one layer's K/V pools) over the paged
// attention launchers; the C ABI is include/crane_pkv.h.
//
// Crane keeps one contiguous [B, Hkv, cap, D] buffer per layer and sequence
// group (Attention::update_kv_cache, qwen3/modeling.rs:313-370) and copies
// whole caches to set up and tear down every batched-decode round
// (setup_batch_decode / pad_and_stack_kv_caches :973-1030, 1141-1200;
// extract_batch_kv :1066-1102).  Here rows live in fixed pages of a pool and a
// sequence is a list of page ids: appends fill the last page and then take a
// new one from the free list, and a batch is B rows of a block table, so no KV
// row is ever moved.  Page lists and lengths are kept on the host (the source
// of truth) and mirrored on the device for the current batch only: set_batch
// uploads them, and an append that opens new pages patches the device table
// with a kernel whose arguments carry the new entries (no host buffer, no
// synchronisation on the decode path).
#include <algorithm>
#include <new>
#include <vector>

#include "common.h"
#include "../../include/crane_pkv.h"

namespace crane {
namespace {

constexpr int kPatch = 64;  // table entries per patch launch
struct TablePatch {
    int n;
    int32_t idx[kPatch];
    int32_t val[kPatch];
};

__global__ void patch_table_kernel(int32_t* table, TablePatch p) {
    const int i = threadIdx.x;
    if (i < p.n) table[p.idx[i]] = p.val[i];
}

__global__ void pkv_add_lengths_kernel(int32_t* len, int B, int S) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) len[i] += S;
}

__global__ void pkv_starts_kernel(const int32_t* len, int32_t* start, int B, int S) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) start[i] = len[i] - S;
}

// Contiguous rows [B, Hkv, S, D] -> rows (start[b] or 0) + s of the pages.
// One thread moves 16 bytes; K and V together.
__global__ __launch_bounds__(256) void scatter_rows_kernel(const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
                                                           uint8_t* __restrict__ k_pool, uint8_t* __restrict__ v_pool,
                                                           PagedRows rows, const int32_t* __restrict__ start, int B,
                                                           int Hkv, int S, int row_bytes, int64_t n_chunks) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_chunks) return;
    const int cpr = row_bytes / 16;
    const int64_t row = t / cpr;
    const int chunk = (int)(t % cpr);
    const int s = (int)(row % S);
    const int kvh = (int)((row / S) % Hkv);
    const int b = (int)(row / ((int64_t)S * Hkv));
    const int64_t off = rows.offset(b, Hkv, kvh, (int64_t)(start ? start[b] : 0) + s);
    if (off < 0) return;
    const int64_t dst = off * (row_bytes / kHeadDim) + 16 * chunk;
    const int64_t src = row * row_bytes + 16 * chunk;
    *reinterpret_cast<uint4*>(k_pool + dst) = *reinterpret_cast<const uint4*>(k + src);
    *reinterpret_cast<uint4*>(v_pool + dst) = *reinterpret_cast<const uint4*>(v + src);
}

// Rows [0, len) of sequence (table row) 0 -> contiguous [Hkv, len, D].
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ k_pool,
                                                          const uint8_t* __restrict__ v_pool, uint8_t* __restrict__ k,
                                                          uint8_t* __restrict__ v, PagedRows rows, int Hkv, int64_t len,
                                                          int row_bytes, int64_t n_chunks) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_chunks) return;
    const int cpr = row_bytes / 16;
    const int64_t row = t / cpr;
    const int chunk = (int)(t % cpr);
    const int64_t j = row % len;
    const int kvh = (int)(row / len);
    const int64_t off = rows.offset(0, Hkv, kvh, j);
    const int64_t dst = row * row_bytes + 16 * chunk;
    uint4 zk = make_uint4(0, 0, 0, 0), zv = zk;
    if (off >= 0) {
        const int64_t src = off * (row_bytes / kHeadDim) + 16 * chunk;
        zk = *reinterpret_cast<const uint4*>(k_pool + src);
        zv = *reinterpret_cast<const uint4*>(v_pool + src);
    }
    *reinterpret_cast<uint4*>(k + dst) = zk;
    *reinterpret_cast<uint4*>(v + dst) = zv;
}

int hip_rc(hipError_t e) { return e == hipSuccess ? CRANE_HIP_OK : CRANE_HIP_E_LAUNCH; }

struct Seq {
    bool live = false;
    int64_t len = 0;
    std::vector<int32_t> pages;
};

}  // namespace

class PagedKv {
  public:
    PagedKv(int Hkv, int D, int dtype, int P, int64_t n_pages, int max_seqs, int max_pps)
        : Hkv_(Hkv), D_(D), dtype_(dtype), es_(elem_size(dtype)), P_(P), n_pages_(n_pages), max_seqs_(max_seqs),
          max_pps_(max_pps), seqs_(max_seqs) {}
    ~PagedKv() { release(); }
    PagedKv(const PagedKv&) = delete;
    PagedKv& operator=(const PagedKv&) = delete;

    int init() {
        const size_t pool = pool_bytes();
        if (hipMalloc(&k_pool_, pool) != hipSuccess || hipMalloc(&v_pool_, pool) != hipSuccess ||
            hipMalloc(&d_table_, sizeof(int32_t) * (size_t)max_seqs_ * max_pps_) != hipSuccess ||
            hipMalloc(&d_len_, sizeof(int32_t) * (size_t)max_seqs_) != hipSuccess ||
            hipMalloc(&d_start_, sizeof(int32_t) * (size_t)max_seqs_) != hipSuccess ||
            hipMalloc(&d_one_, sizeof(int32_t) * (size_t)max_pps_) != hipSuccess) {
            release();
            return CRANE_HIP_E_LAUNCH;
        }
        free_.reserve((size_t)n_pages_);
        for (int64_t p = n_pages_ - 1; p >= 0; --p) free_.push_back((int32_t)p);
        return CRANE_HIP_OK;
    }

    size_t row_bytes() const { return (size_t)D_ * es_; }
    size_t pool_bytes() const { return (size_t)n_pages_ * Hkv_ * P_ * row_bytes(); }
    uint64_t bytes() const { return 2ull * pool_bytes(); }
    int64_t free_pages() const { return (int64_t)free_.size(); }
    int B() const { return (int)batch_.size(); }
    int Hkv() const { return Hkv_; }
    int D() const { return D_; }
    int dtype() const { return dtype_; }

    bool live(int id) const { return id >= 0 && id < max_seqs_ && seqs_[id].live; }
    bool in_batch(int id) const { return std::find(batch_.begin(), batch_.end(), id) != batch_.end(); }
    int64_t len(int id) const { return live(id) ? seqs_[id].len : -1; }
    int64_t max_len() const {
        int64_t m = 0;
        for (int id : batch_) m = std::max(m, seqs_[id].len);
        return m;
    }
    PagedRows batch_rows() const { return PagedRows{d_table_, max_pps_, n_pages_, P_}; }

    int seq_add(int* id) {
        for (int i = 0; i < max_seqs_; ++i)
            if (!seqs_[i].live) {
                seqs_[i].live = true;
                seqs_[i].len = 0;
                seqs_[i].pages.clear();
                *id = i;
                return CRANE_HIP_OK;
            }
        return CRANE_HIP_E_CAPACITY;
    }

    int seq_free(int id) {
        if (!live(id) || in_batch(id)) return CRANE_HIP_E_INVALID;
        Seq& s = seqs_[id];
        for (auto it = s.pages.rbegin(); it != s.pages.rend(); ++it) free_.push_back(*it);
        s = Seq();
        return CRANE_HIP_OK;
    }

    int set_batch(const int* ids, int B, hipStream_t st) {
        if (B < 0 || B > max_seqs_ || (B > 0 && !ids)) return CRANE_HIP_E_INVALID;
        std::vector<char> seen((size_t)max_seqs_, 0);
        for (int b = 0; b < B; ++b) {
            if (!live(ids[b]) || seen[ids[b]]) return CRANE_HIP_E_INVALID;
            seen[ids[b]] = 1;
        }
        batch_.assign(ids, ids + B);
        if (B == 0) return CRANE_HIP_OK;
        std::vector<int32_t> table((size_t)B * max_pps_, -1), lens((size_t)B);
        for (int b = 0; b < B; ++b) {
            const Seq& s = seqs_[ids[b]];
            std::copy(s.pages.begin(), s.pages.end(), table.begin() + (size_t)b * max_pps_);
            lens[b] = (int32_t)s.len;
        }
        int rc = hip_rc(hipMemcpyAsync(d_table_, table.data(), sizeof(int32_t) * table.size(), hipMemcpyHostToDevice, st));
        if (!rc) rc = hip_rc(hipMemcpyAsync(d_len_, lens.data(), sizeof(int32_t) * lens.size(), hipMemcpyHostToDevice, st));
        if (!rc) rc = hip_rc(hipStreamSynchronize(st));  // the staging vectors go out of scope
        if (rc) batch_.clear();
        return rc;
    }

    // Pages for S more rows in every batch sequence: checked first, then taken
    // from the free list, and the new device table entries patched in.
    // added[b] counts the pages batch sequence b received (for unreserve).
    int reserve(int64_t S, hipStream_t st, std::vector<int>* added = nullptr) {
        if (S < 0) return CRANE_HIP_E_INVALID;
        int64_t need_total = 0;
        for (int id : batch_) {
            const Seq& s = seqs_[id];
            const int64_t need = (s.len + S + P_ - 1) / P_;
            if (need > max_pps_ || s.len + S > 0x7fffffffLL) return CRANE_HIP_E_CAPACITY;
            need_total += std::max<int64_t>(0, need - (int64_t)s.pages.size());
        }
        if (need_total > (int64_t)free_.size()) return CRANE_HIP_E_CAPACITY;
        TablePatch patch;
        patch.n = 0;
        if (added) added->assign((size_t)B(), 0);
        for (int b = 0; b < B(); ++b) {
            Seq& s = seqs_[batch_[b]];
            const int64_t need = (s.len + S + P_ - 1) / P_;
            while ((int64_t)s.pages.size() < need) {
                if (added) ++(*added)[b];
                const int32_t page = free_.back();
                free_.pop_back();
                patch.idx[patch.n] = (int32_t)((int64_t)b * max_pps_ + (int64_t)s.pages.size());
                patch.val[patch.n] = page;
                ++patch.n;
                s.pages.push_back(page);
                if (patch.n == kPatch) {
                    const int rc = launch_patch(d_table_, patch, st);
                    if (rc) return rc;
                    patch.n = 0;
                }
            }
        }
        return patch.n ? launch_patch(d_table_, patch, st) : CRANE_HIP_OK;
    }

    // Give back the pages a reserve() took when the launch it was for was
    // rejected.  Their device table entries stay, past the sequences' page
    // counts, where no kernel reads them; the next reserve() overwrites them.
    void unreserve(const std::vector<int>& added) {
        for (int b = B() - 1; b >= 0; --b) {
            Seq& s = seqs_[batch_[b]];
            for (int i = 0; i < added[b]; ++i) {
                free_.push_back(s.pages.back());
                s.pages.pop_back();
            }
        }
    }

    int grow_lengths(int S, hipStream_t st) {
        for (int id : batch_) seqs_[id].len += S;
        if (batch_.empty()) return CRANE_HIP_OK;
        hipLaunchKernelGGL(pkv_add_lengths_kernel, dim3((B() + 255) / 256), dim3(256), 0, st, d_len_, B(), S);
        return launch_status(hipGetLastError());
    }

    int update(const void* k, const void* v, int S, hipStream_t st) {
        if (S < 0) return CRANE_HIP_E_INVALID;
        if (S == 0 || batch_.empty()) return CRANE_HIP_OK;
        if (!k || !v || !aligned16(k) || !aligned16(v)) return !k || !v ? CRANE_HIP_E_INVALID : CRANE_HIP_E_ALIGN;
        int rc = reserve(S, st);
        if (rc) return rc;
        rc = scatter(k, v, batch_rows(), d_len_, B(), S, st);
        return rc ? rc : grow_lengths(S, st);
    }

    int append_qkv(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w, const void* k_norm_w, float eps,
                   int order, const void* cos, const void* sin, int64_t cs_stride, int64_t table_rows,
                   const int32_t* positions, void* q_out, int S, int Hq, hipStream_t st) {
        if (S < 0 || Hq <= 0) return CRANE_HIP_E_INVALID;
        if (S == 0 || batch_.empty()) return CRANE_HIP_OK;
        std::vector<int> added;
        int rc = reserve(S, st, &added);
        if (rc) return rc;
        rc = crane_hip_qknorm_rope_append_paged(qkv, qkv_row_stride, q_norm_w, k_norm_w, eps, order, cos, sin,
                                                cs_stride, table_rows, positions, q_out, k_pool_, v_pool_, n_pages_,
                                                P_, d_table_, max_pps_, d_len_, B(), S, Hq, Hkv_, D_, dtype_, st);
        if (rc) {  // rejected arguments: nothing ran, the pages go back
            unreserve(added);
            return rc;
        }
        return grow_lengths(S, st);
    }

    int decode(const void* q, int Hq, float scale, int score_mode, void* ws, size_t ws_bytes, void* out,
               hipStream_t st) const {
        if (batch_.empty()) return CRANE_HIP_OK;
        const int64_t m = max_len();
        if (m == 0) return CRANE_HIP_E_INVALID;
        return crane_hip_attn_decode_paged(q, k_pool_, v_pool_, n_pages_, P_, d_table_, max_pps_, d_len_, m, B(), Hq,
                                           Hkv_, D_, scale, score_mode, ws, ws_bytes, out, dtype_, st);
    }

    int prefill(const void* q, int Hq, int S, float scale, int flags, void* out, hipStream_t st) {
        if (S < 0) return CRANE_HIP_E_INVALID;
        if (batch_.empty() || S == 0) return CRANE_HIP_OK;
        for (int id : batch_)
            if (seqs_[id].len < S) return CRANE_HIP_E_INVALID;  // every sequence holds its S new rows
        hipLaunchKernelGGL(pkv_starts_kernel, dim3((B() + 255) / 256), dim3(256), 0, st, d_len_, d_start_, B(), S);
        const int rc = launch_status(hipGetLastError());
        if (rc) return rc;
        return crane_hip_attn_prefill_paged(q, k_pool_, v_pool_, n_pages_, P_, d_table_, max_pps_, d_start_,
                                            max_len() - S, B(), S, Hq, Hkv_, D_, scale, flags, out, dtype_, st);
    }

    int read_seq(int id, void* k, void* v, hipStream_t st) {
        if (!live(id)) return CRANE_HIP_E_INVALID;
        const Seq& s = seqs_[id];
        if (s.len == 0) return CRANE_HIP_OK;
        if (!k || !v) return CRANE_HIP_E_INVALID;
        if (!aligned16(k) || !aligned16(v)) return CRANE_HIP_E_ALIGN;
        int rc = upload_one(s.pages, st);
        if (rc) return rc;
        const int64_t n_chunks = (int64_t)Hkv_ * s.len * (int64_t)(row_bytes() / 16);
        hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t*)k_pool_, (const uint8_t*)v_pool_, (uint8_t*)k, (uint8_t*)v, one_rows(), Hkv_,
                           s.len, (int)row_bytes(), n_chunks);
        return launch_status(hipGetLastError());
    }

    int write_seq(int id, const void* k, const void* v, int64_t len, hipStream_t st) {
        if (!live(id) || in_batch(id) || len < 0) return CRANE_HIP_E_INVALID;
        if (len > 0 && (!k || !v)) return CRANE_HIP_E_INVALID;
        if (len > 0 && (!aligned16(k) || !aligned16(v))) return CRANE_HIP_E_ALIGN;
        Seq& s = seqs_[id];
        const int64_t need = (len + P_ - 1) / P_;
        if (need > max_pps_ || len > 0x7fffffffLL) return CRANE_HIP_E_CAPACITY;
        if (need - (int64_t)s.pages.size() > (int64_t)free_.size()) return CRANE_HIP_E_CAPACITY;
        while ((int64_t)s.pages.size() > need) {
            free_.push_back(s.pages.back());
            s.pages.pop_back();
        }
        while ((int64_t)s.pages.size() < need) {
            s.pages.push_back(free_.back());
            free_.pop_back();
        }
        s.len = len;
        if (len == 0) return CRANE_HIP_OK;
        const int rc = upload_one(s.pages, st);
        return rc ? rc : scatter(k, v, one_rows(), nullptr, 1, len, st);
    }

    void views(void** k, void** v, const int32_t** table, int64_t* stride, const int32_t** dlen) const {
        if (k) *k = k_pool_;
        if (v) *v = v_pool_;
        if (table) *table = d_table_;
        if (stride) *stride = max_pps_;
        if (dlen) *dlen = d_len_;
    }

  private:
    static int launch_patch(int32_t* table, const TablePatch& p, hipStream_t st) {
        hipLaunchKernelGGL(patch_table_kernel, dim3(1), dim3(kPatch), 0, st, table, p);
        return launch_status(hipGetLastError());
    }

    PagedRows one_rows() const { return PagedRows{d_one_, max_pps_, n_pages_, P_}; }

    // One sequence's page ids into the single-row table d_one_.
    int upload_one(const std::vector<int32_t>& pages, hipStream_t st) {
        std::vector<int32_t> row((size_t)max_pps_, -1);
        std::copy(pages.begin(), pages.end(), row.begin());
        int rc = hip_rc(hipMemcpyAsync(d_one_, row.data(), sizeof(int32_t) * row.size(), hipMemcpyHostToDevice, st));
        return rc ? rc : hip_rc(hipStreamSynchronize(st));  // `row` is a local staging buffer
    }

    int scatter(const void* k, const void* v, const PagedRows& rows, const int32_t* start, int B, int64_t S,
                hipStream_t st) {
        const int64_t n_chunks = (int64_t)B * Hkv_ * S * (int64_t)(row_bytes() / 16);
        if ((n_chunks + 255) / 256 > 0x7fffffffLL || S > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
        hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t*)k, (const uint8_t*)v, (uint8_t*)k_pool_, (uint8_t*)v_pool_, rows, start, B,
                           Hkv_, (int)S, (int)row_bytes(), n_chunks);
        return launch_status(hipGetLastError());
    }

    void release() {
        for (void* p : {k_pool_, v_pool_, (void*)d_table_, (void*)d_len_, (void*)d_start_, (void*)d_one_})
            if (p) (void)hipFree(p);
        k_pool_ = v_pool_ = nullptr;
        d_table_ = d_len_ = d_start_ = d_one_ = nullptr;
    }

    int Hkv_, D_, dtype_;
    size_t es_;
    int P_;
    int64_t n_pages_;
    int max_seqs_, max_pps_;
    void* k_pool_ = nullptr;
    void* v_pool_ = nullptr;
    int32_t* d_table_ = nullptr;  // current batch: B rows of max_pps_ page ids
    int32_t* d_len_ = nullptr;    // current batch lengths
    int32_t* d_start_ = nullptr;  // prefill chunk starts
    int32_t* d_one_ = nullptr;    // one sequence's page ids (read_seq / write_seq)
    std::vector<int32_t> free_;
    std::vector<Seq> seqs_;
    std::vector<int> batch_;
};

}  // namespace crane

using crane::PagedKv;

struct crane_pkv {
    PagedKv impl;
    crane_pkv(int Hkv, int D, int dtype, int P, int64_t n_pages, int max_seqs, int max_pps)
        : impl(Hkv, D, dtype, P, n_pages, max_seqs, max_pps) {}
};

extern "C" int crane_pkv_create(int Hkv, int D, int dtype, int page_rows, int64_t n_pages, int max_seqs,
                                int max_pages_per_seq, crane_pkv** out) {
    if (!out) return CRANE_HIP_E_INVALID;
    *out = nullptr;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != crane::kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (Hkv <= 0 || Hkv > 65535 || max_seqs <= 0 || max_seqs > 65535 || max_pages_per_seq <= 0)
        return CRANE_HIP_E_INVALID;
    int32_t dummy = 0;  // the table pointer is not known yet; only the sizes are checked here
    const int rc = crane::check_paged(n_pages, page_rows, &dummy, max_pages_per_seq, Hkv);
    if (rc) return rc;
    crane_pkv* p = new (std::nothrow) crane_pkv(Hkv, D, dtype, page_rows, n_pages, max_seqs, max_pages_per_seq);
    if (!p) return CRANE_HIP_E_INVALID;
    const int irc = p->impl.init();
    if (irc) {
        delete p;
        return irc;
    }
    *out = p;
    return CRANE_HIP_OK;
}

extern "C" void crane_pkv_destroy(crane_pkv* pkv) { delete pkv; }

extern "C" int crane_pkv_seq_add(crane_pkv* pkv, int* seq_id) {
    if (!pkv || !seq_id) return CRANE_HIP_E_INVALID;
    return pkv->impl.seq_add(seq_id);
}

extern "C" int crane_pkv_seq_free(crane_pkv* pkv, int seq_id) {
    return pkv ? pkv->impl.seq_free(seq_id) : CRANE_HIP_E_INVALID;
}

extern "C" int64_t crane_pkv_seq_len(const crane_pkv* pkv, int seq_id) { return pkv ? pkv->impl.len(seq_id) : -1; }

extern "C" int64_t crane_pkv_free_pages(const crane_pkv* pkv) { return pkv ? pkv->impl.free_pages() : 0; }

extern "C" uint64_t crane_pkv_bytes(const crane_pkv* pkv) { return pkv ? pkv->impl.bytes() : 0; }

extern "C" int crane_pkv_set_batch(crane_pkv* pkv, const int* seq_ids, int B, void* stream) {
    return pkv ? pkv->impl.set_batch(seq_ids, B, (hipStream_t)stream) : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_update(crane_pkv* pkv, const void* k, const void* v, int S, void* stream) {
    return pkv ? pkv->impl.update(k, v, S, (hipStream_t)stream) : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_append_qkv(crane_pkv* pkv, const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                    const void* k_norm_w, float eps, int order, const void* cos, const void* sin,
                                    int64_t cs_stride, int64_t table_rows, const int32_t* positions, void* q_out,
                                    int S, int Hq, void* stream) {
    if (!pkv) return CRANE_HIP_E_INVALID;
    return pkv->impl.append_qkv(qkv, qkv_row_stride, q_norm_w, k_norm_w, eps, order, cos, sin, cs_stride, table_rows,
                                positions, q_out, S, Hq, (hipStream_t)stream);
}

extern "C" int crane_pkv_decode(const crane_pkv* pkv, const void* q, int Hq, float scale, int score_mode,
                                void* workspace, size_t ws_bytes, void* out, void* stream) {
    return pkv ? pkv->impl.decode(q, Hq, scale, score_mode, workspace, ws_bytes, out, (hipStream_t)stream)
               : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_prefill(crane_pkv* pkv, const void* q, int Hq, int S, float scale, int flags, void* out,
                                 void* stream) {
    return pkv ? pkv->impl.prefill(q, Hq, S, scale, flags, out, (hipStream_t)stream) : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_read_seq(crane_pkv* pkv, int seq_id, void* k, void* v, void* stream) {
    return pkv ? pkv->impl.read_seq(seq_id, k, v, (hipStream_t)stream) : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_write_seq(crane_pkv* pkv, int seq_id, const void* k, const void* v, int64_t len,
                                   void* stream) {
    return pkv ? pkv->impl.write_seq(seq_id, k, v, len, (hipStream_t)stream) : CRANE_HIP_E_INVALID;
}

extern "C" int crane_pkv_views(const crane_pkv* pkv, void** k_pool, void** v_pool, const int32_t** block_table,
                               int64_t* table_stride, const int32_t** dev_len) {
    if (!pkv) return CRANE_HIP_E_INVALID;
    pkv->impl.views(k_pool, v_pool, block_table, table_stride, dev_len);
    return CRANE_HIP_OK;
}
