// decode.hip -- batched split-KV (flash-decoding) attention for one new token
// per sequence over Crane's [B, Hkv, cap, D] KV cache (gfx950).
//
// Replaces the GQA-grouped decode SDPA of qwen3/modeling.rs:432-467 (and
// hunyuan_dense/modeling.rs:575-608, qwen2.rs:185-206) together with the
// batched-decode right-aligned padding + -1e9 mask of qwen3/modeling.rs:1118-1200:
// sequence b reads exactly its own kv_len[b] rows, which gives the same
// softmax as padding with masked columns (exp(-1e9 - m) == 0 in f32).
//
// Kernel 1 (decode_chunk_kernel): one workgroup (4 waves) per (chunk of 256
// keys -- 512 when the longest sequence passes 12288 -- kv head group, sequence).  The G query heads sharing the kv head are
// done together, so each K/V row is read from HBM once for the whole GQA
// group, and no MFMA is used: the path is HBM-bound.  Rows are read with
// bounds-checked buffer loads (rows past the sequence end read as zero, so no
// branch guards a load).
//   A. scores: 8 lanes read one K row (two 16-byte loads each, 16 dims per
//      lane; a wave covers 8 rows per load pair), each lane does the dot
//      product of its 16 dims with v_dot2_f32_bf16 for all G heads, and a
//      3-step DPP butterfly inside the 8 lanes completes it.  Lane a of the 8
//      reads bytes [16a, 16a+16) and [128+16a, 128+16a+16) of the row, so
//      each load instruction covers whole 128-byte lines (the q dims follow
//      the same map); pieces 32 bytes apart would touch every line twice,
//      which measured 5% (8 heads: 9%) slower.
//   B. the chunk's softmax statistics per head (max m and sum l of the
//      bf16-rounded exp2(s - m), log2 domain), computed once per (head, key)
//      with DPP wave reductions; probabilities go to LDS as packed bf16 pairs
//      of consecutive keys.
//   C. P @ V: 16 lanes read a V row (8 dims each); two consecutive rows are
//      interleaved with v_perm so v_dot2_f32_bf16 takes (p_j, p_j+1) x
//      (v_j, v_j+1) per dim.  The 4 row groups of a wave are summed with lane
//      permutes and the 4 waves through LDS.
// A sequence that fits one chunk is normalised and written directly; longer
// ones leave a partial row and its (m, l) in the workspace: for bf16 the row
// normalised by the chunk's sum l and stored in bf16 (half the bytes the
// merge reads; sums stay in f32), for f32 the unnormalised f32 row.
// Kernel 2 (decode_merge_kernel): the log-sum-exp merge of those partials.
//
// Scores follow the candle path the caller names (score_mode).  The
// GQA-grouped decode (qwen3/modeling.rs:432-467 for n_rep > 1,
// hunyuan_dense/modeling.rs:575-608) pre-scales q in the model dtype (affine
// with the scale converted to T, :440-441) and rounds q@K^T to T.  The
// standard SDPA (qwen3/modeling.rs:485-488 for n_rep == 1, every qwen2.rs
// decode :196-197) rounds q@K^T to T, then multiplies by the T scale and
// rounds again.  Either way every rounding point of the scores is reproduced.
// A sequence of at most kChunkShort (256) keys also gets candle's
// softmax_last_dim chain in T (candle-nn ops.rs, CPU softmax: e =
// T(exp(T(s - max))), sum in f32 rounded to T, p = T(e / sum), then p @ V with
// f32 accumulation): the whole row is in one workgroup, so the exact chain
// costs nothing measurable.  The choice follows the sequence's own length.
// Longer sequences keep the split-KV form (unnormalised bf16 p per chunk, f32
// sums); its last bits depend on the chunk size, 512 keys when the launch's
// max_kv passes kLongKv, else 256, so a long sequence's output can differ in
// the last bits between batches with different max_kv.
#include <mutex>
#include <type_traits>

#include "common.h"

namespace crane {
namespace {

constexpr int kChunkShort = 256;  // keys per workgroup
constexpr int kChunkLong = 512;   // keys per workgroup when max_kv > kLongKv
constexpr int kLongKv = 12288;
constexpr int kThreads = 256;     // 4 waves
constexpr int kMaxSplits = 4096;  // chunks per sequence the merge handles
constexpr int kKRows = 4;         // K rows in flight per lane in phase A (of 8)
constexpr int kMaxGroup = 8;    // q heads handled per workgroup

// Sum over the 4 rows (16-lane groups) of the wave; every lane gets the total.
__device__ __forceinline__ float rows4_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a), __builtin_bit_cast(bf16x2_v, b), c, false);
}

// Buffer resource over `bytes` bytes from `base`: loads outside it return 0,
// so rows past the end of a chunk need no branch (gfx9 raw buffer, dword3 = 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));
// K and V rows are read once per decode step: non-temporal loads (cache
// policy bit 1, `nt`) stream them without displacing other data; measured on
// this access pattern they raise the read rate by about 14%.
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
    const u32x4_v v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum over the 8 lanes of a DPP half-row; every lane gets the total.
__device__ __forceinline__ float row8_sum(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror
    return x;
}

template <typename T, int G, int CH>
struct DecodeShared {
    static constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
    float s[G][CH];                                      // raw scores
    uint32_t p[kBf16 ? CH / 2 * G : 1];                  // bf16 probability pairs (key 2m, 2m+1) per head
    float pf[kBf16 ? 1 : CH * G];                        // f32 probabilities
    __attribute__((aligned(16))) float red[4][G][kHeadDim];  // per-wave partial rows
    float ml[G][2];                                      // chunk (max, sum) per head
};

// One work item: chunk c (keys [c CH, (c+1) CH)) of sequence b for the
// G q heads of head group gi.  Writes the normalised rows when the sequence
// fits one chunk, otherwise the unnormalised partial and its (max, sum).
template <typename T, int G, int CH, class ROWS>
__device__ __forceinline__ void decode_item(
    DecodeShared<T, G, CH>& sm, const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
    const ROWS& rows, int L, int b, int gi, int c, int Hq, int Hkv, int n_rep, float scale, bool post, int nsplit,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, T* __restrict__ out) {
    constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
    constexpr int kVecA = 16 * (int)sizeof(T) / 16;  // 16-byte loads per lane per K row (16 dims)
    constexpr int kVecC = 8 * (int)sizeof(T) / 16;   // 16-byte loads per lane per V row (8 dims)
    constexpr int kStepsA = CH / 32;  // 8-key row steps per wave in phase A
    constexpr int kPairsC = CH / 32;  // key pairs per 16-lane group in phase C
    // V row pairs held in registers for C: all 8 of a 256-key chunk, or for 8
    // heads (whose accumulators take 64 VGPRs) and for 512-key chunks a ring of
    // 4 refilled as pairs are consumed.
    constexpr int kVRing = (G >= 8 || kPairsC > 8) ? 4 : kPairsC;
    const int sub_per_kv = n_rep / G;
    const int kvh = gi / sub_per_kv;
    const int h0 = kvh * n_rep + (gi % sub_per_kv) * G;  // first q head of this group
    const int j0 = c * CH;
    const int tid = threadIdx.x;
    if (j0 >= L) {  // uniform over the workgroup
        if (c == 0)  // an empty sequence attends to nothing: its rows are zero
            for (int e = tid; e < G * kHeadDim; e += kThreads)
                Elem<T>::store(out + ((int64_t)b * Hq + h0) * kHeadDim + e, 0.f);
        return;
    }
    const int n = min(CH, L - j0);
    const int lane = tid & 63, wave = tid >> 6;
    const int a8 = lane & 7, r8 = lane >> 3;     // phase A: 8 lanes per key, 16 dims per lane
    const int grp = lane >> 4, l16 = lane & 15;  // phase C: 16 lanes per key, 8 dims per lane
    auto& s_lds = sm.s;
    uint32_t* p_lds = sm.p;
    float* pf_lds = sm.pf;
    auto& red = sm.red;
    auto& ml = sm.ml;

    // Rows [j0, j0 + n) of this (sequence, kv head), contiguous in both
    // layouts (a page holds whole chunks); loads past them return 0, and so
    // do all of them for a page id outside the pool.
    const int64_t off = rows.offset(b, Hkv, kvh, j0);
    const int nbytes = off < 0 ? 0 : n * kHeadDim * (int)sizeof(T);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc + (off < 0 ? 0 : off), nbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vc + (off < 0 ? 0 : off), nbytes);
    constexpr int kRowBytes = kHeadDim * (int)sizeof(T);

    // q's pieces, then the first kKRows K row steps, are all issued before
    // any of them is used (the scheduling barrier keeps q's unpacking behind
    // the K loads), so q's round trip and the first K rows' overlap.
    // The lane's q dims are those of its K pieces: bytes [128 v + 16 a8, +16)
    // of the row.
    constexpr int kQPieces = 16 * (int)sizeof(T) / 16;  // 16-byte pieces per lane and head
    uint4 qraw[G][kQPieces];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const T* qr = q + ((int64_t)b * Hq + h0 + h) * kHeadDim;
#pragma unroll
        for (int v = 0; v < kQPieces; ++v)
            qraw[h][v] = *reinterpret_cast<const uint4*>(qr + (128 * v + 16 * a8) / (int)sizeof(T));
    }
    uint4 kr[kKRows][kVecA];
    auto k_load = [&](int step, int slot) __attribute__((always_inline)) {
        const int j = wave * (CH / 4) + step * 8 + r8;
#pragma unroll
        for (int v = 0; v < kVecA; ++v) kr[slot][v] = buf_load16(rk, j * kRowBytes + 128 * v + 16 * a8);
    };
#pragma unroll
    for (int t = 0; t < kKRows; ++t) k_load(t, t);
    __builtin_amdgcn_sched_barrier(0);

    // Grouped path: q_g = q * scale in T, for this lane's 16 dims of every head.
    // Standard path: q as is (q * 1 rounds to q itself).
    const float scale_t = rt<T>(scale);
    const float qmul = post ? 1.0f : scale_t;
    uint32_t qp[kBf16 ? G : 1][8];
    float qf[kBf16 ? 1 : G][16];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float x[16];
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&qraw[h][0]);
        if constexpr (kBf16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[2 * i] = bf16_lo(w[i]);
                x[2 * i + 1] = bf16_hi(w[i]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) qp[h][i] = pack_bf16x2(x[2 * i] * qmul, x[2 * i + 1] * qmul);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) qf[h][i] = __uint_as_float(w[i]) * qmul;
        }
    }
    // This lane's first V row pairs for C: ring slot t holds pair m =
    // w CH/8 + 4t + grp, rows 2m and 2m+1.  The first kVEarly slots are
    // issued during A's last steps, each as a K slot frees up (a V slot takes
    // the registers of a K slot), the others after A.
    uint4 vr[kVRing][2][kVecC];
    auto v_load = [&](int t) __attribute__((always_inline)) {
        const int m = wave * (CH / 8) + 4 * t + grp;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int v = 0; v < kVecC; ++v)
                vr[t][r][v] = buf_load16(rv, (2 * m + r) * kRowBytes + 16 * (kVecC * l16 + v));
    };
    constexpr int kVEarly = kKRows < kVRing ? kKRows : kVRing;

    // ---- A: raw scores q_g . k; wave w owns keys [w CH/4, (w+1) CH/4), 8 per
    // load instruction, through a ring of kKRows row steps, each refilled with
    // the step kKRows ahead as soon as it is used (no drain between groups)
#pragma unroll
    for (int step = 0; step < kStepsA; ++step) {
        const int t = step % kKRows;
        const int j = wave * (CH / 4) + step * 8 + r8;
        float acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float a = 0.f;
            if constexpr (kBf16) {
                const uint32_t* kw = reinterpret_cast<const uint32_t*>(&kr[t][0]);
#pragma unroll
                for (int i = 0; i < 8; ++i) a = dot2(qp[h][i], kw[i], a);
            } else {
                const float* kf = reinterpret_cast<const float*>(&kr[t][0]);
#pragma unroll
                for (int i = 0; i < 16; ++i) a += qf[h][i] * kf[i];
            }
            acc[h] = row8_sum(a);
        }
        float mine = acc[0];
#pragma unroll
        for (int h = 1; h < G; ++h) mine = a8 == h ? acc[h] : mine;
        if (a8 < G && j < n) s_lds[a8][j] = mine;
        if (step + kKRows < kStepsA) k_load(step + kKRows, t);
        else if (step + kKRows - kStepsA < kVEarly) v_load(step + kKRows - kStepsA);
    }

    // The rest of the V ring's first fill, in flight while B runs.
#pragma unroll
    for (int t = kVEarly; t < kVRing; ++t) v_load(t);
    __syncthreads();

    // ---- B: per-head chunk max and sum; probabilities to LDS
    const int n_chunks = (L + CH - 1) / CH;
    const bool single = n_chunks == 1;  // uniform: the whole row is in this workgroup
    // candle's exact chain for a row of at most kChunkShort keys, whatever the
    // chunk size: a sequence's arithmetic follows its own length, not the
    // launch's max_kv
    const bool exact = L <= kChunkShort;
    for (int h = wave; h < G; h += 4) {
        float sv[CH / 64];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < CH / 64; ++i) {
            const int j = lane + 64 * i;
            // the score as candle's T tensor holds it
            sv[i] = j < n ? (post ? rt<T>(rt<T>(s_lds[h][j]) * scale_t) : rt<T>(s_lds[h][j])) : -INFINITY;
            m = fmaxf(m, sv[i]);
        }
        m = wave_max(m);
        float l = 0.f;
        if (exact) {
            // candle's softmax_last_dim in T over the whole row
            float e[CH / 64];
#pragma unroll
            for (int i = 0; i < CH / 64; ++i) {
                const int j = lane + 64 * i;
                e[i] = j < n ? rt<T>(expf(rt<T>(sv[i] - m))) : 0.f;
                l += e[i];
            }
            l = rt<T>(wave_sum(l));
#pragma unroll
            for (int i = 0; i < CH / 64; ++i) {
                const int j = lane + 64 * i;
                const float p = rt<T>(e[i] / l);
                if constexpr (kBf16)
                    reinterpret_cast<bf16_t*>(p_lds)[((j >> 1) * G + h) * 2 + (j & 1)] = f32_to_bf16(p);
                else
                    pf_lds[j * G + h] = p;
            }
            l = 1.f;  // the probabilities are normalised
        } else {
            // log2 domain, unnormalised: p = exp2((s - m) log2 e), rounded to
            // bf16 for the P V product and summed as rounded
            m *= kLog2e;
#pragma unroll
            for (int i = 0; i < CH / 64; ++i) {
                const int j = lane + 64 * i;
                float p = j < n ? fast_exp2(__builtin_fmaf(sv[i], kLog2e, -m)) : 0.f;
                if constexpr (kBf16) {
                    const bf16_t pb = f32_to_bf16(p);
                    p = bf16_to_f32(pb);
                    reinterpret_cast<bf16_t*>(p_lds)[((j >> 1) * G + h) * 2 + (j & 1)] = pb;
                } else {
                    pf_lds[j * G + h] = p;
                }
                l += p;
            }
            l = wave_sum(l);
        }
        if (lane == 0) {
            ml[h][0] = m;
            ml[h][1] = l;
        }
    }
    __syncthreads();

    // ---- C: unnormalised P @ V over the chunk (rows past n were read as 0, p = 0)
    float o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) o[h][d] = 0.f;
#pragma unroll
    for (int t = 0; t < kPairsC; ++t) {
        const int m = wave * (CH / 8) + 4 * t + grp;
        if constexpr (kBf16) {
            // interleave rows 2m and 2m+1 per dim: (v_2m[d], v_2m+1[d])
            const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&vr[t % kVRing][0][0]);
            const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&vr[t % kVRing][1][0]);
            uint32_t vv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                vv[2 * i] = __builtin_amdgcn_perm(r1[i], r0[i], 0x05040100u);      // low halves
                vv[2 * i + 1] = __builtin_amdgcn_perm(r1[i], r0[i], 0x07060302u);  // high halves
            }
            if (t + kVRing < kPairsC) {  // refill the ring slot just consumed
                const int m2 = wave * (CH / 8) + 4 * (t + kVRing) + grp;
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int v = 0; v < kVecC; ++v)
                        vr[t % kVRing][r][v] = buf_load16(rv, (2 * m2 + r) * kRowBytes + 16 * (kVecC * l16 + v));
            }
            const uint32_t* pp = p_lds + m * G;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const uint32_t pr = pp[h];
#pragma unroll
                for (int d = 0; d < 8; ++d) o[h][d] = dot2(pr, vv[d], o[h][d]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const float* vf = reinterpret_cast<const float*>(&vr[t % kVRing][r][0]);
                const float* pp = pf_lds + (2 * m + r) * G;
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float p = pp[h];
#pragma unroll
                    for (int d = 0; d < 8; ++d) o[h][d] += p * vf[d];
                }
            }
            if (t + kVRing < kPairsC) {  // refill the ring slot just consumed
                const int m2 = wave * (CH / 8) + 4 * (t + kVRing) + grp;
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int v = 0; v < kVecC; ++v)
                        vr[t % kVRing][r][v] = buf_load16(rv, (2 * m2 + r) * kRowBytes + 16 * (kVecC * l16 + v));
            }
        }
    }
    // Sum the 4 row groups of the wave, then the 4 waves through LDS.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) o[h][d] = rows4_sum(o[h][d]);
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int d = 0; d < 8; d += 4)
                *reinterpret_cast<float4*>(&red[wave][h][8 * l16 + d]) =
                    make_float4(o[h][d], o[h][d + 1], o[h][d + 2], o[h][d + 3]);
    }
    __syncthreads();

    for (int e = tid; e < G * kHeadDim; e += kThreads) {
        const int h = e / kHeadDim, d = e % kHeadDim;
        const float v = red[0][h][d] + red[1][h][d] + red[2][h][d] + red[3][h][d];
        if (single)  // the whole sequence fits one chunk: finish here (exact: p was normalised, l = 1)
            Elem<T>::store(out + ((int64_t)b * Hq + h0 + h) * kHeadDim + d, exact ? v : v / ml[h][1]);
        else if constexpr (kBf16)  // bf16 partials are stored normalised by the chunk's sum (merge weight w l)
            reinterpret_cast<bf16_t*>(ws_o)[(((int64_t)b * Hq + h0 + h) * nsplit + c) * kHeadDim + d] =
                f32_to_bf16(v / ml[h][1]);
        else
            ws_o[(((int64_t)b * Hq + h0 + h) * nsplit + c) * kHeadDim + d] = v;
    }
    if (!single && tid < G) {
        float* dst = ws_ml + (((int64_t)b * Hq + h0 + tid) * nsplit + c) * 2;
        dst[0] = ml[tid][0];
        dst[1] = ml[tid][1];
    }
}

// Dispatch order: the chunk index is the slowest grid dimension, counted
// down: the workgroups past the shorter sequences' ends (which exit at once)
// are dispatched first instead of delaying the tail, the longest sequences'
// last chunks start earliest, and the last wave of workgroups is every
// sequence's full chunk 0 (c3 -1.2%, c5 -0.4% against counting up).
// grid: (groups, B, nsplit).
template <typename T, int G, int CH, class ROWS>
__global__ __launch_bounds__(kThreads) void decode_chunk_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, ROWS rows,
    const int32_t* __restrict__ kv_len, int max_kv, int Hq, int Hkv, int n_rep, float scale, int post, int nsplit,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, T* __restrict__ out) {
    __shared__ DecodeShared<T, G, CH> sm;
    const int c = (int)gridDim.z - 1 - (int)blockIdx.z;
    const int b = blockIdx.y;
    const int L = min(kv_len[b], max_kv);  // never read past the rows the host vouched for
    decode_item<T, G, CH, ROWS>(sm, q, kc, vc, rows, L, b, blockIdx.x, c, Hq, Hkv, n_rep, scale, post != 0, nsplit, ws_o,
                                ws_ml, out);
}

// Kernel 2: log-sum-exp merge of one (sequence, q head)'s partials.  Wave p
// is partition p: its lane l owns output dims 2l and 2l+1 for splits p,
// p + P, p + 2P, ... (one 4-byte load per split for bf16 partials, 8 bytes
// for f32).  Every first load is issued before kv_len is known: each lane
// loads its first kMergeRegs partials and each thread the (m, l) of split
// tid (indices clamped to the nsplit slots the workspace holds for the head;
// slots past the sequence's chunks hold stale values and are dropped by
// selects), so up to P * kMergeRegs splits cost one memory round trip.  The P
// partition sums meet in LDS.  Used for more than kMergeRegs splits.
constexpr int kMergeRegs = 16;
template <typename T, int CH, int P>
__global__ __launch_bounds__(64 * P) void decode_merge_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, const int32_t* __restrict__ kv_len,
    int max_kv, int Hq, int n_rep, int nsplit, T* __restrict__ out) {
    constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
    __shared__ float w_lds[kMaxSplits];
    __shared__ float red[P];
    __shared__ float2 part[P - 1][kHeadDim / 2];
    // grid (groups, B, G), the chunk kernel's (groups, B) with the group's G
    // heads last: workgroup ids then fall on the XCD that ran the head's
    // chunks (measured 0.5% at config 3, 1% at config 5).
    const int G = (int)gridDim.z, sub = n_rep / G, gi = (int)blockIdx.x, b = (int)blockIdx.y;
    const int bh = b * Hq + (gi / sub) * n_rep + (gi % sub) * G + (int)blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63, p = tid >> 6;
    const float* pm = ws_ml + (int64_t)bh * nsplit * 2;
    const float2* po = reinterpret_cast<const float2*>(ws_o + (int64_t)bh * nsplit * kHeadDim) + lane;
    const uint32_t* pob = reinterpret_cast<const uint32_t*>(reinterpret_cast<const bf16_t*>(ws_o) +
                                                            (int64_t)bh * nsplit * kHeadDim) + lane;
    auto partial_at = [&](int cc) {
        if constexpr (kBf16) {
            const uint32_t u = pob[(int64_t)cc * (kHeadDim / 2)];
            return make_float2(bf16_lo(u), bf16_hi(u));
        } else {
            return po[(int64_t)cc * (kHeadDim / 2)];
        }
    };
    constexpr int kWords = kBf16 ? 1 : 2;
    uint32_t raw[kMergeRegs][kWords];
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i) {
        const int64_t ci = min(p + P * i, nsplit - 1);
        if constexpr (kBf16) {
            raw[i][0] = pob[ci * (kHeadDim / 2)];
        } else {
            const float2 v = po[ci * (kHeadDim / 2)];
            raw[i][0] = __builtin_bit_cast(uint32_t, v.x);
            raw[i][kWords - 1] = __builtin_bit_cast(uint32_t, v.y);
        }
    }
    const float2 ml0 = reinterpret_cast<const float2*>(pm)[min(tid, nsplit - 1)];
    const int kvl = kv_len[b];
    // Uses of every loaded value ahead of the kv_len branch (see the wave merge).
    asm volatile("" ::"s"(kvl));
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i)
#pragma unroll
        for (int j = 0; j < kWords; ++j) asm volatile("" ::"v"(raw[i][j]));
    asm volatile("" ::"v"(ml0.x), "v"(ml0.y));
    const int L = min(kvl, max_kv);
    const int nc = (L + CH - 1) / CH;
    if (nc <= 1) return;  // written by the split kernel
    float mx = tid < nc ? ml0.x : -INFINITY;
    for (int cc = tid + 64 * P; cc < nc; cc += 64 * P) mx = fmaxf(mx, pm[2 * cc]);
    mx = wave_max(mx);
    if (lane == 0) red[p] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < P; ++w) M = fmaxf(M, red[w]);
    float den = 0.f;
    if (tid < nc) {
        const float w = fast_exp2(ml0.x - M);
        w_lds[tid] = kBf16 ? w * ml0.y : w;  // a normalised partial weighs w l
        den = w * ml0.y;
    }
    for (int cc = tid + 64 * P; cc < nc; cc += 64 * P) {
        const float w = fast_exp2(pm[2 * cc] - M);
        w_lds[cc] = kBf16 ? w * pm[2 * cc + 1] : w;
        den += w * pm[2 * cc + 1];
    }
    den = wave_sum(den);
    __syncthreads();  // w_lds complete; red[] reads of the max are done
    if (lane == 0) red[p] = den;
    __syncthreads();
    den = red[0];
#pragma unroll
    for (int w = 1; w < P; ++w) den += red[w];
    float n0 = 0.f, n1 = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i) {
        if (p + P * i < nc) {
            const float wc = w_lds[p + P * i];
            const float2 x = kBf16 ? make_float2(bf16_lo(raw[i][0]), bf16_hi(raw[i][0]))
                                   : make_float2(__builtin_bit_cast(float, raw[i][0]),
                                                 __builtin_bit_cast(float, raw[i][kWords - 1]));
            n0 += wc * x.x;
            n1 += wc * x.y;
        }
    }
    for (int cc = p + P * kMergeRegs; cc < nc; cc += P) {
        const float2 v = partial_at(cc);
        n0 += w_lds[cc] * v.x;
        n1 += w_lds[cc] * v.y;
    }
    if (p > 0) part[p - 1][lane] = make_float2(n0, n1);
    __syncthreads();
    if (p > 0) return;
#pragma unroll
    for (int q = 0; q < P - 1; ++q) {
        n0 += part[q][lane].x;
        n1 += part[q][lane].y;
    }
    T* o = out + (int64_t)bh * kHeadDim + 2 * lane;
    Elem<T>::store(o, n0 / den);
    Elem<T>::store(o + 1, n1 / den);
}

// Kernel 2 for up to kMergeRegs splits: one wave per (sequence, q head), four
// heads of a group per workgroup.  Lane l owns dims 2l and 2l+1 and lane c
// holds split c's (m, l), so the max and the denominator are DPP wave
// reductions and each split's weight reaches every lane by readlane: no LDS
// and no barrier.  Every load is issued before kv_len is known (indices
// clamped to the nsplit slots the workspace holds for the head; slots past
// the sequence's chunks hold stale values and are dropped by selects), so the
// merge costs one memory round trip instead of two.
// grid (groups, B, ceil(G / 4)), as the chunk kernel's (groups, B).
template <typename T, int CH>
__global__ __launch_bounds__(256) void decode_merge_wave_kernel(
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, const int32_t* __restrict__ kv_len,
    int max_kv, int Hq, int n_rep, int G, int nsplit, T* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int hh = (int)blockIdx.z * 4 + (threadIdx.x >> 6);
    if (hh >= G) return;  // whole waves
    const int sub = n_rep / G, gi = (int)blockIdx.x, b = (int)blockIdx.y;
    const int bh = b * Hq + (gi / sub) * n_rep + (gi % sub) * G + hh;
    const float* pm = ws_ml + (int64_t)bh * nsplit * 2;
    constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
    const float2* po = reinterpret_cast<const float2*>(ws_o + (int64_t)bh * nsplit * kHeadDim) + lane;
    const uint32_t* pob = reinterpret_cast<const uint32_t*>(reinterpret_cast<const bf16_t*>(ws_o) +
                                                            (int64_t)bh * nsplit * kHeadDim) + lane;
    // raw partial words: bf16 pairs (one word per split) or f32 pairs (two)
    constexpr int kWords = kBf16 ? 1 : 2;
    uint32_t raw[kMergeRegs][kWords];
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i) {
        const int ci = min(i, nsplit - 1);
        if constexpr (kBf16) {
            raw[i][0] = pob[ci * (kHeadDim / 2)];
        } else {
            const float2 v = po[ci * (kHeadDim / 2)];
            raw[i][0] = __builtin_bit_cast(uint32_t, v.x);
            raw[i][kWords - 1] = __builtin_bit_cast(uint32_t, v.y);
        }
    }
    const float2 ml = reinterpret_cast<const float2*>(pm)[min(lane, nsplit - 1)];
    const int kvl = kv_len[b];
    // Uses of every loaded value ahead of the kv_len branch: without them the
    // compiler sinks the loads below it, behind the kv_len load's round trip.
    asm volatile("" ::"s"(kvl));
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i)
#pragma unroll
        for (int j = 0; j < kWords; ++j) asm volatile("" ::"v"(raw[i][j]));
    asm volatile("" ::"v"(ml.x), "v"(ml.y));
    float2 x[kMergeRegs];
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i)
        x[i] = kBf16 ? make_float2(bf16_lo(raw[i][0]), bf16_hi(raw[i][0]))
                     : make_float2(__builtin_bit_cast(float, raw[i][0]), __builtin_bit_cast(float, raw[i][kWords - 1]));
    const int L = min(kvl, max_kv);
    const int nc = (L + CH - 1) / CH;
    if (nc <= 1) return;  // written by the split kernel
    const float m = lane < nc ? ml.x : -INFINITY;
    const float l = lane < nc ? ml.y : 0.f;
    const float M = wave_max(m);
    const float w = lane < nc ? fast_exp2(m - M) : 0.f;
    const float den = wave_sum(w * l);
    const float wn = kBf16 ? w * l : w;  // a normalised partial weighs w l
    float n0 = 0.f, n1 = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i) {
        if (i < nc) {
            const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wn), i));
            n0 += wi * x[i].x;
            n1 += wi * x[i].y;
        }
    }
    T* o = out + (int64_t)bh * kHeadDim + 2 * lane;
    Elem<T>::store(o, n0 / den);
    Elem<T>::store(o + 1, n1 / den);
}

int pick_group(int n_rep) {
    for (int g = kMaxGroup; g >= 1; --g)
        if (n_rep % g == 0) return g;
    return 1;
}

template <typename T, int G, int CH, class ROWS>
int launch_decode_g(const T* q, const T* kc, const T* vc, const ROWS& rows, const int32_t* kv_len, int max_kv,
                    int nsplit, int B, int Hq, int Hkv, float scale, int post, float* ws_o, float* ws_ml, T* out,
                    hipStream_t st) {
    const int n_rep = Hq / Hkv;
    const int groups = Hkv * (n_rep / G);
    const dim3 grid((unsigned)groups, (unsigned)B, (unsigned)nsplit);
    hipLaunchKernelGGL((decode_chunk_kernel<T, G, CH, ROWS>), grid, dim3(kThreads), 0, st, q, kc, vc, rows, kv_len,
                       max_kv, Hq, Hkv, n_rep, scale, post, nsplit, ws_o, ws_ml, out);
    return hipGetLastError() == hipSuccess ? CRANE_HIP_OK : CRANE_HIP_E_LAUNCH;
}

// nsplit = ceil(max_kv / CH) chunks per sequence.
template <typename T, int CH, class ROWS>
int launch_decode(const T* q, const T* kc, const T* vc, const ROWS& rows, const int32_t* kv_len, int max_kv, int nsplit,
                  int B, int Hq, int Hkv, float scale, int post, float* ws_o, float* ws_ml, T* out, hipStream_t st) {
    int rc;
    switch (pick_group(Hq / Hkv)) {
#define CRANE_DECODE_CASE(g)                                                                                          \
    case g:                                                                                                           \
        rc = launch_decode_g<T, g, CH, ROWS>(q, kc, vc, rows, kv_len, max_kv, nsplit, B, Hq, Hkv, scale, post, ws_o,  \
                                             ws_ml, out, st);                                                         \
        break;
        CRANE_DECODE_CASE(1)
        CRANE_DECODE_CASE(2)
        CRANE_DECODE_CASE(3)
        CRANE_DECODE_CASE(4)
        CRANE_DECODE_CASE(5)
        CRANE_DECODE_CASE(6)
        CRANE_DECODE_CASE(7)
        CRANE_DECODE_CASE(8)
#undef CRANE_DECODE_CASE
        default: return CRANE_HIP_E_GQA;
    }
    if (rc != CRANE_HIP_OK) return rc;
    const int n_rep = Hq / Hkv, G = pick_group(n_rep);
    const dim3 mgrid((unsigned)(Hkv * (n_rep / G)), (unsigned)B, (unsigned)G);
    if (nsplit > kMergeRegs)
        hipLaunchKernelGGL((decode_merge_kernel<T, CH, 8>), mgrid, dim3(64 * 8), 0, st, ws_o, ws_ml, kv_len,
                           max_kv, Hq, n_rep, nsplit, out);
    else if (nsplit > 1)
        hipLaunchKernelGGL((decode_merge_wave_kernel<T, CH>), dim3(mgrid.x, mgrid.y, (unsigned)((G + 3) / 4)), dim3(256),
                           0, st, ws_o, ws_ml, kv_len, max_kv, Hq, n_rep, G, nsplit, out);
    return launch_status(hipGetLastError());
}

// Chunk size: 512 keys for long contexts (fewer work items and half the
// partials to merge: 9% faster at 32768 keys, 2% at 16384), 256 otherwise
// (more parallelism; 6% faster at 8192 keys for 8 sequences).  A paged cache
// takes 512 only when a page holds whole 512-row chunks.
template <typename T, class ROWS>
int launch_decode_any(const T* q, const T* kc, const T* vc, const ROWS& rows, const int32_t* kv_len, int max_kv, int B,
                      int Hq, int Hkv, float scale, int post, float* ws_o, float* ws_ml, T* out, hipStream_t st) {
    bool long_chunks = max_kv > kLongKv;
    if constexpr (ROWS::kPaged) long_chunks = long_chunks && rows.page_rows % kChunkLong == 0;
    if (long_chunks)
        return launch_decode<T, kChunkLong>(q, kc, vc, rows, kv_len, max_kv, (max_kv + kChunkLong - 1) / kChunkLong,
                                            B, Hq, Hkv, scale, post, ws_o, ws_ml, out, st);
    return launch_decode<T, kChunkShort>(q, kc, vc, rows, kv_len, max_kv, (max_kv + kChunkShort - 1) / kChunkShort, B,
                                         Hq, Hkv, scale, post, ws_o, ws_ml, out, st);
}

// Splits the workspace is sized for: the short chunk, which gives the most.
int64_t n_splits(int64_t max_kv) { return (max_kv + kChunkShort - 1) / kChunkShort; }

// Workspace: the partial rows (bf16 rows for bf16 calls, f32 rows for f32
// calls), then their f32 (max, sum) pairs.
struct WsLayout {
    size_t o_off, ml_off, total;
};

WsLayout ws_layout(int B, int Hq, int64_t ns, int dtype) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout w;
    w.o_off = 0;
    w.ml_off = w.o_off + up((size_t)B * Hq * ns * kHeadDim * (size_t)elem_size(dtype));
    w.total = w.ml_off + up((size_t)B * Hq * ns * 2 * sizeof(float));
    return w;
}

// Checks shared by both layouts, then the launch; `rows` addresses the cache.
template <class ROWS>
int attn_decode(const void* q, const void* k_cache, const void* v_cache, const ROWS& rows, const int32_t* kv_len,
                int64_t max_kv, int B, int Hq, int Hkv, int D, float scale, int score_mode, void* workspace,
                size_t ws_bytes, void* out, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || Hq <= 0 || Hkv <= 0) return CRANE_HIP_E_INVALID;
    if (Hq % Hkv != 0) return CRANE_HIP_E_GQA;
    if (max_kv <= 0) return CRANE_HIP_E_INVALID;
    if (!(scale > 0.0f) || !__builtin_isfinite(scale)) return CRANE_HIP_E_INVALID;
    if (score_mode != CRANE_HIP_SCORE_GROUPED && score_mode != CRANE_HIP_SCORE_STANDARD) return CRANE_HIP_E_INVALID;
    if (B == 0) return CRANE_HIP_OK;
    if (!q || !k_cache || !v_cache || !kv_len || !out) return CRANE_HIP_E_INVALID;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return CRANE_HIP_E_ALIGN;
    const int64_t ns = n_splits(max_kv);
    if (max_kv > 0x7fffffffLL || ns > kMaxSplits || B > 65535 || (int64_t)B * Hq > 0x7fffffffLL)
        return CRANE_HIP_E_INVALID;
    const WsLayout w = ws_layout(B, Hq, ns, dtype);
    if (!workspace || ws_bytes < w.total || !aligned16(workspace)) return CRANE_HIP_E_WORKSPACE;
    float* ws_o = (float*)((char*)workspace + w.o_off);
    float* ws_ml = (float*)((char*)workspace + w.ml_off);
    hipStream_t st = (hipStream_t)stream;
    const int post = score_mode == CRANE_HIP_SCORE_STANDARD;
    if (dtype == CRANE_HIP_F32)
        return launch_decode_any<float>((const float*)q, (const float*)k_cache, (const float*)v_cache, rows, kv_len,
                                        (int)max_kv, B, Hq, Hkv, scale, post, ws_o, ws_ml, (float*)out, st);
    return launch_decode_any<bf16_t>((const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, rows, kv_len,
                                     (int)max_kv, B, Hq, Hkv, scale, post, ws_o, ws_ml, (bf16_t*)out, st);
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" size_t crane_hip_attn_decode_workspace(int B, int Hq, int Hkv, int D, int64_t max_kv, int dtype) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || D != kHeadDim || max_kv <= 0) return 0;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return 0;
    return ws_layout(B, Hq, n_splits(max_kv), dtype).total;
}

extern "C" int crane_hip_attn_decode(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                     const int32_t* kv_len, int64_t max_kv, int B, int Hq, int Hkv, int D,
                                     float scale, int score_mode, void* workspace, size_t ws_bytes, void* out,
                                     int dtype, void* stream) {
    if (cache_cap <= 0 || max_kv > cache_cap) return CRANE_HIP_E_CAPACITY;
    return attn_decode(q, k_cache, v_cache, DenseRows{cache_cap}, kv_len, max_kv, B, Hq, Hkv, D, scale, score_mode,
                       workspace, ws_bytes, out, dtype, stream);
}

// ---- Allocation-free decode: the split-KV partials in a device array that
// lives as long as the process (one copy per GPU), for callers that cannot
// allocate (HIP graph capture, serving loops that forbid hipMalloc).  Calls
// that overlap in time on one GPU share the array and race; the partials need
// no clearing (each chunk's slot is written before the merge reads it).
static constexpr size_t kScratchBytes = (size_t)32 << 20;  // 32 MiB: c5 (8 x 64 heads, 32769 keys, bf16) needs 17.0 MiB
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace crane {
namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices];  // the array's device address on each GPU, looked up once per device

// The array's address on the device that runs `stream` (set-up on the
// device's first call: hipGetSymbolAddress with that device current, the
// caller's current device restored after).  Returns a CRANE_HIP_E_* code;
// *ptr is valid only on success.
int device_scratch(hipStream_t stream, void** ptr) {
    const int dev = stream_device(stream);
    if (dev < 0 || dev >= kMaxDevices) return CRANE_HIP_E_LAUNCH;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return CRANE_HIP_E_LAUNCH;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return CRANE_HIP_E_LAUNCH;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev && hipSetDevice(cur) != hipSuccess) return CRANE_HIP_E_LAUNCH;
        if (e != hipSuccess || !p) return CRANE_HIP_E_LAUNCH;
        scratch_ptr[dev] = p;
    }
    *ptr = scratch_ptr[dev];
    return CRANE_HIP_OK;
}
}  // namespace
}  // namespace crane

extern "C" size_t crane_hip_attn_decode_noalloc_limit(void) { return kScratchBytes; }

extern "C" int crane_hip_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                             int64_t cache_cap, const int32_t* kv_len, int64_t max_kv, int B, int Hq,
                                             int Hkv, int D, float scale, int score_mode, void* out, int dtype,
                                             void* stream) {
    if (cache_cap <= 0 || max_kv > cache_cap) return CRANE_HIP_E_CAPACITY;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || max_kv <= 0 || max_kv > 0x7fffffffLL || B > 65535) return CRANE_HIP_E_INVALID;
    if (B == 0) return CRANE_HIP_OK;
    if (ws_layout(B, Hq, n_splits(max_kv), dtype).total > kScratchBytes) return CRANE_HIP_E_WORKSPACE;
    void* ws = nullptr;
    const int rc = device_scratch((hipStream_t)stream, &ws);
    if (rc) return rc;
    return attn_decode(q, k_cache, v_cache, DenseRows{cache_cap}, kv_len, max_kv, B, Hq, Hkv, D, scale, score_mode, ws,
                       kScratchBytes, out, dtype, stream);
}

extern "C" int crane_hip_attn_decode_paged(const void* q, const void* k_pool, const void* v_pool, int64_t n_pages,
                                           int page_rows, const int32_t* block_table, int64_t table_stride,
                                           const int32_t* kv_len, int64_t max_kv, int B, int Hq, int Hkv, int D,
                                           float scale, int score_mode, void* workspace, size_t ws_bytes, void* out,
                                           int dtype, void* stream) {
    const int rc = check_paged(n_pages, page_rows, block_table, table_stride, Hkv);
    if (rc) return rc;
    if (max_kv > table_stride * page_rows) return CRANE_HIP_E_CAPACITY;
    return attn_decode(q, k_pool, v_pool, PagedRows{block_table, table_stride, n_pages, page_rows}, kv_len, max_kv, B,
                       Hq, Hkv, D, scale, score_mode, workspace, ws_bytes, out, dtype, stream);
}
