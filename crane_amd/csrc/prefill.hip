// prefill.hip -- causal GQA flash prefill over Crane's [B, Hkv, cap, D] cache (gfx950).
//
// Replaces the prefill SDPA of qwen3/modeling.rs:469-502 (K/V expanded to Hq
// heads, (q@K^T)*scale, + the causal -1e9 mask of :866-884, softmax_last_dim,
// @V, transpose to [B,S,Hq*D]); the same op chain is in
// hunyuan_dense/modeling.rs:610-645 and qwen2.rs:191-211 (-inf mask).  The
// [S, start+S] score matrix is never materialised: scores live in registers,
// the softmax is online (running max and sum per query row, log2 domain) and
// key tiles that lie entirely above the diagonal are never visited.
//
// bf16 kernel (MFMA): a workgroup owns 128 query rows of one q head (4 waves
// x 32 rows).  Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16,
// so a lane holds 16 keys of ONE query row (lane%32) and the row max/sum need
// one cross-half exchange only.  The resulting P^T tile is already laid out as
// the B operand of O^T = V^T P^T: no data movement between the two products.
// K and V tiles are copied HBM -> LDS row-major, as Crane stores them, by
// bounds-checked buffer_load ... lds (no VGPRs, no VALU, zero rows past the
// cache end), double-buffered so tile t+1 is in flight while tile t is
// computed.  K rows are the A operand of the first product; the second
// product's A operand V^T comes from the same row-major tile through
// ds_read_b64_tr_b16 transposed reads.  16-byte chunks are XOR-swizzled per
// row so both read patterns avoid LDS bank conflicts.
// Workgroup ids are remapped so that heavy (late) query tiles start first and
// the q heads sharing a kv head run on the same XCD (shared L2).
//
// Rounding points (bf16): candle's bf16 matmul returns Q K^T rounded to bf16,
// and its affine multiplies that by the scale converted to bf16 and rounds the
// product to bf16 again (qwen3/modeling.rs:488).  Workgroups whose rows see
// fewer than kLongRowKeys keys reproduce both roundings for every score: each
// rounding is a v_cvt_pk_bf16_f32 with a zero low half, read back as an f32,
// and the product of the two bf16 values is exact in f32 (a v_mul_f32).
// Workgroups whose first row sees at least kLongRowKeys keys keep the first
// rounding only and fold the scale into the exp2 argument's FMA: two VALU
// instructions fewer per score (the kernel is as much VALU- as MFMA-bound),
// while over that many keys the second rounding's effect on an output
// averages out (about 7% of the time at config 4, and 1.3e-3 more
// mean-relative distance from candle's chain on such rows).
// candle's softmax_last_dim then rounds s - max, exp, the row sum and the
// quotient p = e / sum to bf16 before the P V product (:493-494).  A one-pass
// kernel only has the row's max and sum at the end, so for rows with more than
// one 64-key tile these roundings are not reproduced: the online softmax keeps
// them in f32, P enters the P V product in bf16, and the row sum l adds the
// same bf16 p (v_dot2_f32_bf16 against (1, 1)), so numerator and denominator
// see the same weights.  A wave whose 32 rows all see keys of the first tile
// only (the first rows of a causal prefill, where few keys carry large
// weights and candle's roundings move the output most) runs candle's chain
// exactly: the row max, e = bf16(exp(bf16(s - max))), the bf16 sum, p =
// bf16(e / sum), and O = P V without a final division.
//
// f32 kernel: a plain wave-per-query-row online-softmax kernel; Crane serves
// prefill in bf16 on GPU (crane-serve/src/lib.rs:123-150), f32 is kept for
// completeness of the operator.
#include <atomic>
#include <type_traits>

#include "common.h"

namespace crane {
namespace {

#ifndef CRANE_PREFILL_WAVES
#define CRANE_PREFILL_WAVES 4
#endif
constexpr int kWaves = CRANE_PREFILL_WAVES;   // waves per workgroup, 32 query rows each
constexpr int kBM = 32 * kWaves;              // query rows per workgroup
constexpr int kCopies = 16 / kWaves;          // 1 KiB blocks of a 16 KiB tile each wave copies
constexpr int kBN = 64;                       // keys per tile
constexpr int kTileBytes = kBN * kHeadDim * 2;  // 16 KiB of K (or V) per tile
constexpr float kPsumMax = 256.0f;            // largest tile sum of p in a lane before the running max moves
constexpr float kMaskRaw = -1.0e30f;          // raw score of a masked key (finite: see scores_bf16)
constexpr int kLongRowKeys = 1024;           // keys a workgroup's first row sees for its rows to be long
constexpr int kLongRowRounding = 1;          // candle's score roundings kept in long rows (of 2)

__device__ __forceinline__ f32x16_v mfma32(bf16x8_v a, bf16x8_v b, f32x16_v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_v as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_v, u); }

// LDS tiles keep Crane's row-major rows (256 B per key, a full sweep of the 64
// banks) with the 16-byte chunks of row r XOR-permuted by swz(r), which swaps
// the two 2-bit halves of r mod 16.  Then 16 consecutive rows read at one chunk
// index (K fragments, 16 lanes per cycle) hit 16 different chunks, and a
// transposed V read (32 lanes per cycle: 4 rows x 4 consecutive chunks) hits
// 16 different chunks, so neither read pattern has bank conflicts.
__device__ __forceinline__ int swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4_v;
typedef __attribute__((address_space(3))) s16x4_v lds_s16x4_v;

// ds_read_b64_tr_b16: within each 16-lane group, lane i supplies 4 consecutive
// bf16 x[i][0..3] and receives x[4k + i/4][i%4] for k = 0..3.  With lane i
// pointing at row base + i/4, columns c0 + 4(i%4) .. +3 of a row-major tile,
// lane i receives column c0 + i of rows base .. base + 3: a transposed read.
__device__ __forceinline__ uint2 read_tr16(const uint8_t* p) {
    const s16x4_v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_v*)(p));
    return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Copy keys [64 t, 64 t + 64) of K (or V) into one 16 KiB LDS buffer with
// bounds-checked buffer_load ... lds (rows past the cache rows read as zero).
// Wave w copies the 1 KiB blocks kCopies*w .. +kCopies-1 of the tile; lane l of
// block blk fills row 4 blk + l/16, chunk l%16, with global chunk (l%16) ^ swz(row).
__device__ __forceinline__ int copy_voffset(int i, int wave, int lane) {
    const int row = 4 * (wave * kCopies + i) + (lane >> 4);
    return row * (kHeadDim * 2) + 16 * ((lane & 15) ^ swz(row));
}
// vofs[i] = copy_voffset(i, ...): the lane part of the source offset, fixed per
// lane; the tile part (t * 16 KiB) is the wave-uniform soffset.
__device__ __forceinline__ void issue_tile(__amdgpu_buffer_rsrc_t rsrc, int t, int wave, const uint32_t (&vofs)[kCopies],
                                           uint8_t* dst) {
#pragma unroll
    for (int i = 0; i < kCopies; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst + (wave * kCopies + i) * 1024, 16, vofs[i], t * kTileBytes,
                                                 0, 0);
}

// s_waitcnt with only vmcnt constrained (expcnt and lgkmcnt at their maxima).
#define CRANE_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))

// S^T = K Q^T for the 64 keys of a tile: two 32x32 blocks of 8 MFMAs each.
// Lane (n, hh) holds keys nb*32 + 8*(r/4) + 4*hh + r%4 of query row n in s[nb][r].
// koff[ks] is the lane's byte offset of chunk 2ks+hh of row n; row 32+n has the
// same swizzle (it depends on the row mod 16), so block nb adds nb * 8 KiB.
__device__ __forceinline__ void qk_tile(const uint8_t* kt_lds, const bf16x8_v (&qf)[8], const uint32_t (&koff)[8],
                                        f32x16_v (&s)[2]) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[nb][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const uint4 ku = *reinterpret_cast<const uint4*>(kt_lds + koff[ks] + nb * 8192);
            s[nb] = mfma32(as_bf16x8(ku), qf[ks], s[nb]);
        }
}

// candle's bf16 rounding of an f32 (round to nearest even), read back as an
// f32: v_cvt_pk_bf16_f32 with a zero low half.  Written as an instruction
// because the compiler rounds into the low half and moves it up.  A masked
// key carries the finite raw score kMaskRaw, which stays a huge negative
// score through both roundings.
__device__ __forceinline__ float round_bf16(float x) {
    float r;
    asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
    return r;
}
// candle's bf16 score of a raw f32 product: s = bf16(bf16(acc) * scale), with
// scale a bf16 value held as an f32.  The product of two bf16 values is exact
// in f32, so a plain v_mul_f32 forms it: no v_dot2_f32_bf16, which on gfx950
// does not run beside the MFMAs (a dot2 and an MFMA stream on one SIMD take
// longer together than one after the other).
__device__ __forceinline__ float score_bf16(float acc, float scale) { return round_bf16(round_bf16(acc) * scale); }

// Keep a value in a register as computed: the compiler may not split it into
// a base plus a per-use offset (which would cost an add per use in the loop).
__device__ __forceinline__ uint32_t pinned(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Map the 1-D workgroup id to (q tile, sequence, q head).  Groups of
// 8*n_rep consecutive ids hold 8 (qtile, b, kv head) units x n_rep heads, laid
// out so that ids congruent mod 8 (dispatched to the same XCD) share a unit.
// Units are ordered heaviest (last q tile) first.  Returns false for padding ids.
__device__ __forceinline__ bool map_block(int id, int n_qt, int B, int Hkv, int n_rep, int& qt, int& b, int& hq) {
    const int chunk = 8 * n_rep;
    const int c = id / chunk, rem = id % chunk;
    const int r = rem / 8, x = rem % 8;
    const int unit = c * 8 + x;
    const int n_units = n_qt * B * Hkv;
    if (unit >= n_units) return false;
    const int qt_rank = unit / (B * Hkv);
    const int rest = unit % (B * Hkv);
    b = rest / Hkv;
    const int kvh = rest % Hkv;
    qt = n_qt - 1 - qt_rank;
    hq = kvh * n_rep + r;
    return true;
}

// The kernel body (prefill_bf16_kernel below).  R: the score roundings of candle that the workgroup's waves reproduce (2:
// both, for rows that see fewer than kLongRowKeys keys; kLongRowRounding for
// the rest).
template <bool CAUSAL, class ROWS, int SPLIT, int R>
__device__ __forceinline__ void prefill_bf16_body(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                                  const bf16_t* __restrict__ vc, const ROWS& rows, int start, int S,
                                                  int Hq, int Hkv, uint32_t scale_bits, bf16_t* __restrict__ out,
                                                  int qt, int b, int hq, uint8_t (&kbufs)[SPLIT][2][kTileBytes],
                                                  uint8_t (&vbufs)[SPLIT][2][kTileBytes]) {
    const int n_rep = Hq / Hkv;
    const int kvh = hq / n_rep;
    const int m0 = qt * kBM;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS copy targets are scalar
    const int grp = SPLIT > 1 ? wave_all / kWaves : 0;              // key-range group
    const int wave = SPLIT > 1 ? wave_all % kWaves : wave_all;      // wave within the group: its query rows
    auto& kbuf = kbufs[grp];
    auto& vbuf = vbufs[grp];
    const int n = lane & 31, hh = lane >> 5;

    const int L = start + S;                                 // cache rows holding keys for this chunk
    const int kend = CAUSAL ? min(start + m0 + kBM, L) : L;  // keys any row of the tile can see
    const int n_all = (kend + kBN - 1) / kBN;
    const int half = (n_all + SPLIT - 1) / SPLIT;            // steps every group takes
    const int t0 = grp * half;                               // this group's first tile
    const int n_tiles = max(0, min(half, n_all - t0));       // ... and how many it has
    uint32_t vofs[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) vofs[i] = pinned(copy_voffset(i, wave, lane));
    // Tile x of K (or V) into LDS.  Dense: one resource over the sequence's L
    // rows, the tile picked by the scalar offset.  Paged: a resource over the
    // tile's rows inside its page (a page holds whole tiles); rows past L, and
    // a page id outside the pool, read as zero.
    const int64_t head0 = ROWS::kPaged ? 0 : rows.offset(b, Hkv, kvh, 0);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc + head0, L * kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vc + head0, L * kHeadDim * 2);
    auto issue = [&](const bf16_t* pool, const __amdgpu_buffer_rsrc_t& whole, int x, uint8_t* dst)
        __attribute__((always_inline)) {
        if constexpr (ROWS::kPaged) {
            const int key0 = x * kBN;
            const int64_t off = key0 < L ? rows.offset(b, Hkv, kvh, key0) : -1;
            const int bytes = off < 0 ? 0 : min(kBN, L - key0) * kHeadDim * 2;
            issue_tile(make_rsrc(pool + (off < 0 ? 0 : off), bytes), 0, wave, vofs, dst);
        } else {
            issue_tile(whole, x, wave, vofs, dst);
        }
    };
    if (n_tiles > 0) {
        issue(kc, rk, t0, kbuf[0]);
        issue(vc, rv, t0, vbuf[0]);
    }
    if (n_tiles > 1) issue(kc, rk, t0 + 1, kbuf[1]);

    // Q fragments (B operand of S^T = K Q^T): query row qrow, dims 16ks + 8hh .. +7.
    const int qrow = m0 + wave * 32 + n;
    bf16x8_v qf[8];
    {
        const bf16_t* qp = q + (((int64_t)b * Hq + hq) * S + min(qrow, S - 1)) * kHeadDim + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            uint4 u = *reinterpret_cast<const uint4*>(qp + 16 * ks);
            if (qrow >= S) u = make_uint4(0, 0, 0, 0);
            qf[ks] = as_bf16x8(u);
        }
    }
    f32x16_v oacc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const int qpos = start + qrow;                      // absolute position of my query
    const int wave_first = start + m0 + wave * 32;      // first position of this wave's rows
    // Every key this wave's rows see lies in tile 0: candle's softmax chain runs exactly.
    const bool exact = grp == 0 && (CAUSAL ? wave_first + 31 < kBN : L <= kBN);
    // the bf16 scale as the pairs (scale, 0) and (0, scale), and as an f32
    const float scale_f = __uint_as_float(scale_bits << 16);  // the bf16 scale as an f32
    const float scale_log2 = scale_f * kLog2e;                 // raw-score scale of the running max
    // transposed-read coordinates of this lane for the V^T fragments
    const int vg = lane >> 4, vi = lane & 15;
    const int v_h = vg >> 1;                            // key half of the A operand
    const int v_col = 16 * (vg & 1) + 4 * (vi & 3);     // column inside a 32-dim block
    const bf16x2_v ones = {(__bf16)1.f, (__bf16)1.f};
    // Per-lane LDS byte offsets, fixed for the whole loop.  K: chunk 2ks+hh of
    // row n.  V (transposed reads): rows r = 4 v_h + vi/4 (+8 for the high
    // half) at column 32 db + v_col; key step st adds 16 rows = 4 KiB, with
    // the same swizzle (rows mod 16 are unchanged).
    uint32_t koff[8], voff[4][2];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) koff[ks] = pinned(n * 256 + 16 * ((2 * ks + hh) ^ swz(n)));
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = 4 * v_h + (vi >> 2) + 8 * h, col = 32 * db + v_col;
            voff[db][h] = pinned(r * 256 + 16 * ((col >> 3) ^ swz(r)) + 2 * (col & 7));
        }

    // Tile 0 is visible to every row (key 0 precedes every query position);
    // a later group's first tile need not be (see the -inf guards below).
    if (n_tiles > 1) CRANE_WAIT_VMCNT(2 * kCopies); else CRANE_WAIT_VMCNT(kCopies);  // this wave's K(0) copies
    __syncthreads();                                                   // ... and every wave's
    f32x16_v sa[2], sb[2];
    qk_tile(kbuf[0], qf, koff, sa);

    // O^T += V^T P^T over one V tile: 4 dim blocks x 4 key steps of 16; the A
    // operand (dims x keys) comes straight from the row-major V tile by
    // transposed reads, issued one key step ahead of the MFMAs that use them
    // (no VALU work here covers their latency; c2 -3.5%, c4 unchanged).
    auto pv_tile = [&](const uint8_t* vt_lds, const bf16x8_v (&pf)[4]) __attribute__((always_inline)) {
        uint4 cur[4], nxt[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const uint2 lo = read_tr16(vt_lds + voff[db][0]);
            const uint2 hi = read_tr16(vt_lds + voff[db][1]);
            cur[db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st + 1 < 4) {
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const uint2 lo = read_tr16(vt_lds + voff[db][0] + (st + 1) * 4096);  // keys of slots 0..3
                    const uint2 hi = read_tr16(vt_lds + voff[db][1] + (st + 1) * 4096);  // slots 4..7: 8 rows on
                    nxt[db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                }
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) oacc[db] = mfma32(as_bf16x8(cur[db]), pf[st], oacc[db]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int db = 0; db < 4; ++db) cur[db] = nxt[db];
        }
    };

    // Waves whose rows see keys of tile 0 only (the first rows of a causal
    // prefill, or a short non-causal one) run candle's softmax_last_dim chain
    // in bf16 exactly, before the loop: the row max, e = bf16(exp(bf16(s -
    // max))), the sum in f32 rounded to bf16, p = bf16(e / sum) (e times the
    // sum's reciprocal), then O = P V with no division at the end.  Their
    // workgroup waits for V(0) once more; the loop skips their tile 0.
    if (CAUSAL ? start + m0 + 31 < kBN : L <= kBN) {  // uniform: wave 0 of the workgroup is exact
        if (n_tiles > 1) CRANE_WAIT_VMCNT(kCopies); else CRANE_WAIT_VMCNT(0);  // this wave's V(0) copies
        __syncthreads();                                                     // ... and every wave's
        if (exact) {
            if (CAUSAL || L < kBN) {
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = nb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                        if (key >= L || (CAUSAL && key > qpos)) sa[nb][r] = kMaskRaw;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; r += 4) {
                    const float s0 = score_bf16(sa[nb][r], scale_f), s1 = score_bf16(sa[nb][r + 1], scale_f);
                    const float s2 = score_bf16(sa[nb][r + 2], scale_f), s3 = score_bf16(sa[nb][r + 3], scale_f);
                    sa[nb][r] = s0;
                    sa[nb][r + 1] = s1;
                    sa[nb][r + 2] = s2;
                    sa[nb][r + 3] = s3;
                    mx = fmaxf(mx, fmaxf(fmaxf(s0, s1), fmaxf(s2, s3)));
                }
            mx = fmaxf(mx, __shfl_xor(mx, 32));  // the row's other 32 keys sit in the other lane half
            float sum = 0.f;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    sa[nb][r] = rt<bf16_t>(fast_exp2(rt<bf16_t>(sa[nb][r] - mx) * kLog2e));
                    sum += sa[nb][r];
                }
            const float inv = 1.0f / rt<bf16_t>(sum + __shfl_xor(sum, 32));
            bf16x8_v pf[4];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const bf16x2_v pw = __builtin_bit_cast(bf16x2_v, pack_bf16x2(sa[nb][r] * inv, sa[nb][r + 1] * inv));
                    pf[nb * 2 + (r >> 3)][r & 7] = pw[0];
                    pf[nb * 2 + (r >> 3)][(r & 7) + 1] = pw[1];
                }
            pv_tile(vbuf[0], pf);
            m_run = 0.f;   // finite, so a key-split merge keeps these rows as they are
            l_run = 0.5f;  // each lane half holds half of the normalised row sum
        }
    }

    // One tile: softmax of tile t's scores (sc), S^T of tile t+1 (into sn),
    // then O^T += V^T P^T for tile t.  The exp work of tile t and the MFMAs of
    // tile t+1 are independent, so one wave keeps both pipes busy.
    // The step's parity (t & 1) is a compile-time constant, so every LDS
    // address below is a per-lane offset plus an immediate.
    auto step = [&](auto parity, int t, f32x16_v (&sc)[2], f32x16_v (&sn)[2]) {
        constexpr int par = decltype(parity)::value;
        CRANE_WAIT_VMCNT(0);  // this wave's copies of V(t) and K(t+1) have landed
        __syncthreads();      // ... and every wave's; K(t) and V(t-1) are fully consumed
        if (t + 2 < n_tiles) issue(kc, rk, t0 + t + 2, kbuf[par]);
        if (t + 1 < n_tiles) issue(vc, rv, t0 + t + 1, vbuf[par ^ 1]);
        if (SPLIT > 1 && t >= n_tiles) return;  // past this group's half: only the barrier
        const int kt = (t0 + t) * kBN;
        if (CAUSAL && kt > wave_first + 31) return;  // the whole tile is above this wave's diagonal
        if (exact) return;                           // done before the loop (its only tile is tile 0)
        if (kt + kBN > kend || (CAUSAL && kt + kBN - 1 > wave_first)) {  // diagonal or last tile
            // key = kt + 4 hh + e(nb, r) is masked when key >= kend or, causal,
            // key > qpos: one compare of the lane-constant offset e per key
            const int thr = (CAUSAL ? min(qpos, kend - 1) : kend - 1) - kt - 4 * hh;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (nb * 32 + 8 * (r >> 2) + (r & 3) > thr) sc[nb][r] = kMaskRaw;
        }
        bf16x8_v pf[4];
        {
            // p = exp2(s log2(e) - m) for the score s of every key, bf16 for
            // the P V product, summed as rounded.
            auto tile_p = [&](float neg_m) __attribute__((always_inline)) {
                float psum = 0.f;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int r = 0; r < 16; r += 4) {
                        float sv[4];  // the exp2 argument's score and its factor
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            sv[e] = R == 2 ? score_bf16(sc[nb][r + e], scale_f)
                                           : (R == 1 ? round_bf16(sc[nb][r + e]) : sc[nb][r + e]);
                        const float fac = R == 2 ? kLog2e : scale_log2;
#pragma unroll
                        for (int u = 0; u < 4; u += 2) {
                            const float p0 = fast_exp2(__builtin_fmaf(sv[u], fac, neg_m));
                            const float p1 = fast_exp2(__builtin_fmaf(sv[u + 1], fac, neg_m));
                            const bf16x2_v pw = __builtin_bit_cast(bf16x2_v, pack_bf16x2(p0, p1));
                            psum = __builtin_amdgcn_fdot2_f32_bf16(pw, ones, psum, false);
                            pf[nb * 2 + (r >> 3)][(r & 7) + u] = pw[0];
                            pf[nb * 2 + (r >> 3)][(r & 7) + u + 1] = pw[1];
                        }
                    }
                return psum;
            };
            // Lazy rescaling: the reference max m_run stays where it is while
            // every lane's tile sum of p stays at most kPsumMax (so every p <=
            // kPsumMax; no max over the tile is taken).  Otherwise the wave
            // moves m_run to each row's running max, rescales O and l, and
            // takes the tile's p again; a wave with a row at m = -inf (no key
            // seen yet) moves first.  A row that has seen no key keeps
            // m = -inf, with p = exp2(huge negative) = 0.
            // tmax: this lane half's raw max; the row's max over both halves in
            // the log2 domain (the scale is positive); no key: -inf
            auto row_max_log2 = [&](float tmax) __attribute__((always_inline)) {
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
                return tmax > 0.5f * kMaskRaw ? tmax * scale_log2 : -INFINITY;
            };
            auto rescale = [&](float tmax) __attribute__((always_inline)) {
                const float m_new = fmaxf(m_run, row_max_log2(tmax));
                const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
                m_run = m_new;
            };
            auto tile_max = [&]() __attribute__((always_inline)) {
                float tmax = kMaskRaw;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sc[nb][r]);
                return tmax;
            };
            // A wave whose rows have seen no key yet (m = -inf, O = 0, l = 0,
            // where p would be inf): m moves to the row's max first, rather
            // than taking the tile's p twice.
            if (__all(m_run == -INFINITY)) m_run = row_max_log2(tile_max());
            float psum = tile_p(m_run == -INFINITY ? 0.f : -m_run);
            // Unconditional, so this stays in one basic block with the exp
            // work above: past the last tile (or above this wave's diagonal)
            // the result is simply not used, and nothing is in flight into
            // that buffer.
            qk_tile(kbuf[par ^ 1], qf, koff, sn);
            if (__any(!(psum <= kPsumMax) || m_run == -INFINITY)) {
                rescale(tile_max());
                psum = tile_p(m_run == -INFINITY ? 0.f : -m_run);
            }
            l_run += psum;
        }
        pv_tile(vbuf[par], pf);
    };
    const int n_steps = SPLIT > 1 ? half : n_tiles;
    for (int t = 0; t < n_steps; t += 2) {
        step(std::integral_constant<int, 0>{}, t, sa, sb);
        if (t + 1 < n_steps) step(std::integral_constant<int, 1>{}, t + 1, sb, sa);
    }

    if constexpr (SPLIT > 1) {
        // Group 1's O (in the freed K tiles) and (m, l) (in the freed V tiles)
        // for each lane, lane-minor; group 0's wave w merges the same query
        // rows' values.
        static_assert(SPLIT == 2, "two key groups");
        static_assert(kWaves * 64 * 64 * 4 <= (int)sizeof(kbufs) && kWaves * 2 * 64 * 4 <= (int)sizeof(vbufs),
                      "exchange fits the tile space");
        float* xo = reinterpret_cast<float*>(&kbufs[0][0][0]) + wave * 64 * 64 + lane;
        float* xml = reinterpret_cast<float*>(&vbufs[0][0][0]) + wave * 2 * 64 + lane;
        __syncthreads();  // every wave is done with the tiles
        if (grp == 1) {
            xml[0] = m_run;
            xml[64] = l_run;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) xo[64 * (16 * i + r)] = oacc[i][r];
        }
        __syncthreads();
        if (grp == 1) return;
        const float m1 = xml[0], l1 = xml[64];
        const float mm = fmaxf(m_run, m1);
        const float a0 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - mm);
        const float a1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - mm);
        l_run = l_run * a0 + l1 * a1;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[i][r] = oacc[i][r] * a0 + xo[64 * (16 * i + r)] * a1;
    }

    l_run += __shfl_xor(l_run, 32);  // the two lane halves hold different keys of the row (exact rows: 1)
    if (qrow < S) {
        const float inv = 1.0f / l_run;
        bf16_t* op = out + (((int64_t)b * S + qrow) * Hq + hq) * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dim = db * 32 + 8 * g + 4 * hh;
                const uint2 w = make_uint2(pack_bf16x2(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv),
                                           pack_bf16x2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv));
                *reinterpret_cast<uint2*>(op + dim) = w;
            }
    }
}

// SPLIT = 2 (a grid too small to fill the chip): 8 waves, two groups of 4 on
// the same 128 query rows; group g walks its half of the key tiles through its
// own LDS tiles, and group 1's running (max, sum, O) merge into group 0's
// through LDS at the end.  Every wave passes the same barriers: a step past a
// group's half does no copy and no work.
template <bool CAUSAL, class ROWS, int SPLIT>
__global__ __launch_bounds__(64 * kWaves * SPLIT) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_bf16_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc, ROWS rows,
    const int32_t* __restrict__ start_pos, int max_start, int S, int B, int Hq, int Hkv, uint32_t scale_bits,
    bf16_t* __restrict__ out) {
    const int n_rep = Hq / Hkv;
    const int n_qt = (S + kBM - 1) / kBM;
    int qt, b, hq;
    if (!map_block(blockIdx.x, n_qt, B, Hkv, n_rep, qt, b, hq)) return;
    const int start = min(max(start_pos[b], 0), max_start);
    // K tiles t and t+1 and V tile t are resident while tile t is computed;
    // K(t+2) and V(t+1) are in flight.  One set per group.
    __shared__ __attribute__((aligned(1024))) uint8_t kbufs[SPLIT][2][kTileBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t vbufs[SPLIT][2][kTileBytes];
    // The workgroup's first row sees at least kLongRowKeys keys (and so does every other row).
    const bool long_rows = CAUSAL ? start + qt * kBM + 1 >= kLongRowKeys : start + S >= kLongRowKeys;
    if (long_rows)
        prefill_bf16_body<CAUSAL, ROWS, SPLIT, kLongRowRounding>(q, kc, vc, rows, start, S, Hq, Hkv, scale_bits, out,
                                                                 qt, b, hq, kbufs, vbufs);
    else
        prefill_bf16_body<CAUSAL, ROWS, SPLIT, 2>(q, kc, vc, rows, start, S, Hq, Hkv, scale_bits, out, qt, b, hq,
                                                  kbufs, vbufs);
}

// f32: one wave per (query row, q head, sequence); lane owns dims 2*lane, 2*lane+1.
template <bool CAUSAL, class ROWS>
__global__ __launch_bounds__(64) void prefill_f32_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                         const float* __restrict__ vc, ROWS rows,
                                                         const int32_t* __restrict__ start_pos, int max_start, int S,
                                                         int Hq, int Hkv, float scale_log2, float* __restrict__ out) {
    const int i = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int n_rep = Hq / Hkv, kvh = hq / n_rep;
    const int start = min(max(start_pos[b], 0), max_start);
    const int L = start + S;
    const int kend = CAUSAL ? start + i + 1 : L;
    const float2 qv = *reinterpret_cast<const float2*>(q + (((int64_t)b * Hq + hq) * S + i) * kHeadDim + 2 * lane);
    float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int j = 0; j < kend; ++j) {
        const int64_t off = rows.offset(b, Hkv, kvh, j);  // a row on an invalid page reads as zero
        const float2 kv = off < 0 ? make_float2(0.f, 0.f) : *reinterpret_cast<const float2*>(kc + off + 2 * lane);
        float s = qv.x * kv.x + qv.y * kv.y;
#pragma unroll
        for (int msk = 32; msk >= 1; msk >>= 1) s += __shfl_xor(s, msk);
        s *= scale_log2;
        const float m_new = fmaxf(m, s);
        const float alpha = fast_exp2(m - m_new), p = fast_exp2(s - m_new);
        const float2 vv = off < 0 ? make_float2(0.f, 0.f) : *reinterpret_cast<const float2*>(vc + off + 2 * lane);
        l = l * alpha + p;
        o0 = o0 * alpha + p * vv.x;
        o1 = o1 * alpha + p * vv.y;
        m = m_new;
    }
    float* op = out + (((int64_t)b * S + i) * Hq + hq) * kHeadDim + 2 * lane;
    *reinterpret_cast<float2*>(op) = make_float2(o0 / l, o1 / l);
}

// Compute units of the current device (cached per device; host threads may
// race to fill an entry, with the same value).
int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Checks shared by both layouts, then the launch; `rows` addresses the cache.
template <class ROWS>
int attn_prefill(const void* q, const void* k_cache, const void* v_cache, const ROWS& rows, const int32_t* start_pos,
                 int64_t max_start, int B, int S, int Hq, int Hkv, int D, float scale, int causal, void* out,
                 int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (B < 0 || S < 0 || Hq <= 0 || Hkv <= 0 || max_start < 0) return CRANE_HIP_E_INVALID;
    if (Hq % Hkv != 0) return CRANE_HIP_E_GQA;
    if (!(scale > 0.0f) || !__builtin_isfinite(scale)) return CRANE_HIP_E_INVALID;
    if (B == 0 || S == 0) return CRANE_HIP_OK;
    if (!q || !k_cache || !v_cache || !start_pos || !out) return CRANE_HIP_E_INVALID;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out)) return CRANE_HIP_E_ALIGN;
    if (max_start + (int64_t)S > 0x7fffffffLL / (kHeadDim * 4) || B > 65535 || Hq > 65535) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == CRANE_HIP_BF16) {
        // candle scales the bf16 scores by the scale converted to bf16 (affine in T)
        const uint32_t sl = f32_bits(host_round_bf16(scale)) >> 16;
        const int n_rep = Hq / Hkv;
        const int64_t n_qt = (S + kBM - 1) / kBM;
        const int64_t units = n_qt * B * Hkv;
        const int64_t chunk = 8LL * n_rep;
        const int64_t blocks = ((units + 7) / 8) * chunk;
        if (blocks > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
        // A grid of at most one workgroup per CU leaves each SIMD one wave and the
        // last query tiles' key walk as the critical path: split the keys of
        // each tile between two groups of waves instead.
        const bool split = blocks <= (int64_t)device_cus();
#define CRANE_PREFILL_LAUNCH(C, SP)                                                                              \
    hipLaunchKernelGGL((prefill_bf16_kernel<C, ROWS, SP>), dim3((unsigned)blocks), dim3(64 * kWaves * SP), 0, st, \
                       (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, rows, start_pos,        \
                       (int)max_start, S, B, Hq, Hkv, sl, (bf16_t*)out)
        if (causal) {
            if (split) CRANE_PREFILL_LAUNCH(true, 2); else CRANE_PREFILL_LAUNCH(true, 1);
        } else {
            if (split) CRANE_PREFILL_LAUNCH(false, 2); else CRANE_PREFILL_LAUNCH(false, 1);
        }
#undef CRANE_PREFILL_LAUNCH
    } else {
        const float sl = scale * kLog2e;
        const dim3 grid((unsigned)S, (unsigned)Hq, (unsigned)B);
        if (causal)
            hipLaunchKernelGGL((prefill_f32_kernel<true, ROWS>), grid, dim3(64), 0, st, (const float*)q,
                               (const float*)k_cache, (const float*)v_cache, rows, start_pos, (int)max_start, S, Hq,
                               Hkv, sl, (float*)out);
        else
            hipLaunchKernelGGL((prefill_f32_kernel<false, ROWS>), grid, dim3(64), 0, st, (const float*)q,
                               (const float*)k_cache, (const float*)v_cache, rows, start_pos, (int)max_start, S, Hq,
                               Hkv, sl, (float*)out);
    }
    return launch_status(hipGetLastError());
}

}  // namespace
}  // namespace crane

using namespace crane;

extern "C" int crane_hip_attn_prefill(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                      const int32_t* start_pos, int64_t max_start, int B, int S, int Hq, int Hkv,
                                      int D, float scale, int causal, void* out, int dtype, void* stream) {
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (D != kHeadDim) return CRANE_HIP_E_HEAD_DIM;
    if (max_start < 0 || S < 0) return CRANE_HIP_E_INVALID;
    if (cache_cap <= 0 || max_start + (int64_t)S > cache_cap) return CRANE_HIP_E_CAPACITY;
    if (cache_cap > 0x7fffffffLL) return CRANE_HIP_E_INVALID;
    return attn_prefill(q, k_cache, v_cache, DenseRows{cache_cap}, start_pos, max_start, B, S, Hq, Hkv, D, scale,
                        causal, out, dtype, stream);
}

extern "C" int crane_hip_attn_prefill_paged(const void* q, const void* k_pool, const void* v_pool, int64_t n_pages,
                                            int page_rows, const int32_t* block_table, int64_t table_stride,
                                            const int32_t* start_pos, int64_t max_start, int B, int S, int Hq, int Hkv,
                                            int D, float scale, int causal, void* out, int dtype, void* stream) {
    const int rc = check_paged(n_pages, page_rows, block_table, table_stride, Hkv);
    if (rc) return rc;
    if (max_start < 0 || S < 0) return CRANE_HIP_E_INVALID;
    if (max_start + (int64_t)S > table_stride * page_rows) return CRANE_HIP_E_CAPACITY;
    return attn_prefill(q, k_pool, v_pool, PagedRows{block_table, table_stride, n_pages, page_rows}, start_pos,
                        max_start, B, S, Hq, Hkv, D, scale, causal, out, dtype, stream);
}
