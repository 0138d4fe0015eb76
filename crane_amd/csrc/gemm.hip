// gemm.hip -- the projections of a decoder layer and the lm_head (candle
// Linear, y = x W^T + b); C ABI in include/crane_gemm.h.
//
// Row-major y[M, N] = x[M, K] W[N, K]^T is, in hipBLASLt's column-major
// terms, D[N, M] = op(A) B with A = W viewed as [K, N] (transposed: N x K),
// B = x viewed as [K, M], D = y viewed as [N, M]; the bias vector (one value
// per row of D, i.e. per output feature) is the BIAS epilogue.
//
// Decode products (bf16, M <= 32 token rows) go to hand-written kernels
// instead: at M = 32 the product is a stream of W through the chip (2 bytes of
// W per 2 M flops).  Those whose K is a whole number of the per-wave rings
// (K <= 8192; the Qwen3-8B decode step's qkv_proj, o_proj, gate_up and
// lm_head) take the per-wave ring kernel below; other wide ones (N >= 16384)
// the streaming kernel; the rest, down_proj among them, hipBLASLt.  A
// product whose output only feeds a residual add (a decode step's o_proj and
// down_proj) or the fused append (its qkv_proj) can instead leave f32 split-K
// partial products for the add + norm or the append to sum
// (crane_gemm_linear_split: the ring kernel's PARTIAL form).  The
// streaming kernel (measured at the Qwen3-8B decode shapes before the ring
// kernel: gate_up [24576, 4096] 43 us vs hipBLASLt's 47 us, lm_head
// [151936, 4096] 241 us vs ~355 us):
//  - a workgroup of 4 waves owns 64 output features and all of K; wave w
//    multiplies features 16 w .. 16 w + 15 (the A operand of
//    v_mfma_f32_16x16x32_bf16) by the token rows (the B operand), f32
//    accumulation;
//  - K is streamed in stages of 128: the 64 W rows (256 bytes each) and the
//    token rows of x are copied HBM -> LDS by bounds-checked buffer_load ...
//    lds, each 1 KiB copy reading 4 whole 256-byte row pieces (x rows past M
//    read as zero), into a ring of three stage buffers so two stages are in
//    flight while one is multiplied;
//  - 16-byte chunks are XOR-swizzled by row in LDS, so the 16 rows of one
//    fragment read (ds_read_b128) fall in 16 different bank groups.
// Rounding: f32 accumulation, y = bf16(acc + b) (one rounding, as the
// hipBLASLt bias epilogue).
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

// ---------------------------------------------------------------- streaming

constexpr int kSkStageK = 128;   // k per pipeline stage (256 bytes of every row)
constexpr int kSkWaves = 4;      // waves per workgroup; each owns 16 output features
constexpr int kSkRows = 16 * kSkWaves;
constexpr int kSkMaxM = 32;      // token rows the streaming kernel takes

__device__ __forceinline__ bf16x8_v as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_v, u); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// LDS image of one stage: rows of 256 bytes (16 chunks of 16 bytes, chunk c
// of row r stored at slot c ^ (r & 15), so the 16 rows one fragment read
// touches hit 16 different bank groups), W rows first, then x rows.
template <int MT>
struct SkStage {
    static constexpr int kWBytes = kSkRows * 256;
    static constexpr int kXBytes = 16 * MT * 256;
    static constexpr int kBytes = kWBytes + kXBytes;
    static constexpr int kCopies = kBytes / 1024 / kSkWaves;  // 1 KiB copies per wave per stage
    static_assert(kBytes % (1024 * kSkWaves) == 0, "stage copies split evenly over the waves");
};

// The voffset of copy i of a wave: copy blk (of the stage's kBytes / 1024)
// fills LDS bytes [1024 blk, +1024): rows 4 blk + lane / 16 of the stage, slot
// lane % 16, from chunk slot ^ (row & 15) of that row's 256 bytes.  The stage's
// k offset is the scalar offset; W rows read from the W resource, x rows
// (token rows; rows past M read as zero) from the x resource.
template <int MT>
__device__ __forceinline__ uint32_t sk_voffset(int blk, int lane, int K) {
    const int row = 4 * blk + (lane >> 4);
    const int slot = lane & 15;
    const int r = row < kSkRows ? row : row - kSkRows;
    return (uint32_t)r * (uint32_t)K * 2u + 16u * (uint32_t)(slot ^ (r & 15));
}

// The W resource covers the workgroup's 64 rows (wb, wbytes), the x resource
// the M token rows (xb, xbytes).
struct SkSrc {
    const bf16_t* wb;
    const bf16_t* xb;
    uint32_t wbytes, xbytes;
};

// Issue this wave's copies of one stage into `dst`; soff is the stage's byte
// offset along k.  (Not a template: the host pass cannot form the LDS pointer
// the copy takes.)
__device__ __forceinline__ void sk_issue(uint8_t* dst, const SkSrc& src, const uint32_t* vofs, const bool* isw, int nc,
                                         int wave, int soff) {
#pragma unroll
    for (int i = 0; i < nc; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isw[i] ? sk_rsrc(src.wb, src.wbytes) : sk_rsrc(src.xb, src.xbytes),
                                                 dst + (wave * nc + i) * 1024, 16, vofs[i], soff, 0, 0);
}

// One pipeline stage: wait for stage st (in `cur`), refill `nxt` (the buffer
// of stage st - 1, which every wave has finished) with stage st + 2, and
// multiply stage st.
template <int MT>
__device__ __forceinline__ void sk_stage(const uint8_t* cur, uint8_t* nxt, int st, int nst, const SkSrc& src,
                                         const uint32_t (&vofs)[SkStage<MT>::kCopies],
                                         const bool (&isw)[SkStage<MT>::kCopies], int wave, int wrow, int r, int q,
                                         f32x4_v (&acc)[MT]) {
    using St = SkStage<MT>;
    // this wave's copies of stage st have landed (those of st + 1 may fly),
    // and its LDS reads of stage st - 1 have completed (lgkmcnt 0: the
    // compiler may have left the last products of stage st - 1, and their
    // waits, below this point)
    if (st + 1 < nst)
        __builtin_amdgcn_s_waitcnt(0x0070 | (St::kCopies & 15) | ((St::kCopies >> 4) << 14));
    else
        __builtin_amdgcn_s_waitcnt(0x0070);
    // Every wave's copies of stage st have landed and every wave has finished
    // reading stage st - 1, so the refill below may overwrite it.  A plain
    // barrier: a release fence here would wait for the copies still in flight
    // (they count as LDS writes); the acquire fence keeps the reads below it.
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (st + 2 < nst) sk_issue(nxt, src, vofs, isw, St::kCopies, wave, (st + 2) * kSkStageK * 2);
#pragma unroll
    for (int j = 0; j < kSkStageK / 32; ++j) {
        const int c = 4 * j + q;
        const uint4 a = *reinterpret_cast<const uint4*>(cur + wrow * 256 + 16 * (c ^ (wrow & 15)));
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int t = 16 * m + r;
            const uint4 bx = *reinterpret_cast<const uint4*>(cur + St::kWBytes + t * 256 + 16 * (c ^ (t & 15)));
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(bx), acc[m], 0, 0, 0);
        }
    }
}

// y = x[M, K] W[N, K]^T (+ b): N / 64 workgroups of 256 threads; workgroup
// `tile` owns features [64 tile, +64).  Wave w multiplies features 16 w .. +15
// (the A operand) by the MT token groups of 16 (the B operand).  Lane l holds
// A row l % 16 / B column l % 16 with the k elements of chunk (4 j + l / 16) of
// k-step j of a stage; accumulator element i is feature 16 w + 4 (l / 16) + i
// and token 16 m + l % 16.
template <int MT>
__global__ __launch_bounds__(64 * kSkWaves) void skinny_gemm_kernel(const bf16_t* __restrict__ x,
                                                                    const bf16_t* __restrict__ w,
                                                                    const bf16_t* __restrict__ bias,
                                                                    bf16_t* __restrict__ y, int M, int N, int K) {
    using St = SkStage<MT>;
    // three stage buffers as separate objects: the compiler's wait-count pass
    // then knows which buffer each copy writes and waits only for that one
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[St::kBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[St::kBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[St::kBytes];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.x;
    const int nst = K / kSkStageK;
    const SkSrc src{w + (int64_t)tile * kSkRows * K, x, (uint32_t)kSkRows * K * 2, (uint32_t)M * K * 2};
    uint32_t vofs[St::kCopies];
    bool isw[St::kCopies];
#pragma unroll
    for (int i = 0; i < St::kCopies; ++i) {
        const int blk = wave * St::kCopies + i;
        vofs[i] = sk_voffset<MT>(blk, lane, K);
        isw[i] = 4 * blk < kSkRows;  // uniform per copy
    }
    const int r = lane & 15, q = lane >> 4;
    const int wrow = 16 * wave + r;
    f32x4_v acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = f32x4_v{};
    sk_issue(lds0, src, vofs, isw, St::kCopies, wave, 0);
    if (nst > 1) sk_issue(lds1, src, vofs, isw, St::kCopies, wave, kSkStageK * 2);
    // stage st lives in buffer st % 3; the loop is unrolled by three so every
    // access names its buffer
    for (int st = 0; st < nst; st += 3) {
        sk_stage<MT>(lds0, lds2, st, nst, src, vofs, isw, wave, wrow, r, q, acc);
        if (st + 1 < nst) sk_stage<MT>(lds1, lds0, st + 1, nst, src, vofs, isw, wave, wrow, r, q, acc);
        if (st + 2 < nst) sk_stage<MT>(lds2, lds1, st + 2, nst, src, vofs, isw, wave, wrow, r, q, acc);
    }
    const int n = tile * kSkRows + 16 * wave + 4 * q;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int t = 16 * m + r;
        if (t >= M) continue;
        float v[4] = {acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
        if (bias) {
            float bv[4];
            load4(bias + n, bv);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += bv[e];
        }
        store4(y + (int64_t)t * N + n, v);
    }
}

// The streaming kernel takes bf16 products with few token rows and enough
// output features for 256 workgroups (one per CU); K in whole stages, and
// buffer offsets of the 64 W rows and of x within 32 bits.
bool skinny_fits(int64_t M, int64_t N, int64_t K) {
    return M >= 1 && M <= kSkMaxM && N % kSkRows == 0 && N / kSkRows >= 256 && N <= 0x7fffffff &&
           K % kSkStageK == 0 && (int64_t)kSkRows * K * 2 <= 0xffffffffLL && M * K * 2 <= 0xffffffffLL;
}

int launch_skinny(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* y, int M, int N, int K,
                  hipStream_t st) {
    const dim3 grid((unsigned)(N / kSkRows)), block(64 * kSkWaves);
    if (M <= 16)
        hipLaunchKernelGGL((skinny_gemm_kernel<1>), grid, block, 0, st, x, w, bias, y, M, N, K);
    else
        hipLaunchKernelGGL((skinny_gemm_kernel<2>), grid, block, 0, st, x, w, bias, y, M, N, K);
    return launch_status(hipGetLastError());
}

// ---------------------------------------------------------------- per-wave rings
//
// Decode products with few token rows whose K splits into whole pipelines:
// a workgroup owns 16 FT output features and splits K over its KS waves.  A
// wave streams its FT x 16 W rows over its quarter (or half) of K through a
// ring of D LDS slots of its own (buffer_load ... lds, 4 whole 256-byte row
// pieces per 1 KiB copy, non-temporal), and reads the token rows of x for the
// same k range straight into registers; no workgroup barrier until the end,
// where waves 1.. KS-1 hand their f32 partial products to wave 0 through LDS
// and wave 0 adds them in wave order (fixed, so a call's bits repeat).
// Measured at the Qwen3-8B decode shapes (32 rows, weights rotated past the
// Infinity Cache): o_proj [4096, 4096] 11.4 us against hipBLASLt's 13.8,
// qkv_proj [6144, 4096] 13.5 against 15.8, gate_up [24576, 4096] 31.8 against
// the streaming kernel's 43.0, lm_head [151936, 4096] 221 against 238.  The x
// reads are what bounds it: without them the same kernel streams W at 5.2-6.0
// TB/s, and x (the same bytes for every workgroup, read from L2) grows with
// 32 token rows / 16 FT features per W byte, so wider workgroups pay less x
// per W byte but leave CUs idle at narrow N.  The configuration follows N:
//   N <= 4096          FT 1, KS 4, D 4 (at most 256 workgroups)
//   4096 < N <= 8192   FT 2, KS 2, D 4, each workgroup starting its k walk
//                      at its own stage (spreads the x reads of the two
//                      waves' halves)
//   N > 8192           one workgroup per CU (LDS): FT 6 (KS 2, D 2, rotated
//                      k walk), FT 4 or FT 3 (KS 4, D 2), whichever leaves
//                      the busiest CU the fewest tiles (gate_up: 256
//                      workgroups of 96 features 31.8 us, 512 of 48 36.6 us,
//                      384 of 64 42.2 us)
// down_proj's shape [4096, 12288] stays on hipBLASLt through
// crane_gemm_linear (26 us against 29); split over 4 ranges of K with 64
// features per workgroup (crane_gemm_linear_split, 1 wave and a ring of 3
// slots) it takes 18.4 us, and o_proj (2 waves, a ring of 2) 8.6 us.

constexpr int kRingMaxK = 8192;

template <int N>
__device__ __forceinline__ void vm_wait() {
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Wait until at most `stages` later stages' loads (P loads each) are in
// flight; `stages` is a compile-time constant after unrolling.
template <int P>
__device__ __forceinline__ void vm_wait_stages(int stages) {
    switch (stages) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<P>(); break;
        case 2: vm_wait<2 * P>(); break;
        default: vm_wait<3 * P>(); break;
    }
}

// One stage of a wave's W rows into its ring slot: n copies of 1 KiB (4 rows
// x 256 bytes each), non-temporal.  (Not a template: the host pass cannot
// form the LDS pointer the copy takes.)
__device__ __forceinline__ void ring_copy(__amdgpu_buffer_rsrc_t src, uint8_t* dst, const uint32_t* vofs, int n,
                                          int soff) {
    for (int c = 0; c < n; ++c) __builtin_amdgcn_raw_ptr_buffer_load_lds(src, dst + c * 1024, 16, vofs[c], soff, 0, 2);
}

// y = x[M, K] W[N, K]^T (+ b), M <= 16 MT: N / (16 FT) workgroups of 64 KS
// threads.  Wave w covers k in [w K / KS, (w + 1) K / KS) in stages of 128
// (nst = K / (128 KS), a multiple of D and at least D); stage s of it lives in
// ring slot s % D, D - 1 stages in flight.  Lane l holds A row l % 16 (feature
// 16 f + l % 16 of the workgroup's FT tiles) and B column l % 16 (token
// 16 m + l % 16) with 8 k elements of chunk (l / 16 + 4 i) of a stage's 256
// bytes in k-step i: A and B take the same k order, so the sum is the dot
// product.  Token rows past M read row M - 1 (their columns are not stored).
// GATED: W is a merged gate_up [2 I, K] (N = 2 I rows) and y = T(silu(T(g))
// T(u)) [M, I]: the workgroup's first FT / 2 tiles are gate rows
// [8 FT tile, +8 FT), the others the up rows I + 8 FT tile .. of the same
// features, so each lane holds the gate and up sums of the same outputs.
// PARTIAL: K is split over gridDim.y workgroups as well (split ks takes k in
// [ks K', (ks + 1) K'), K' = K / gridDim.y), and the workgroup writes its f32
// partial sums, unrounded and without bias, to parts[ks][M][N]; whoever reads
// the product adds the splits in split order (one rounding of the sum, as the
// whole product's).  Each workgroup then covers gridDim.y times more features
// for the same grid, and reads that much less of x per W byte.
template <int MT, int KS, int D, int FT, bool ROT, bool GATED, bool PARTIAL = false>
__global__ __launch_bounds__(64 * KS) void ring_gemm_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                            const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
                                                            int M, int N, int K, float* __restrict__ parts) {
    constexpr int kLoads = 4 * FT + 4 * MT;  // loads per stage: W copies, then x fragments
    constexpr int H = GATED ? FT / 2 : FT;   // tiles per W row range
    static_assert(D >= 2 && D <= 4 && FT >= 1 && FT <= 6, "ring depth and width");
    static_assert(!GATED || FT % 2 == 0, "gated tiles come in gate / up pairs");
    static_assert((D - 1) * kLoads <= 63, "the loads in flight fit the 6-bit vmcnt");
    __shared__ f32x4_v part[KS > 1 ? KS - 1 : 1][FT][MT][64];
    // one LDS object per (ring slot, feature tile): the compiler's wait-count
    // pass then tells the copies in flight apart from the rows being read
#define CRANE_RING_SLOT(d, f) \
    __shared__ __attribute__((aligned(1024))) uint8_t ring##d##f[D > d && FT > f ? KS : 1][4096];
#define CRANE_RING_SLOTS(d) \
    CRANE_RING_SLOT(d, 0) CRANE_RING_SLOT(d, 1) CRANE_RING_SLOT(d, 2) CRANE_RING_SLOT(d, 3) CRANE_RING_SLOT(d, 4) \
    CRANE_RING_SLOT(d, 5)
    CRANE_RING_SLOTS(0) CRANE_RING_SLOTS(1) CRANE_RING_SLOTS(2) CRANE_RING_SLOTS(3)
#undef CRANE_RING_SLOTS
#undef CRANE_RING_SLOT
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // slot d's rows of feature tile f (d, f compile-time constants after unrolling)
    auto slot = [&](int d, int f) -> uint8_t* {
        const int wv = D > d && FT > f ? wave : 0;
        switch (6 * d + f) {
            case 0: return ring00[wv]; case 1: return ring01[wv]; case 2: return ring02[wv];
            case 3: return ring03[wv]; case 4: return ring04[wv]; case 5: return ring05[wv];
            case 6: return ring10[wv]; case 7: return ring11[wv]; case 8: return ring12[wv];
            case 9: return ring13[wv]; case 10: return ring14[wv]; case 11: return ring15[wv];
            case 12: return ring20[wv]; case 13: return ring21[wv]; case 14: return ring22[wv];
            case 15: return ring23[wv]; case 16: return ring24[wv]; case 17: return ring25[wv];
            case 18: return ring30[wv]; case 19: return ring31[wv]; case 20: return ring32[wv];
            case 21: return ring33[wv]; case 22: return ring34[wv]; default: return ring35[wv];
        }
    };
    const int tile = blockIdx.x;
    const int kp = PARTIAL ? K / (int)gridDim.y : K;  // this workgroup's share of K
    const int kw = kp / KS, k0 = (PARTIAL ? (int)blockIdx.y * kp : 0) + wave * kw, nst = kw / 128;
    const int r = lane & 15, g = lane >> 4;
    // The W resources span the workgroup's rows from this wave's k0: its 16 H
    // rows (GATED: the gate rows, and the up rows N / 2 further).
    const int64_t row0 = (int64_t)tile * 16 * H;
    const __amdgpu_buffer_rsrc_t src_lo = sk_rsrc(w + row0 * K + k0, (uint32_t)16 * H * K * 2);
    const __amdgpu_buffer_rsrc_t src_hi = sk_rsrc(w + (row0 + (GATED ? N / 2 : 0)) * K + k0, (uint32_t)16 * H * K * 2);
    uint32_t vofs[4 * H];
#pragma unroll
    for (int c = 0; c < 4 * H; ++c) {
        const int row = 4 * c + (lane >> 4), sl = lane & 15;
        vofs[c] = (uint32_t)row * K * 2 + 16u * (sl ^ (row & 15));  // chunk sl ^ (row & 15) lands in slot sl
    }
    const bf16_t* xp[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) xp[m] = x + (int64_t)min(16 * m + r, M - 1) * K + k0 + 8 * g;
    const int rot = ROT ? tile % nst : 0;
    uint4 xb[D][MT][4];
    f32x4_v acc[FT][MT];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[f][m] = f32x4_v{};
    auto load = [&](int d, int s) {
        if (ROT) {
            s += rot;
            if (s >= nst) s -= nst;
        }
#pragma unroll
        for (int f = 0; f < FT; ++f)
            ring_copy(f < H ? src_lo : src_hi, slot(d, f), vofs + 4 * (f < H ? f : f - H), 4, s * 256);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int m = 0; m < MT; ++m) xb[d][m][i] = *reinterpret_cast<const uint4*>(xp[m] + s * 128 + 32 * i);
        __builtin_amdgcn_sched_barrier(0);
    };
    // multiply the stage in slot d once its loads have landed (`later` later
    // stages' loads may stay in flight)
    auto mul = [&](int d, int later) {
        vm_wait_stages<kLoads>(later);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");  // keeps the LDS reads below the wait
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int f = 0; f < FT; ++f) {
                const uint4 a = *reinterpret_cast<const uint4*>(slot(d, f) + r * 256 + 16 * ((g + 4 * i) ^ r));
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    acc[f][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(xb[d][m][i]), acc[f][m],
                                                                        0, 0, 0);
            }
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int d = 0; d < D - 1; ++d) load(d, d);
    for (int s = 0; s + D < nst; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load((d + D - 1) % D, s + d + D - 1);
            mul(d, D - 1);
        }
    }
    load(D - 1, nst - 1);
    mul(0, D - 1);
#pragma unroll
    for (int d = 1; d < D; ++d) mul(d, D - 1 - d);
    if (KS > 1) {
        if (wave > 0)
#pragma unroll
            for (int f = 0; f < FT; ++f)
#pragma unroll
                for (int m = 0; m < MT; ++m) part[wave - 1][f][m][lane] = acc[f][m];
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int j = 0; j < KS - 1; ++j)
#pragma unroll
            for (int f = 0; f < FT; ++f)
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[f][m] += part[j][f][m][lane];
    }
    if (PARTIAL) {
        float* pp = parts + (int64_t)blockIdx.y * M * N;
#pragma unroll
        for (int f = 0; f < FT; ++f) {
            const int n = (tile * FT + f) * 16 + 4 * g;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int t = 16 * m + r;
                if (t >= M) continue;
                *reinterpret_cast<f32x4_v*>(pp + (int64_t)t * N + n) = acc[f][m];
            }
        }
        return;
    }
    if (GATED) {
        const int I = N / 2;
#pragma unroll
        for (int f = 0; f < H; ++f) {
            const int n = (tile * H + f) * 16 + 4 * g;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int t = 16 * m + r;
                if (t >= M) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)  // gate_up rounded to T, then Crane's silu * up rounded once
                    v[e] = silu(bf16_to_f32(f32_to_bf16(acc[f][m][e]))) * bf16_to_f32(f32_to_bf16(acc[f + H][m][e]));
                store4(y + (int64_t)t * I + n, v);
            }
        }
        return;
    }
#pragma unroll
    for (int f = 0; f < FT; ++f) {
        const int n = (tile * FT + f) * 16 + 4 * g;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int t = 16 * m + r;
            if (t >= M) continue;
            float v[4] = {acc[f][m][0], acc[f][m][1], acc[f][m][2], acc[f][m][3]};
            if (bias) {
                float bv[4];
                load4(bias + n, bv);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] += bv[e];
            }
            store4(y + (int64_t)t * N + n, v);
        }
    }
}

// The ring configuration for a shape: features per workgroup (16 FT), waves
// (KS) and ring depth (D); 0 when the shape does not take the ring kernel.
struct RingCfg {
    int ft, ks, d;  // features / 16 per workgroup, waves, ring depth; ft == 0: not taken
};

// Wide N (> 8192): one workgroup per CU by LDS, 48, 64 or 96 features each
// (96: two waves and a rotated k walk), the one whose busiest CU streams the
// fewest 16-feature tiles, ceil(workgroups / 256) * FT, the widest on a tie
// (least x per W byte).  GATED (a gate_up pair per workgroup) takes an even
// FT.
constexpr int kRingCUs = 256;

RingCfg ring_cfg(int64_t M, int64_t N, int64_t K, bool gated = false) {
    if (M < 1 || M > kSkMaxM || K < 1 || K > kRingMaxK || N < 1 || N > 0x7fffffff) return {0, 0, 0};
    RingCfg c{0, 0, 0};
    if (N > 8192) {
        int64_t best = 0;
        for (const RingCfg cand : {RingCfg{6, 2, 2}, RingCfg{4, 4, 2}, RingCfg{3, 4, 2}}) {
            if (N % (16 * cand.ft) || K % (128 * cand.ks * cand.d) || (gated && cand.ft % 2)) continue;
            const int64_t load = (N / (16 * cand.ft) + kRingCUs - 1) / kRingCUs * cand.ft;
            if (!c.ft || load < best) c = cand, best = load;
        }
        return c;
    }
    if (gated) return c;
    c = N <= 4096 ? RingCfg{1, 4, 4} : RingCfg{2, 2, 4};
    if (N % (16 * c.ft) || K % (128 * c.ks * c.d)) return {0, 0, 0};
    return c;
}

template <int MT, bool GATED>
void launch_ring_mt(const RingCfg& c, const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* y, int M, int N,
                    int K, hipStream_t st) {
    const dim3 grid((unsigned)(N / (16 * c.ft))), block(64 * c.ks);
    if (c.ft == 6)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, 2, 2, 6, true, GATED>), grid, block, 0, st, x, w, bias, y, M, N, K, nullptr);
    else if (c.ft == 4)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, 4, 2, 4, false, GATED>), grid, block, 0, st, x, w, bias, y, M, N, K, nullptr);
    else if (GATED)
        return;  // ring_cfg gives a gated shape an even FT
    else if (c.ft == 3)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, 4, 2, 3, false, false>), grid, block, 0, st, x, w, bias, y, M, N, K, nullptr);
    else if (c.ft == 2)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, 2, 4, 2, true, false>), grid, block, 0, st, x, w, bias, y, M, N, K, nullptr);
    else
        hipLaunchKernelGGL((ring_gemm_kernel<MT, 4, 4, 1, false, false>), grid, block, 0, st, x, w, bias, y, M, N, K, nullptr);
}

// GATED: w is gate_up [N = 2 inter, K] and y is [M, inter].
template <bool GATED>
int launch_ring(const RingCfg& c, const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* y, int M, int N, int K,
                hipStream_t st) {
    if (M <= 16)
        launch_ring_mt<1, GATED>(c, x, w, bias, y, M, N, K, st);
    else
        launch_ring_mt<2, GATED>(c, x, w, bias, y, M, N, K, st);
    return launch_status(hipGetLastError());
}

// Split-K partial products (decode rows, M <= 32): K cut into `splits`
// ranges over gridDim.y; a workgroup of KS waves takes 16 FT features of one
// range, each wave its part of the range walked in 128-wide stages through a
// ring of D slots of its own.  The shape sets the form:
//   FT: 4, 3 or 2, the one whose busiest CU streams the fewest 16-feature
//       tiles, ceil(N / (16 FT) * splits / 256) * FT, the widest on a tie;
//   KS: 1 wave when a range holds at least 3072 of K, else 2;
//   D:  3 when each wave's stage count is a multiple of 3, else 2.
// (The ring loop needs the stage count a multiple of the depth and at least
// 2; the (D - 1) stages in flight fit the 6-bit vmcnt.)  Qwen3-8B at 32 rows,
// same-box sweep of these and 4-wave forms, back to back with the weights
// read from HBM: qkv_proj [6144 x 4096] in 2 splits 12.7 -> 10.7 us (FT 3 and
// 2 waves: 256 workgroups, where 64 features and 4 waves left 64 of the 256
// CUs idle), o_proj [4096 x 4096] in 4 splits 9.4 -> 8.6 us (2 waves against
// 4), down_proj [4096 x 12288] in 4 splits 19.3 -> 18.4 us (1 wave and a ring
// of 3 against 2 waves).  {0, 0, 0} when the shape does not split this way.
RingCfg split_cfg(int64_t M, int64_t N, int64_t K, int64_t splits) {
    if (M < 1 || M > kSkMaxM || N < 32 || N > 0x7fffffff || K < 1 || splits < 2 || splits > 16 || K % splits)
        return {0, 0, 0};
    const int64_t kp = K / splits;
    if (kp > 32768) return {0, 0, 0};
    RingCfg c{0, 0, 0};
    int64_t best = 0;
    for (const int ft : {4, 3, 2}) {
        if (N % (16 * ft)) continue;
        const int64_t load = (N / (16 * ft) * splits + kRingCUs - 1) / kRingCUs * ft;
        if (!c.ft || load < best) c.ft = ft, best = load;
    }
    if (!c.ft) return {0, 0, 0};
    c.ks = kp >= 3072 ? 1 : 2;
    if (kp % (256 * c.ks)) return {0, 0, 0};  // an even number of 128-wide stages per wave
    c.d = kp / c.ks / 128 % 3 == 0 ? 3 : 2;
    return c;
}

template <int MT, int KS, int D>
void launch_split_ft(int ft, dim3 grid, const bf16_t* x, const bf16_t* w, float* part, int M, int N, int K,
                     hipStream_t st) {
    const dim3 block(64 * KS);
    if (ft == 4)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, KS, D, 4, false, false, true>), grid, block, 0, st, x, w, nullptr,
                           nullptr, M, N, K, part);
    else if (ft == 3)
        hipLaunchKernelGGL((ring_gemm_kernel<MT, KS, D, 3, false, false, true>), grid, block, 0, st, x, w, nullptr,
                           nullptr, M, N, K, part);
    else
        hipLaunchKernelGGL((ring_gemm_kernel<MT, KS, D, 2, false, false, true>), grid, block, 0, st, x, w, nullptr,
                           nullptr, M, N, K, part);
}

template <int MT>
void launch_split(const RingCfg& c, const bf16_t* x, const bf16_t* w, float* part, int M, int N, int K, int splits,
                  hipStream_t st) {
    const dim3 grid((unsigned)(N / (16 * c.ft)), (unsigned)splits);
    if (c.ks == 1 && c.d == 3)
        launch_split_ft<MT, 1, 3>(c.ft, grid, x, w, part, M, N, K, st);
    else if (c.ks == 1)
        launch_split_ft<MT, 1, 2>(c.ft, grid, x, w, part, M, N, K, st);
    else if (c.d == 3)
        launch_split_ft<MT, 2, 3>(c.ft, grid, x, w, part, M, N, K, st);
    else
        launch_split_ft<MT, 2, 2>(c.ft, grid, x, w, part, M, N, K, st);
}

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
        if (dtype == CRANE_HIP_BF16) {
            const RingCfg rc = ring_cfg(M, N, K);
            if (rc.ft)
                return launch_ring<false>(rc, (const bf16_t*)x, (const bf16_t*)w, (const bf16_t*)bias, (bf16_t*)y,
                                          (int)M, (int)N, (int)K, st);
        }
        if (dtype == CRANE_HIP_BF16 && skinny_fits(M, N, K))
            return launch_skinny((const bf16_t*)x, (const bf16_t*)w, (const bf16_t*)bias, (bf16_t*)y, (int)M, (int)N,
                                 (int)K, st);
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

    // The gated product out = T(silu(g) * u) of [g | u] = x w^T, w = gate_up
    // [2 inter, K], in one launch (ring_cfg(M, 2 inter, K, true) must take it).
    int linear_silu_mul(const void* x, const void* w, void* out, int64_t M, int64_t inter, int64_t K, hipStream_t st) {
        const RingCfg rc = ring_cfg(M, 2 * inter, K, true);
        if (rc.ft != 4 && rc.ft != 6) return CRANE_HIP_E_INVALID;  // the gated instantiations
        return launch_ring<true>(rc, (const bf16_t*)x, (const bf16_t*)w, nullptr, (bf16_t*)out, (int)M, (int)(2 * inter),
                                 (int)K, st);
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

extern "C" int crane_gemm_silu_mul_supported(int64_t M, int64_t inter, int64_t K, int dtype) {
    if (dtype != CRANE_HIP_BF16 || inter <= 0 || inter > 0x3fffffffLL) return 0;
    return crane::ring_cfg(M, 2 * inter, K, true).ft != 0;
}

extern "C" int crane_gemm_linear_silu_mul(crane_gemm* g, const void* x, const void* w, void* out, int64_t M,
                                          int64_t inter, int64_t K, int dtype, void* stream) {
    if (!g) return CRANE_HIP_E_INVALID;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (M < 0 || inter <= 0 || K <= 0 || M > 0x7fffffffLL || inter > 0x3fffffffLL || K > 0x7fffffffLL)
        return CRANE_HIP_E_INVALID;
    if (M == 0) return CRANE_HIP_OK;
    if (!x || !w || !out) return CRANE_HIP_E_INVALID;
    if (!crane::aligned16(x) || !crane::aligned16(w) || !crane::aligned16(out)) return CRANE_HIP_E_ALIGN;
    if (!crane_gemm_silu_mul_supported(M, inter, K, dtype)) return CRANE_HIP_E_INVALID;
    return g->impl.linear_silu_mul(x, w, out, M, inter, K, (hipStream_t)stream);
}

extern "C" int crane_gemm_split_supported(int64_t M, int64_t N, int64_t K, int splits, int dtype) {
    return dtype == CRANE_HIP_BF16 && crane::split_cfg(M, N, K, splits).ft != 0;
}

extern "C" int crane_gemm_linear_split(crane_gemm* g, const void* x, const void* w, float* part, int64_t M, int64_t N,
                                       int64_t K, int splits, int dtype, void* stream) {
    if (!g) return CRANE_HIP_E_INVALID;
    if (dtype != CRANE_HIP_F32 && dtype != CRANE_HIP_BF16) return CRANE_HIP_E_DTYPE;
    if (M < 0 || N <= 0 || K <= 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
        return CRANE_HIP_E_INVALID;
    if (M == 0) return CRANE_HIP_OK;
    if (!x || !w || !part) return CRANE_HIP_E_INVALID;
    if (!crane::aligned16(x) || !crane::aligned16(w) || !crane::aligned16(part)) return CRANE_HIP_E_ALIGN;
    if (dtype != CRANE_HIP_BF16) return CRANE_HIP_E_INVALID;
    const crane::RingCfg c = crane::split_cfg(M, N, K, splits);
    if (!c.ft) return CRANE_HIP_E_INVALID;
    hipStream_t st = (hipStream_t)stream;
    if (M <= 16)
        crane::launch_split<1>(c, (const crane::bf16_t*)x, (const crane::bf16_t*)w, part, (int)M, (int)N, (int)K,
                               splits, st);
    else
        crane::launch_split<2>(c, (const crane::bf16_t*)x, (const crane::bf16_t*)w, part, (int)M, (int)N, (int)K,
                               splits, st);
    return crane::launch_status(hipGetLastError());
}
