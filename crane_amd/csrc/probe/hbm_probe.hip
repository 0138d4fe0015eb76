// hbm_probe.hip -- measurement helper for bench.py, not part of the
// attention library: the HBM read rate this GPU reaches with the decode
// kernel's access pattern and load form -- one workgroup per contiguous span
// (the decode kernel's is a 256-key chunk: 64 KiB of K, then 64 KiB of V),
// every 16-byte load of the span in flight at once, buffer loads with the
// non-temporal policy.  bench.py reports the decode call's rate against it
// beside the 8 TB/s datasheet peak.  Built into its own libcrane_probe.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;

typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

// Workgroup w reads the span [w S, (w + 1) S), S = 16 L kThreads bytes: each
// thread issues its L loads (16 bytes each, kThreads * 16 bytes apart, so a
// wave's load covers 1 KiB in one piece) before using any, then folds the
// words by xor into one value per workgroup, so no load is dead.  Bytes past
// the buffer read as zero (bounds-checked buffer loads): no branch.
template <int L>
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const uint8_t* __restrict__ src, uint32_t bytes,
                                                              uint32_t* __restrict__ sink) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)bytes, 0x00020000);
    const uint32_t base = blockIdx.x * (uint32_t)(16 * L * kThreads) + 16u * threadIdx.x;
    u32x4_v v[L];
#pragma unroll
    for (int u = 0; u < L; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(base + 16u * kThreads * u), 0, 2);
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < L; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    __shared__ uint32_t part[kThreads / 64];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= __shfl_xor(acc, m);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace

// Workgroups (and sink words) a read of `bytes` takes with `loads` 16-byte
// loads per thread: ceil(bytes / (4096 loads)).
extern "C" int64_t crane_probe_workgroups(int64_t bytes, int loads) {
    const int64_t span = 16LL * kThreads * loads;
    return loads > 0 && bytes > 0 ? (bytes + span - 1) / span : 0;
}

// Reads `bytes` bytes (a multiple of 16, at most 2^31 - 2^20) from the
// 16-byte-aligned `src` on `stream`, `loads` (8, 16 or 32) loads per thread;
// sink holds crane_probe_workgroups(bytes, loads) words.  0, or -1 for
// arguments out of range, or -2 when the launch fails.
extern "C" int crane_probe_read(const void* src, int64_t bytes, uint32_t* sink, int loads, void* stream) {
    if (!src || !sink || bytes < 16 || bytes % 16 || bytes > 0x7ff00000LL || ((uintptr_t)src & 15) ||
        (loads != 8 && loads != 16 && loads != 32))
        return -1;
    const dim3 grid((unsigned)crane_probe_workgroups(bytes, loads));
    hipStream_t st = (hipStream_t)stream;
    if (loads == 8)
        hipLaunchKernelGGL(read_probe_kernel<8>, grid, dim3(kThreads), 0, st, (const uint8_t*)src, (uint32_t)bytes, sink);
    else if (loads == 16)
        hipLaunchKernelGGL(read_probe_kernel<16>, grid, dim3(kThreads), 0, st, (const uint8_t*)src, (uint32_t)bytes, sink);
    else
        hipLaunchKernelGGL(read_probe_kernel<32>, grid, dim3(kThreads), 0, st, (const uint8_t*)src, (uint32_t)bytes, sink);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
