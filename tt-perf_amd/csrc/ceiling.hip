// ceiling.hip — libttperf_ceiling: the practical HBM ceilings that bench.py measures beside
// the optimizer step, on the same GPU in the same run.
//
//   ttpc_copy_nt  streams `n16` 16-byte words from src to dst: half reads, half writes, the
//                 read/write mix of the fused update, which reads and writes its fp32 state
//                 in equal parts with non-temporal 16-byte loads and stores;
//   ttpc_copy_nt64  the same copy in 64-lane blocks, one 1 KiB tile each (straight-line):
//                 the fastest copy measured on MI355X (6.7 TB/s against 6.5 for 256-lane
//                 blocks at 1.7 and 10.8 GB, same runs);
//   ttpc_read_nt  reads `n16` 16-byte words, the norm pass's read-only pattern, and folds
//                 them into a sum that is stored only if it equals a sentinel, so the loads
//                 cannot be dropped.
//
// Both kernels move one 16-byte word per thread per iteration over tiles of 256 words, one
// tile per 256-thread block per iteration; `grid` blocks walk the tiles (grid <= 0: one block
// per tile, a straight-line launch).  Of the forms measured on MI355X for a 1.7 GB stream
// (unrolled 2-8 words per thread, block tiles, grids of 4-512 blocks per CU, cached or
// non-temporal), the straight-line copy was the fastest copy (6.5 TB/s) and the grid-stride
// read over 8 blocks per CU the fastest read (7.1 TB/s); bench.py launches those.
//
// They return the launch's hipError_t (0 on success).  Measurement support only: not part of
// the optimizer's C ABI (include/ttperf/ttperf.h), and nothing in a step uses them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint64_t kTile = 256;  // 16-byte words per tile = threads per block

template <int kLanes>
__global__ __launch_bounds__(kLanes) void copy_nt_kernel(const f32x4* __restrict__ src,
                                                         f32x4* __restrict__ dst, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kLanes + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kLanes)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ __launch_bounds__(256) void read_nt_kernel(const f32x4* __restrict__ src, uint64_t n,
                                                      float* __restrict__ sink) {
    float s = 0.0f;
    for (uint64_t i = (uint64_t)blockIdx.x * kTile + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kTile) {
        const f32x4 v = __builtin_nontemporal_load(src + i);
        s += (v.x + v.y) + (v.z + v.w);
    }
    if (s == 1234.5f) sink[0] = s;
}

// blocks of a launch: `grid`, or one per tile of `tile` words (one word per lane), at most as
// many as keep the launch under 2^32 work-items; larger streams loop
uint32_t blocks(uint64_t n16, int grid, uint64_t tile = kTile) {
    if (grid > 0) return (uint32_t)grid;
    const uint64_t cap = ((1ull << 32) - 1) / tile;
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>((n16 + tile - 1) / tile, cap));
}

}  // namespace

extern "C" {

int ttpc_copy_nt(const void* src, void* dst, uint64_t n16, int grid, void* stream) {
    if (n16 && (!src || !dst)) return (int)hipErrorInvalidValue;
    if (((uintptr_t)src | (uintptr_t)dst) & 15u) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_nt_kernel<256>, dim3(blocks(n16, grid)), dim3(256), 0,
                       (hipStream_t)stream, (const f32x4*)src, (f32x4*)dst, n16);
    return (int)hipGetLastError();
}

int ttpc_copy_nt64(const void* src, void* dst, uint64_t n16, void* stream) {
    if (n16 && (!src || !dst)) return (int)hipErrorInvalidValue;
    if (((uintptr_t)src | (uintptr_t)dst) & 15u) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_nt_kernel<64>, dim3(blocks(n16, 0, 64)), dim3(64), 0,
                       (hipStream_t)stream, (const f32x4*)src, (f32x4*)dst, n16);
    return (int)hipGetLastError();
}

int ttpc_read_nt(const void* src, uint64_t n16, int grid, void* stream, float* sink) {
    if (n16 && !src) return (int)hipErrorInvalidValue;
    if (!sink || ((uintptr_t)src & 15u)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(read_nt_kernel, dim3(blocks(n16, grid)), dim3(256), 0,
                       (hipStream_t)stream, (const f32x4*)src, n16, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
