// A bandwidth probe for the roofline: one streaming read of a buffer, nothing written but one
// word a workgroup. It gives the time a single launch needs to move the same bytes as a decode
// layer's split-K pass, the practical floor that pass is compared against.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

/// Reads n16 16-byte units: thread t of workgroup b takes units 1024 b + t + 256 k (k < 4), then
/// steps by the grid; the xor of the words read goes to sink[b] so the loads stay live.
__global__ __launch_bounds__(256) void stream_read_kernel(const u4_t* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    uint32_t x = 0;
    const size_t stride = (size_t)gridDim.x * 1024;
    for (size_t i = (size_t)blockIdx.x * 1024 + threadIdx.x; i < n16; i += stride) {
        u4_t r[4];
#pragma unroll
        for (int k = 0; k < 4; k++) r[k] = i + 256 * k < n16 ? p[i + 256 * k] : (u4_t){0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; k++) x ^= r[k][0] ^ r[k][1] ^ r[k][2] ^ r[k][3];
    }
    __shared__ uint32_t red[4];
    for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

int launch_stream_read(const void* p, size_t bytes, uint32_t* sink, int grid, hipStream_t st) {
    hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, st, (const u4_t*)p, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
