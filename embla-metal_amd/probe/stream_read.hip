// Bench-only probes (libembla_probe.so, not part of the attention library). The bandwidth probe: one streaming
// read of a buffer, nothing written but one word a workgroup. It gives the time a single launch
// needs to move the same bytes as a decode layer's split-K pass, the practical floor that pass is
// compared against, and the rate a large read sustains.
//
// Two ways to keep loads in flight, both with `depth` 16-byte loads a thread before any is used:
//   regs: global_load_dwordx4 into registers, xor-folded into one word a thread;
//   lds:  gfx950's global_load_lds_dwordx4, straight into LDS (no registers held), one word of each
//         wave's region folded at the end.
// Both read every 16-byte unit exactly once (the xor of the sink words checks that for `regs`).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

namespace {

/// Thread t of workgroup b reads units (b + k' * grid) * 256 * D + 256 k + t, k < D.
template <int D>
__global__ __launch_bounds__(256) void read_regs_kernel(const u4_t* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    uint32_t x = 0;
    const size_t step = (size_t)gridDim.x * 256 * D;
    for (size_t i = (size_t)blockIdx.x * 256 * D + threadIdx.x; i < n16; i += step) {
        u4_t r[D];
#pragma unroll
        for (int k = 0; k < D; k++) r[k] = i + 256 * k < n16 ? __builtin_nontemporal_load(p + i + 256 * k) : (u4_t){0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < D; k++) x ^= r[k][0] ^ r[k][1] ^ r[k][2] ^ r[k][3];
    }
    __shared__ uint32_t red[4];
    for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

/// As read_regs_kernel, but workgroup b reads its own contiguous slice [b n16 / grid, (b + 1)
/// n16 / grid) front to back: every workgroup starts at a different place of the buffer.
template <int D>
__global__ __launch_bounds__(256) void read_chunked_kernel(const u4_t* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    uint32_t x = 0;
    const size_t lo = n16 * blockIdx.x / gridDim.x, hi = n16 * (blockIdx.x + 1) / gridDim.x;
    for (size_t i = lo + threadIdx.x; i < hi; i += 256 * D) {
        u4_t r[D];
#pragma unroll
        for (int k = 0; k < D; k++) r[k] = i + 256 * k < hi ? __builtin_nontemporal_load(p + i + 256 * k) : (u4_t){0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < D; k++) x ^= r[k][0] ^ r[k][1] ^ r[k][2] ^ r[k][3];
    }
    __shared__ uint32_t red[4];
    for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

/// As read_regs_kernel, with the loads landing in LDS (each wave its own D KB region); the whole
/// 1 KB units only (n16 a multiple of 64).
template <int D>
__global__ __launch_bounds__(256) void read_lds_kernel(const u4_t* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    __shared__ u4_t buf[4][D][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t x = 0;
    const size_t step = (size_t)gridDim.x * 256 * D;
    for (size_t i = (size_t)blockIdx.x * 256 * D + 64 * w; i < n16; i += step) {
#pragma unroll
        for (int k = 0; k < D; k++)
            if (i + 256 * k < n16)
                __builtin_amdgcn_global_load_lds((const void*)(p + i + 256 * k + lane),
                                                 (__attribute__((address_space(3))) void*)&buf[w][k][0], 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        x ^= buf[w][lane % D][lane][0];
    }
    __shared__ uint32_t red[4];
    for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
    if (lane == 0) red[w] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

extern "C" {

/// Reads `bytes` (a multiple of 16; of 1024 with lds = 1) at p (16-byte aligned) once with `grid`
/// workgroups of 256 threads, `depth` (4, 8, 16 or 32) loads in flight a thread; lds: 0 registers,
/// 1 LDS, 2 registers with a contiguous slice a workgroup; one word a workgroup to sink[grid]. 0 on success, -1 on a bad argument, -2 on a launch error.
int embla_probe_stream_read(const void* p, size_t bytes, uint32_t* sink, int grid, int depth, int lds,
                            hipStream_t stream) {
    if (!p || !sink || bytes == 0 || bytes % 16 || ((uintptr_t)p & 15) || grid <= 0 || grid > 65536) return -1;
    if (lds == 1 && bytes % 1024) return -1;
    const u4_t* q = (const u4_t*)p;
    const size_t n = bytes / 16;
#define PROBE_CASE(D)                                                                              \
    case D:                                                                                        \
        if (lds == 1) hipLaunchKernelGGL(read_lds_kernel<D>, dim3(grid), dim3(256), 0, stream, q, n, sink); \
        else if (lds == 2) hipLaunchKernelGGL(read_chunked_kernel<D>, dim3(grid), dim3(256), 0, stream, q, n, sink); \
        else hipLaunchKernelGGL(read_regs_kernel<D>, dim3(grid), dim3(256), 0, stream, q, n, sink);    \
        break;
    switch (depth) {
        PROBE_CASE(4)
        PROBE_CASE(8)
        PROBE_CASE(16)
        PROBE_CASE(32)
        default: return -1;
    }
#undef PROBE_CASE
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"

// ------------------------------------------------------------------ MFMA rate probe
// Back-to-back v_mfma_f32_32x32x16_f16 with nothing else to do: each wave keeps CH independent
// accumulator chains and runs `iters` rounds of one MFMA a chain (operands in registers, no
// memory traffic but one result word a wave). The rate it reaches is the dense fp16 matrix rate
// the chip sustains at the clock it grants under MFMA load.
namespace {
typedef _Float16 h8p_t __attribute__((ext_vector_type(8)));
typedef float f16p_t __attribute__((ext_vector_type(16)));

template <int CH>
__global__ __launch_bounds__(256) void mfma_rate_kernel(int iters, float* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    h8p_t a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)(0.001f * (lane + i));
        b[i] = (_Float16)(0.002f * (lane - i));
    }
    f16p_t acc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) acc[c] = (f16p_t){};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int c = 0; c < CH; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) s += acc[c][lane & 15];
    if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}
}  // namespace

extern "C" {

/// grid workgroups of 4 waves, each wave 4 chains x iters MFMAs (32768 flop each); sink: grid * 4
/// floats. 0 on success, -1 on a bad argument, -2 on a launch error.
int embla_probe_mfma_rate(int grid, int iters, float* sink, hipStream_t stream) {
    if (grid <= 0 || grid > 65536 || iters <= 0 || !sink) return -1;
    hipLaunchKernelGGL(mfma_rate_kernel<4>, dim3(grid), dim3(256), 0, stream, iters, sink);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
