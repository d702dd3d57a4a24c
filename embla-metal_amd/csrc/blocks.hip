// Prefix-cache block copies: the full layers' int8 K/V of 128 positions and the sliding layers'
// ring slots of 128 positions, between the layer caches and a stored block buffer, in one launch.
//
// Follows Engine.fullSpans / windowSpans / copy (Sources/EmblaMetal/PrefixCache.swift:147-200):
// per layer, k then v; per kv head the block's rows, then (int8 caches) each head's scales; the
// stored buffer holds the spans back to back. In the MFMA tile layout a 128-position block of one
// head is four whole 32-key tiles, contiguous, so the spans keep the reference's shape and order:
// one a head for the rows, one a head for the scales. The reference issues one blit a span (up to
// 16 a layer); here every span of every layer is one grid, a 16-byte unit a thread.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

__global__ __launch_bounds__(256) void block_copy_kernel(BlockCopyArgs a) {
    const int reg = blockIdx.y;   // layer reg / 2, k (0) or v (1)
    const size_t rowu = (size_t)a.row_units, scu = (size_t)a.scale_units;
    const size_t per = (size_t)a.n_kv * (rowu + scu);   // units a region
    const size_t u = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= per) return;
    char* base = a.cache + a.off[reg];
    size_t at;
    if (u < (size_t)a.n_kv * rowu) {   // head h's rows: four whole tiles from position p0
        const int h = (int)(u / rowu);
        at = tile_base(h, a.max_s, a.p0, a.elem) + (u % rowu) * 16;
    } else {                           // head h's scales of positions p0 .. p0 + 127
        const size_t v = u - (size_t)a.n_kv * rowu;
        const int h = (int)(v / scu);
        at = (size_t)a.n_kv * a.max_s * 128 * a.elem + ((size_t)h * a.max_s + a.p0) * a.scale_bytes + (v % scu) * 16;
    }
    u4_t* c = (u4_t*)(base + at);
    u4_t* s = (u4_t*)(a.stored + ((size_t)reg * per + u) * 16);
    if (a.save) *s = *c;
    else *c = *s;
}

int launch_block_copy(const BlockCopyArgs& a, hipStream_t st) {
    const size_t per = (size_t)a.n_kv * (a.row_units + a.scale_units);
    const dim3 grid((unsigned)((per + 255) / 256), 2 * a.n_layers);
    hipLaunchKernelGGL(block_copy_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
