// Key selection for the sparse layers: the ReLU² index scorer and the exact radix top-k.
//
// select_topk_kernel restates select_keys (Sources/EmblaMetal/Kernels/attention.metal:647-744):
// among keys [0, n = S - recent) the topk with the largest order_bits(score) (order_bits,
// attention.metal:657-660), found by four 8-bit MSB-first radix passes, then an ordered
// compaction: keys above the topk-th value in index order, then the first keys equal to it in
// index order, then the recent keys n .. S-1. The output is bit-exact with the reference's
// definition (order included). MI355X design: one 1024-thread workgroup a set stages all n scores'
// order bits in LDS once (gfx950 has 160 KB a CU; 32K scores take 132 KB), so the four passes and
// the compaction read LDS, not HBM.
//
// index_scores_kernel computes score_j = Σ_h w_h relu(q_h·k_j)² (the BASELINE configs' indexer,
// 64-dim fp16 index heads). Its fp32 order is part of the spec, so the top-k is reproducible: lane
// k (0..7) of a key takes dims 8k .. 8k + 7 as an fma chain from 0 (fp16 products are exact in
// fp32); the 8 chains combine as ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)); then
// r = max(dot, 0), s = fma(w_h, r * r, s) over h = 0 .. from s = 0. oracle/oracle.c restates it.
#include "common.hpp"
#include "embla_internal.hpp"

#pragma clang fp contract(off)

namespace embla {

constexpr int SEL_T = 1024;            // threads of the select workgroup
constexpr int SEL_MAXN = 32768 + 256;  // candidates it stages in LDS

__device__ __forceinline__ uint32_t order_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ int lds_pad(int j) { return j + (j >> 5); }   // conflict-free segments

/// Exclusive prefix sum over the 1024 threads, and the total.
__device__ __forceinline__ uint32_t block_scan_excl(uint32_t v, uint32_t* buf, uint32_t& total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const uint32_t o = __shfl_up(incl, s, 64);
        if (lane >= s) incl += o;
    }
    if (lane == 63) buf[w] = incl;
    __syncthreads();
    if (w == 0) {
        uint32_t x = lane < 16 ? buf[lane] : 0u, xi = x;
#pragma unroll
        for (int s = 1; s < 16; s <<= 1) {
            const uint32_t o = __shfl_up(xi, s, 64);
            if (lane >= s) xi += o;
        }
        if (lane < 16) buf[lane] = xi - x;
        if (lane == 15) buf[16] = xi;
    }
    __syncthreads();
    const uint32_t r = buf[w] + incl - v;
    total = buf[16];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(SEL_T) void select_topk_kernel(const float* __restrict__ scores, int score_stride,
                                                            uint32_t* __restrict__ idx, int idx_stride, int S,
                                                            int topk, int recent) {
    __shared__ uint32_t keys[SEL_MAXN + SEL_MAXN / 32];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t buf[17];
    __shared__ uint32_t sel[2];
    const int set = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* sc = scores + (size_t)set * score_stride;
    uint32_t* out = idx + (size_t)set * idx_stride;
    const int n = S - recent;

    // one round of independent loads: 16 bytes a thread a step, every step issued before the stores
    constexpr int NV = (SEL_MAXN + 4 * SEL_T - 1) / (4 * SEL_T);
    if (((uintptr_t)sc & 15) == 0) {
        u4_t v[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = 4 * (tid + SEL_T * i);
            v[i] = j + 3 < n ? ld16(sc + j) : (u4_t){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int j = 4 * (tid + SEL_T * i);
            if (j + 3 < n) {
#pragma unroll
                for (int e = 0; e < 4; e++) keys[lds_pad(j + e)] = order_bits(__uint_as_float(v[i][e]));
            } else {
                for (int e = 0; e < 4 && j + e < n; e++) keys[lds_pad(j + e)] = order_bits(sc[j + e]);
            }
        }
    } else {
        for (int j = tid; j < n; j += SEL_T) keys[lds_pad(j)] = order_bits(sc[j]);
    }
    const int per = (n + SEL_T - 1) / SEL_T, s0 = tid * per, s1 = min(n, s0 + per);
    __syncthreads();

    uint32_t prefix = 0, mask = 0, k = (uint32_t)topk;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int j = s0; j < s1; j++) {
            const uint32_t b = keys[lds_pad(j)];
            if ((b & mask) == prefix) atomicAdd(&hist[(b >> shift) & 255u], 1u);
        }
        __syncthreads();
        // counts at or above each digit, from the top: the digit whose bucket holds the k-th largest
        if (w == 0) {
            uint32_t c[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) { c[i] = hist[255 - (lane * 4 + i)]; s += c[i]; }
            uint32_t above = s;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = __shfl_up(above, d, 64);
                if (lane >= d) above += o;
            }
            above -= s;   // exclusive
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (above < k && above + c[i] >= k) { sel[0] = 255u - (uint32_t)(lane * 4 + i); sel[1] = above; }
                above += c[i];
            }
        }
        __syncthreads();
        prefix |= sel[0] << shift;
        mask |= 255u << shift;
        k -= sel[1];
        __syncthreads();
    }
    // prefix is the topk-th largest; every key above it, then the first k equal to it
    uint32_t gt = 0, eq = 0;
    for (int j = s0; j < s1; j++) {
        const uint32_t b = keys[lds_pad(j)];
        gt += b > prefix;
        eq += b == prefix;
    }
    uint32_t ngt, neq;
    const uint32_t gpos = block_scan_excl(gt, buf, ngt);
    uint32_t epos = block_scan_excl(eq, buf, neq);
    uint32_t gp = gpos;
    for (int j = s0; j < s1; j++) {
        const uint32_t b = keys[lds_pad(j)];
        if (b > prefix) out[gp++] = (uint32_t)j;
        else if (b == prefix) {
            if (epos < k) out[ngt + epos] = (uint32_t)j;
            epos++;
        }
    }
    for (int j = tid; j < recent; j += SEL_T) out[topk + j] = (uint32_t)(n + j);
}

int launch_select_topk(const float* scores, int score_stride, uint32_t* idx, int idx_stride, int S, int n_sets,
                       int topk, int recent, hipStream_t st) {
    if (S - recent > SEL_MAXN) return EMBLA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(select_topk_kernel, dim3(n_sets), dim3(SEL_T), 0, st, scores, score_stride, idx, idx_stride,
                       S, topk, recent);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// ------------------------------------------------------------------ index scorer
/// One set of n_ih (<= 4) fp16 index queries [n_ih][64] and weights; keys ki [n][64] fp16.
/// A wave takes 64 keys a round: load j (16 bytes a lane) covers keys 8j .. 8j + 7, lane l holding
/// key 8j + l / 8, dims 8 (l % 8) .. + 7, so every load of the wave reads 1 KB contiguous.
template <int NIH>
__global__ __launch_bounds__(256) void index_scores_kernel(const uint16_t* __restrict__ qi, const float* __restrict__ wt,
                                                           const uint16_t* __restrict__ ki, float* __restrict__ scores,
                                                           int n) {
    const int lane = threadIdx.x & 63, kq = lane & 7;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;
    float q[NIH][8], w[NIH];
#pragma unroll
    for (int h = 0; h < NIH; h++) {
        const u4_t r = ld16(qi + h * 64 + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[h][2 * i] = h2f((uint16_t)(r[i] & 0xFFFF));
            q[h][2 * i + 1] = h2f((uint16_t)(r[i] >> 16));
        }
        w[h] = wt[h];
    }
    for (int base = wave * 64; base < n; base += nwaves * 64) {
        u4_t raw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int key = base + 8 * j + (lane >> 3);
            raw[j] = key < n ? ld16(ki + (size_t)key * 64 + 8 * kq) : (u4_t){0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float kf[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kf[2 * i] = h2f((uint16_t)(raw[j][i] & 0xFFFF));
                kf[2 * i + 1] = h2f((uint16_t)(raw[j][i] >> 16));
            }
            float s = 0.0f;
#pragma unroll
            for (int h = 0; h < NIH; h++) {
                float c = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) c = __builtin_fmaf(q[h][d], kf[d], c);
                c = c + shfl_xor(c, 1);
                c = c + shfl_xor(c, 2);
                c = c + shfl_xor(c, 4);
                const float r = fmaxf(c, 0.0f);
                const float r2 = r * r;
                s = __builtin_fmaf(w[h], r2, s);
            }
            const int key = base + 8 * j + (lane >> 3);
            if (kq == 0 && key < n) scores[key] = s;
        }
    }
}

int launch_index_scores(const uint16_t* qi, const float* w, const uint16_t* ki, float* scores, int n, int n_ih,
                        hipStream_t st) {
    const int waves = (n + 63) / 64;
    int blocks = (waves + 3) / 4;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    switch (n_ih) {
        case 1: hipLaunchKernelGGL(index_scores_kernel<1>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n); break;
        case 2: hipLaunchKernelGGL(index_scores_kernel<2>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n); break;
        case 4: hipLaunchKernelGGL(index_scores_kernel<4>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n); break;
        default: return EMBLA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
