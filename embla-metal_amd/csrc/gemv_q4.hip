// The 4-bit projections either side of attention at decode: y = W x for one token over stacked
// segments (q, k and v in one launch; or the o-projection accumulating into the residual).
//
// Follows gemv.metal:1-92 (MIX = 0) and GemvRows (common.metal:104-152): W in MLX's affine 4-bit
// layout (words [O][K/8], nibble q of word c the weight of column 8c + q; bf16 scales and biases
// [O][K/64], w = s * nibble + b), segments as the reference's Seg records (rows stacked, each with
// its own input and output offset), epilogues EPI 0-4 (gemv.metal:77-88).
//
// MI355X design. A wave takes RW rows (one, at launch); lane l holds 4 words (16 bytes, columns
// 32 l .. 32 l + 31) of each 2048-column span, so a row is one coalesced 1 KB load a span, and the
// rows' words, scales and biases are requested before x is read. Two columns go through one v_dot2_f32_bf16:
// the nibbles of columns 8j + k and 8j + k + 4 of word j sit 16 bits apart, so
// (word >> 4k) & 0x000F000F | 0x43004300 is the bf16 pair (128 + q, 128 + q') exactly (bf16 holds
// integers to 256), and x is paired the same way once a workgroup (v_perm_b32) as it is staged
// into LDS, with the sums of its 8-column chunks (8.20 -> 7.80 us for the q/k/v + o rows of a
// decode layer, against pairing once a wave after the loads land). The 128 folds into the
// group's bias term: sum (s q + b) x = s sum (128 + q) x + (b - 128 s) sum x. The sums are fp32.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

typedef __bf16 bf2v_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2v_t, a), __builtin_bit_cast(bf2v_t, b), c, false);
}

/// The sum over the wave's 64 lanes, in every lane: within 16-lane rows by DPP (quad xor 1, xor 2,
/// then the half-row and row mirrors), then the 4 rows' totals by readlane. No LDS round trips (a
/// chain of ds_bpermute shuffles waits on LDS each step).
__device__ __forceinline__ float wave_total(float v) {
    auto dpp = [](float x, int ctrl) -> float {
        const int xi = __builtin_bit_cast(int, x);
        switch (ctrl) {   // constant after inlining
            case 0: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0xB1, 0xF, 0xF, false));
            case 1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x4E, 0xF, 0xF, false));
            case 2: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x141, 0xF, 0xF, false));
            default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x140, 0xF, 0xF, false));
        }
    };
    v += dpp(v, 0);   // quad_perm [1, 0, 3, 2]
    v += dpp(v, 1);   // quad_perm [2, 3, 0, 1]: every lane of a quad holds its sum
    v += dpp(v, 2);   // row_half_mirror: the other quad of the 8
    v += dpp(v, 3);   // row_mirror: the other 8 of the row
    return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

template <int EPI, int RW>
__global__ __launch_bounds__(256) void gemv_q4_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + w) * RW;   // the wave's first stacked row
    int si = 0, start = 0;
    while (si < a.nseg && row0 >= (int)a.seg[si].end) { start = (int)a.seg[si].end; si++; }
    if (si >= a.nseg) return;
    const GemvSeg sg = a.seg[si];
    const int r0 = row0 - start;   // the segment's row; a segment's rows come in whole waves
    const int spans = a.K / 2048, wpr = a.K / 8, gpr = a.K / 64;   // words, groups a row
    const char* W = (const char*)a.W;

    constexpr int MAXS = 2;   // spans a lane keeps in registers (K <= 4096)
    u4_t wd[RW][MAXS];
    float sc[RW][MAXS], bi[RW][MAXS];
#pragma unroll
    for (int u = 0; u < RW; u++)
#pragma unroll
        for (int sp = 0; sp < MAXS; sp++)
            if (sp < spans) {
                const size_t r = (size_t)(r0 + u);
                wd[u][sp] = ld16_stream(W + sg.w + (r * wpr + 256 * sp + 4 * lane) * 4);   // read once
                sc[u][sp] = bf2f(*(const uint16_t*)(W + sg.s + (r * gpr + 32 * sp + lane / 2) * 2));
                bi[u][sp] = bf2f(*(const uint16_t*)(W + sg.b + (r * gpr + 32 * sp + lane / 2) * 2));
            }
    // EPI 2 (+= into fp32): the residual of the lane's row (lanes >= RW: the wave's first row,
    // unused) is requested with the weights, not as a round trip after the products
    float yprev = 0.0f;
    if constexpr (EPI == 2) yprev = ((const float*)a.Y)[sg.y + (size_t)(r0 + (lane < RW ? lane : 0))];
    // x: the lane's 32 columns of each span as bf16 pairs (8j + k, 8j + k + 4), and their sum.
    // Paired once a workgroup, in staging: thread t pairs the 8 columns 8t .. 8t + 7 of each span
    // and sums them (its 4 waves' rows share one segment: segment ends are multiples of 4 rows),
    // after the weights are requested; a lane then reads its 4 chunks' pairs and sums.
    const uint16_t* X = (const uint16_t*)a.X + sg.x;
    __shared__ u4_t xq[MAXS * 256];
    __shared__ float xsl[MAXS * 256];
#pragma unroll
    for (int sp = 0; sp < MAXS; sp++) {
        if (sp < spans) {
            const u4_t v = ld16(X + 2048 * sp + 8 * threadIdx.x);
            u4_t pr;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) s += bf2f((uint16_t)(v[i] & 0xFFFF)) + bf2f((uint16_t)(v[i] >> 16));
#pragma unroll
            for (int k = 0; k < 4; k++)   // columns 8t + k (dword k / 2), 8t + k + 4 (dword k / 2 + 2), half k % 2
                pr[k] = __builtin_amdgcn_perm(v[(k >> 1) + 2], v[k >> 1], (k & 1) ? 0x07060302u : 0x05040100u);
            xq[256 * sp + threadIdx.x] = pr;
            xsl[256 * sp + threadIdx.x] = s;
        }
    }
    __syncthreads();
    uint32_t xp[MAXS][16];
    float xs[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; sp++) {
        if (sp < spans) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const u4_t pr = xq[256 * sp + 4 * lane + j];
#pragma unroll
                for (int k = 0; k < 4; k++) xp[sp][4 * j + k] = pr[k];
            }
            const f4_t s4 = *(const f4_t*)&xsl[256 * sp + 4 * lane];
            xs[sp] = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        }
    }
    float acc[RW];
#pragma unroll
    for (int u = 0; u < RW; u++) {
        float r = 0.0f;
#pragma unroll
        for (int sp = 0; sp < MAXS; sp++) {
            if (sp < spans) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        d = dot2_bf16(((wd[u][sp][j] >> (4 * k)) & 0x000F000Fu) | 0x43004300u, xp[sp][4 * j + k], d);
                r += sc[u][sp] * d + (bi[u][sp] - 128.0f * sc[u][sp]) * xs[sp];
            }
        }
        acc[u] = wave_total(r);
    }
    if (lane < RW) {   // lane u writes row u
        float v = acc[0];
#pragma unroll
        for (int u = 1; u < RW; u++) v = lane == u ? acc[u] : v;
        const size_t at = sg.y + (size_t)(r0 + lane);
        if constexpr (EPI == 0) ((uint16_t*)a.Y)[at] = f2bf(v);
        else if constexpr (EPI == 1) {
            const float t = fmaxf(bf2f(f2bf(v)), 0.0f);
            ((uint16_t*)a.Y)[at] = f2bf(t * t);
        } else if constexpr (EPI == 2) ((float*)a.Y)[at] = yprev + bf2f(f2bf(v));
        else if constexpr (EPI == 3) ((float*)a.Y)[at] = bf2f(f2bf(v));
        else ((float*)a.Y)[at] = v;
    }
}

template <int RW>
int launch_gemv_q4_rw(const GemvArgs& a, int epi, hipStream_t st) {
    const int rows = (int)a.seg[a.nseg - 1].end;
    const dim3 grid((rows + 4 * RW - 1) / (4 * RW)), block(256);
    switch (epi) {
        case 0: hipLaunchKernelGGL((gemv_q4_kernel<0, RW>), grid, block, 0, st, a); break;
        case 1: hipLaunchKernelGGL((gemv_q4_kernel<1, RW>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((gemv_q4_kernel<2, RW>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((gemv_q4_kernel<3, RW>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((gemv_q4_kernel<4, RW>), grid, block, 0, st, a); break;
        default: return EMBLA_ERR_INVALID;
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// One row a wave: 3072 q/k/v rows are 768 workgroups, enough requests in flight to cover every
// CU (48-layer q/k/v + o: 4 rows a wave 11.1 us a layer, 2 rows 9.1 us, 1 row 8.4 us; 2-wave
// workgroups 9.1 us, x read by every wave from L2 instead of once into LDS 8.59 against 8.56 us;
// the weights' nontemporal loads 8.44-8.45 against 8.55-8.56 us).
int launch_gemv_q4(const GemvArgs& a, int epi, hipStream_t st) { return launch_gemv_q4_rw<1>(a, epi, st); }

}  // namespace embla
