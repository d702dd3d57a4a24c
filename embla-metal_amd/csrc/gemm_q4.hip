// The 4-bit projections either side of attention at prefill: Y = X W^T for T tokens.
//
// Follows gemm.metal:1-134 (EXPERTS = 0, GATHER = 0): X [T][ldx] bf16, W in MLX's affine 4-bit
// layout (words [O][K/8], nibble q of word c the weight of column 8c + q; bf16 scales and biases
// [O][K/64], w = s * nibble + b), Y [T][ldy] through the epilogues EPI 0-4 (gemm.metal:118-131).
// The reference stages X and the dequantised W tile (one quantisation group, 64 inputs, a step)
// and multiplies 8x8 fragments into fp32 sums; MLX's own GEMM stages W as bf16, as here.
//
// MI355X design. A workgroup computes 128 tokens x 64 rows with 4 waves, each a 64 x 32 block as
// 2 tiles of v_mfma_f32_32x32x16_bf16 (A: X rows, B: W rows, so both operands are 16-byte row
// reads of LDS); two workgroups a CU, so one wave's dequantisation overlaps another's products.
// A step is one group (64 inputs): thread t stages token row t / 2 (32 bf16) and W row t / 4 (2
// words = 16 nibbles, dequantised as s * q + b in fp32, rounded to bf16 by v_cvt_pk_bf16_f32)
// into double-buffered LDS (rows padded to 144 bytes: the 16-byte operand
// reads of 32 lanes land in distinct banks). A step's global loads go out two steps ahead (two
// register stages); one barrier a step. The += epilogue's fp32 residual is read before the first
// step, so those reads overlap the products.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

typedef __bf16 bf8v_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));

constexpr int QM = 128, QK = 64;             // tokens, inputs a step (rows: the template's QN)
constexpr int QROW = QK + 8;                 // bf16 elements an LDS row (144 bytes)

template <int QN>
struct GemmSmem {
    uint16_t x[2][QM * QROW];
    uint16_t w[2][QN * QROW];
};

template <int EPI, int QN>
__global__ __launch_bounds__(256, 2) void gemm_q4_kernel(GemmArgs a) {
    constexpr int J = QN / 64;            // 32-row tiles a wave
    constexpr int WPT = QN / 32;          // W words a staging thread: 4 or 2
    constexpr int TPR = 8 / WPT;          // staging threads a W row
    __shared__ __attribute__((aligned(16))) GemmSmem<QN> sm;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n0 = blockIdx.x * QN, m0 = blockIdx.y * QM;
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * (QN / 2);   // the wave's 64 x QN/2 block
    // X staging: chunk 256 i + tid is row 32 i + tid / 8, columns 8 (tid % 8) .. +7, so one
    // wave load reads 8 whole 128-byte row pieces
    const int sr = tid >> 3, sc = 8 * (tid & 7);
    const int wr_ = tid / TPR, wc = 8 * WPT * (tid % TPR);      // W staging: row, first column
    const char* W = (const char*)a.W;
    const int wpr = a.K / 8, gpr = a.K / 64;
    const uint16_t* xr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) xr[i] = a.X + (size_t)min(m0 + 32 * i + sr, a.T - 1) * a.ldx + sc;
    const size_t wrow = (size_t)min(n0 + wr_, a.O - 1);

    // two register stages of staged data: a step's global loads go out two steps before it is
    // stored to LDS
    struct Stage { u4_t x[4]; uint32_t w[WPT]; float s, b; };
    Stage R0, R1;
    auto load = [&](int k0, Stage& R) {
#pragma unroll
        for (int i = 0; i < 4; i++) R.x[i] = ld16(xr[i] + k0);
        const uint32_t* wp = (const uint32_t*)(W + a.wo) + wrow * wpr + k0 / 8 + WPT * (tid % TPR);
        if constexpr (WPT == 4) {
            const u4_t v = ld16(wp);
#pragma unroll
            for (int j = 0; j < 4; j++) R.w[j] = v[j];
        } else {
            const u2_t v = ld8(wp);
            R.w[0] = v[0];
            R.w[1] = v[1];
        }
        R.s = bf2f(*(const uint16_t*)(W + a.so + (wrow * gpr + k0 / 64) * 2));
        R.b = bf2f(*(const uint16_t*)(W + a.bo + (wrow * gpr + k0 / 64) * 2));
    };
    auto store = [&](int buf, const Stage& R) {
        uint16_t* xd = sm.x[buf] + sr * QROW + sc;
#pragma unroll
        for (int i = 0; i < 4; i++) *(u4_t*)(xd + 32 * i * QROW) = R.x[i];
        uint16_t* wd = sm.w[buf] + wr_ * QROW + wc;
#pragma unroll
        for (int j = 0; j < WPT; j++) {   // word j: columns wc + 8 j + q, q = 0..7
            u4_t o;
#pragma unroll
            for (int q = 0; q < 8; q += 2) {
                const bf2_t p = {(__bf16)(R.s * (float)((R.w[j] >> (4 * q)) & 0xFu) + R.b),
                                 (__bf16)(R.s * (float)((R.w[j] >> (4 * q + 4)) & 0xFu) + R.b)};
                o[q / 2] = __builtin_bit_cast(uint32_t, p);
            }
            *(u4_t*)(wd + 8 * j) = o;
        }
    };

    f16_t acc[2][J];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < J; j++) acc[i][j] = (f16_t){};
    const int fr = lane & 31, fk = 8 * (lane >> 5);   // operand row within a tile, k offset
    auto compute = [&](int buf) {   // every operand of the step read first, then the products
        bf8v_t fa[QK / 16][2], fb[QK / 16][J];
#pragma unroll
        for (int kk = 0; kk < QK / 16; kk++) {
#pragma unroll
            for (int i = 0; i < 2; i++)
                fa[kk][i] = *(const bf8v_t*)(sm.x[buf] + (wm + 32 * i + fr) * QROW + 16 * kk + fk);
#pragma unroll
            for (int j = 0; j < J; j++)
                fb[kk][j] = *(const bf8v_t*)(sm.w[buf] + (wn + 32 * j + fr) * QROW + 16 * kk + fk);
        }
#pragma unroll
        for (int kk = 0; kk < QK / 16; kk++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < J; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
    };
    const int steps = a.K / QK;
    // step st computes buffer st & 1 and stores step st + 1 (loaded at st - 1) into the other;
    // the stage it frees is refilled with step st + 2. Unrolled by two so the stages are static;
    // loads past the last step repeat it and their stores go to a buffer no one reads again, so a
    // step's products and the next step's dequantisation share one block for the scheduler.
    const int last = QK * (steps - 1);
    // EPI 2 (+=): the residual's items are requested first, so that their reads overlap the
    // products instead of following them
    float yp[EPI == 2 ? 2 : 1][EPI == 2 ? J : 1][16];
    if constexpr (EPI == 2) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int n = min(n0 + wn + 32 * j + fr, a.O - 1);
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = min(m0 + wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3), a.T - 1);
                    yp[i][j][e] = ((const float*)a.Y)[(size_t)m * a.ldy + n];
                }
            }
    }
    load(0, R0);
    load(min(QK, last), R1);
    store(0, R0);
    __syncthreads();
    for (int st = 0; st < steps; st += 2) {
        load(min(QK * (st + 2), last), R0);
        compute(0);
        store(1, R1);
        __syncthreads();
        if (st + 1 >= steps) break;
        load(min(QK * (st + 3), last), R1);
        compute(1);
        store(0, R0);
        __syncthreads();
    }

    // epilogue: tile (i, j) item e of lane l is token wm + 32 i + 8 (e / 4) + 4 (l / 32) + e % 4,
    // row wn + 32 j + l % 32
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int n = n0 + wn + 32 * j + fr;
            if (n >= a.O) continue;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m >= a.T) continue;
                const float v = acc[i][j][e];
                const size_t at = (size_t)m * a.ldy + n;
                if constexpr (EPI == 0) ((uint16_t*)a.Y)[at] = f2bf(v);
                else if constexpr (EPI == 1) {
                    const float t = fmaxf(bf2f(f2bf(v)), 0.0f);
                    ((uint16_t*)a.Y)[at] = f2bf(t * t);
                } else if constexpr (EPI == 2) ((float*)a.Y)[at] = yp[i][j][e] + bf2f(f2bf(v));
                else if constexpr (EPI == 3) ((float*)a.Y)[at] = bf2f(f2bf(v));
                else ((float*)a.Y)[at] = v;
            }
        }
}

template <int QN>
int launch_gemm_q4_tile(const GemmArgs& a, int epi, hipStream_t st) {
    const dim3 grid((a.O + QN - 1) / QN, (a.T + QM - 1) / QM), block(256);
    switch (epi) {
        case 0: hipLaunchKernelGGL((gemm_q4_kernel<0, QN>), grid, block, 0, st, a); break;
        case 1: hipLaunchKernelGGL((gemm_q4_kernel<1, QN>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((gemm_q4_kernel<2, QN>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((gemm_q4_kernel<3, QN>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((gemm_q4_kernel<4, QN>), grid, block, 0, st, a); break;
        default: return EMBLA_ERR_INVALID;
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// 64 rows a workgroup (two workgroups a CU); 128 rows measured the same (416 against 423 TFLOP/s
// for C5's q/k/v + o projections) with 170 VGPRs.
int launch_gemm_q4(const GemmArgs& a, int epi, hipStream_t st) { return launch_gemm_q4_tile<64>(a, epi, st); }

}  // namespace embla
