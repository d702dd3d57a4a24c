// The int8 quantisation of one K or V row (128 dims held two a lane by a wave64), shared by the
// quantise-and-append kernel and the decode step that appends the new token itself, so both write
// the same bytes. Follows write_row8 (Sources/EmblaMetal/Kernels/common.metal:72-84):
//   v_i = x_i (bf16-rounded when the input is bf16), a = max |v_i|, q_i = rint(v_i * (127 / a))
//   (0 when a = 0), scale = a / 127; with norm the row is first RMS-normed without gains
//   (r = 1 / sqrt(Σx² / 128 + 2^-23), the squares summed in a fixed butterfly).
// No fma contraction here: the oracle restates these operations one rounding at a time.
#pragma once
#include "common.hpp"

namespace embla {

constexpr float EPS32 = 1.1920929e-07f;

/// Sum (max) over the wave as the xor butterfly 32 .. 1 (v = v + v of lane xor m) gives it.
__device__ __forceinline__ float wave_sum_bfly(float v) {
    return wave_bfly(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max_bfly(float v) {
    return wave_bfly(v, [](float a, float b) { return fmaxf(a, b); });
}

/// RMS factor of a head held two dims a lane, in the fixed order the oracle restates.
__device__ __forceinline__ float rms_factor(float x0, float x1) {
#pragma clang fp contract(off)
    const float s0 = x0 * x0, s1 = x1 * x1;
    const float ss = wave_sum_bfly(s0 + s1);
    return 1.0f / sqrtf(ss / 128.0f + EPS32);
}

/// Σx² of a head row whose lane (n, g = lane >> 4) holds dims 32g .. 32g + 31 in x[32] (every lane
/// of a group n holds the same row): the same value, bit for bit, as rms_factor's butterfly over
/// dim pairs (2l, 2l + 1). Pair l = 16g + i is this lane's i; the butterfly's levels xor 32 and 16
/// cross lane groups (lane xor 32, 16), the levels 8 .. 1 stay inside the lane.
__device__ __forceinline__ float sumsq_grouped32(const float* x) {
#pragma clang fp contract(off)
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float a = x[2 * i] * x[2 * i], b = x[2 * i + 1] * x[2 * i + 1];
        v[i] = a + b;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = sum_xor32(v[i]);
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = sum_xor16(v[i]);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1)
#pragma unroll
        for (int i = 0; i < m; i++) v[i] = v[i] + v[i + m];
    return v[0];
}

/// RoPE's cosine and sine for dim d (< 32) at position pos (common.metal:39-47), with the rounding
/// the oracle fixes: f_d = 10000^(-d/32) rounded to fp32, theta = -(float)pos * f_d in fp32, then
/// cos and sin of that theta evaluated in fp64 and rounded to fp32.
__device__ __forceinline__ void rope_cs(int pos, int d, float& c, float& s) {
#pragma clang fp contract(off)
    const float f = (float)exp2(-(double)d / 32.0 * 13.287712379549449);
    const float th = -(float)pos * f;
    double sd, cd;
    sincos((double)th, &sd, &cd);
    c = (float)cd;
    s = (float)sd;
}

/// Quantises a row held two dims a lane (x0, x1 = dims 2 lane, 2 lane + 1): the int8 pair and the
/// row's absmax a (scale a / 127).
__device__ __forceinline__ float quant_pair(float x0, float x1, bool norm, bool round_bf, int& q0, int& q1) {
#pragma clang fp contract(off)
    if (norm) {
        const float r = rms_factor(x0, x1);
        x0 = x0 * r;
        x1 = x1 * r;
    }
    if (round_bf) { x0 = bf2f(f2bf(x0)); x1 = bf2f(f2bf(x1)); }
    const float am = wave_max_bfly(fmaxf(fabsf(x0), fabsf(x1)));
    const float inv = am > 0.0f ? 127.0f / am : 0.0f;
    q0 = (int)rintf(x0 * inv);
    q1 = (int)rintf(x1 * inv);
    return am;
}

/// Stores a quantised pair of (kv head h, position pos) into an int8 region: rows in the MFMA tile
/// layout (K's two bytes adjacent, V's not) or plain 128-byte rows, the scale a / 127 (fp32 or
/// fp16) at its place after the rows (lane 0 writes it).
__device__ __forceinline__ void store_pair8(int8_t* rows, int n_kv, int max_s, int h, int pos, bool is_v, bool row_major,
                                            bool scale32, int q0, int q1, float am, int lane) {
    const size_t nrow = (size_t)n_kv * max_s * HD;
    if (lane == 0) {
        const size_t si = (size_t)h * max_s + pos;
        if (scale32) ((float*)(rows + nrow))[si] = am / 127.0f;
        else ((uint16_t*)(rows + nrow))[si] = f2h(am / 127.0f);
    }
    if (row_major) {
        *(uint16_t*)(rows + ((size_t)h * max_s + pos) * HD + 2 * lane) = (uint16_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8));
    } else if (!is_v) {
        *(uint16_t*)(rows + kt_off(h, max_s, pos, 2 * lane, 1)) = (uint16_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8));
    } else {
        rows[vt_off(h, max_s, pos, 2 * lane, 1)] = (int8_t)q0;
        rows[vt_off(h, max_s, pos, 2 * lane + 1, 1)] = (int8_t)q1;
    }
}

}  // namespace embla
