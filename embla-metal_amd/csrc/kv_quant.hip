// int8 quantise-and-append of K/V rows, and the reference's query preparation (RMS head norm
// with gains), one wave64 a (token, kv head, K or V) / a (token, head).
//
// Quantisation follows write_row8 (Sources/EmblaMetal/Kernels/common.metal:72-84) with kv_append /
// kv_append_b as callers (attention.metal:113-140, prefill.metal:182-212):
//   v_i = x_i (bf16-rounded when the input is bf16: the reference's bf()),
//   a = max |v_i|, q_i = rint(v_i * (127 / a)) (0 when a = 0), scale = a / 127
// stored as fp32 (reference) or fp16 (config). With norm_k the K row is first RMS-normed without
// gains (head_norm with ng = 0, common.metal:13-26): r = 1 / sqrt(Σx² / 128 + 2^-23).
// Bit-exactness: the squares are summed in a fixed butterfly (lane pairs xor 32, 16, .., 1 over
// per-lane sums of two squares) that the oracle restates; no fma contraction anywhere here.
#include "common.hpp"
#include "embla_internal.hpp"
#include "kv_row.hpp"

#pragma clang fp contract(off)

namespace embla {

/// One wave a (token, kv head, K or V): two dims a lane, quantised, then stored at their places
/// in the MFMA lane-order tiles (common.hpp; K's two bytes are adjacent, V's are not), or in plain
/// 128-byte rows for a cache that is read by gathering (row_major).
__global__ __launch_bounds__(64) void kv_quant_kernel(KVQuantArgs a) {
    const int lane = threadIdx.x;
    const int t = blockIdx.x, h = blockIdx.y;
    const bool is_v = blockIdx.z == 1;
    const int pos = a.p0 + t;
    const uint16_t* src = is_v ? a.v : a.k;
    int8_t* rows = is_v ? a.vc : a.kc;

    const uint32_t raw = *(const uint32_t*)(src + (size_t)t * a.stride + h * HD + 2 * lane);
    const float x0 = a.in_bf16 ? bf2f(raw & 0xFFFF) : h2f(raw & 0xFFFF);
    const float x1 = a.in_bf16 ? bf2f(raw >> 16) : h2f(raw >> 16);
    int q0, q1;
    const float am = quant_pair(x0, x1, !is_v && a.norm_k, a.in_bf16, q0, q1);
    store_pair8(rows, a.n_kv, a.max_s, h, pos, is_v, a.row_major, a.scale32, q0, q1, am, lane);
}

int launch_kv_quant(const KVQuantArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(kv_quant_kernel, dim3(a.T, a.n_kv, 2), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

/// Query rows normed with the gains (head_norm, common.metal:13-26), bf16-rounded as the
/// reference does before its attention (attention.metal:168-169; prefill.metal:406-426).
__global__ __launch_bounds__(64) void q_prep_kernel(QPrepArgs a) {
    const int lane = threadIdx.x, h = blockIdx.x, t = blockIdx.y;
    const uint32_t raw = *(const uint32_t*)(a.qraw + (size_t)t * a.stride + h * HD + 2 * lane);
    float x0 = bf2f(raw & 0xFFFF), x1 = bf2f(raw >> 16);
    const float r = rms_factor(x0, x1);
    float g0 = r, g1 = r;
    if (a.ng >= 1) {
        g0 = g0 * (1.0f + bf2f(a.g1[2 * lane]));
        g1 = g1 * (1.0f + bf2f(a.g1[2 * lane + 1]));
    }
    if (a.ng >= 2) {
        g0 = g0 * (1.0f + bf2f(a.g2[2 * lane]));
        g1 = g1 * (1.0f + bf2f(a.g2[2 * lane + 1]));
    }
    x0 = bf2f(f2bf(x0 * g0));
    x1 = bf2f(f2bf(x1 * g1));
    uint16_t* out = a.out + (a.head_major ? (size_t)h * a.T + t : (size_t)t * a.n_q + h) * HD + 2 * lane;
    out[0] = a.out_bf16 ? f2bf(x0) : f2h(x0);
    out[1] = a.out_bf16 ? f2bf(x1) : f2h(x1);
}

/// T positions p0 .. of 16-bit K and V rows into a ring (slot p % R, tile layout with ES = 2). With
/// gains (the reference's sliding layers, kv_sliding_b, prefill.metal:103-125) K is RMS-normed with
/// them, rotated (RoPE at its position) and rounded to bf16; with norm_k (a bf16 full-layer cache,
/// R = max_s: kv_append / kv_append_b without KV8, attention.metal:113-140, prefill.metal:182-212)
/// only RMS-normed and rounded; V is copied. One wave a (token, head).
__global__ __launch_bounds__(64) void ring_append_kernel(RingAppendArgs a) {
    const int lane = threadIdx.x, t = blockIdx.x, h = blockIdx.y;
    const int pos = a.p0 + t, slot = pos % a.R;
    const uint32_t kraw = *(const uint32_t*)(a.k + (size_t)t * a.stride + h * HD + 2 * lane);
    const uint32_t vraw = *(const uint32_t*)(a.v + (size_t)t * a.stride + h * HD + 2 * lane);
    uint32_t kout = kraw;
    if (a.kg) {   // bf16 rows with pre-ops
        float x0 = bf2f(kraw & 0xFFFF), x1 = bf2f(kraw >> 16);
        const float r = rms_factor(x0, x1);
        x0 = x0 * (r * (1.0f + bf2f(a.kg[2 * lane])));
        x1 = x1 * (r * (1.0f + bf2f(a.kg[2 * lane + 1])));
        // RoPE: dims d and d + 32 (d < 32) rotate together; lane l holds 2l, 2l + 1
        const float o0 = xchg_xor16(x0), o1 = xchg_xor16(x1);
        if (lane < 32) {
            const int d0 = (2 * lane) & 31;
            float s0, c0, s1, c1;
            rope_cs(pos, d0, c0, s0);
            rope_cs(pos, d0 + 1, c1, s1);
            if (lane < 16) { x0 = x0 * c0 - o0 * s0; x1 = x1 * c1 - o1 * s1; }
            else { x0 = o0 * s0 + x0 * c0; x1 = o1 * s1 + x1 * c1; }
        }
        kout = (uint32_t)f2bf(x0) | ((uint32_t)f2bf(x1) << 16);
    } else if (a.norm_k) {   // bf16 rows of a full layer: RMS norm without gains (kv_append, no KV8)
        float x0 = bf2f(kraw & 0xFFFF), x1 = bf2f(kraw >> 16);
        const float r = rms_factor(x0, x1);
        kout = (uint32_t)f2bf(x0 * r) | ((uint32_t)f2bf(x1 * r) << 16);
    }
    *(uint32_t*)(a.kring + kt_off(h, a.R, slot, 2 * lane, 2) / 2) = kout;
    a.vring[vt_off(h, a.R, slot, 2 * lane, 2) / 2] = (uint16_t)(vraw & 0xFFFF);
    a.vring[vt_off(h, a.R, slot, 2 * lane + 1, 2) / 2] = (uint16_t)(vraw >> 16);
}

int launch_ring_append(const RingAppendArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(ring_append_kernel, dim3(a.T, a.n_kv), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

int launch_q_prep(const QPrepArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(q_prep_kernel, dim3(a.n_q, a.T), dim3(64), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
