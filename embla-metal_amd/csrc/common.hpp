// Shared device helpers for the gfx950 attention kernels: element types, exact int8 -> fp16
// conversion, MFMA wrappers, wave reductions and the cache layouts every kernel agrees on.
//
// Cache layouts (one layer; head dim 128; the caller owns the memory). Both K and V are stored in
// 32-key tiles "in MFMA lane order": tile (kv head h, keys 32i .. 32i+31) is 32*128*ES bytes at
// ((h * max_s/32) + i) * 4096 * ES, and inside a tile the bytes are ordered so that load j of
// lane l (16 bytes at (j*64 + l)*16) is exactly what lane l needs as its MFMA operand slice. Every
// load instruction of a wave then reads 1 KB contiguous (a row-major or column-group layout makes
// each 16-byte lane load hit its own cache line and caps a CU at ~20 GB/s).
//   K tile: key k = 16t + m (t = 0, 1), dim d: lane l = m + 16*(d/32) holds dims 32*(d/32) .. +31
//           of key k; byte p = (d % 32) * ES of its slice is load j = t*2ES + p/16, byte p % 16.
//   V tile: key k = 16t + 4g + i, dim d = 8n + u: lane l = n + 16g, byte p = (8u + 4t + i) * ES
//           of its 8*8*ES-byte slice is load j = p/16, byte p % 16.
//   int8 regions: K (or V) tiles [n_kv][max_s/32], then scales [n_kv][max_s] (fp16 or fp32) at
//   byte n_kv * max_s * 128, as the reference's KV8 layout places them (common.metal:53-63), so an
//   engine's per-layer offsets and region sizes are unchanged.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace embla {

constexpr int HD = 128;          // head dim
constexpr float NEG_INF = -__builtin_huge_valf();

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ scalar conversions
__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
/// fp32 -> bf16 bits, round to nearest even (BFloat16.swift:4-9; NaN is not expected here).
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

/// A 16-bit activation (fp16 or bf16 bits) as float.
template <bool BF> __device__ __forceinline__ float a2f(uint16_t b) { return BF ? bf2f(b) : h2f(b); }
template <bool BF> __device__ __forceinline__ uint16_t f2a(float f) { return BF ? f2bf(f) : f2h(f); }

// ------------------------------------------------------------------ int8 -> fp16, exact
// Bytes are biased to unsigned (x ^ 0x80), placed under a 0x64 exponent byte (the fp16 value
// 1024 + u), and 1152 is subtracted: every int8 is exact in fp16, so the result is exact.
__device__ __forceinline__ void i8x4_to_h4(uint32_t x, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = x ^ 0x80808080u;
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, lo) - bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, hi) - bias);
}
/// 8 int8 (two dwords) -> 8 fp16 lanes of an MFMA operand.
__device__ __forceinline__ h8_t i8x8_to_h8(uint32_t a, uint32_t b) {
    uint32_t r0, r1, r2, r3;
    i8x4_to_h4(a, r0, r1);
    i8x4_to_h4(b, r2, r3);
    return __builtin_bit_cast(h8_t, (u4_t){r0, r1, r2, r3});
}
/// 8 bf16 (four dwords) -> 8 fp16; exact for the magnitudes attention inputs take (|x| in
/// [2^-14, 65504]); smaller values lose low bits as fp16 subnormals.
__device__ __forceinline__ h8_t bf8_to_h8(u4_t w) {
    h8_t r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[2 * i] = (_Float16)__uint_as_float(w[i] << 16);
        r[2 * i + 1] = (_Float16)__uint_as_float(w[i] & 0xFFFF0000u);
    }
    return r;
}

// ------------------------------------------------------------------ MFMA (gfx950)
// 16x16x32 f16: A lane = row + 16*(k/8), B lane = col + 16*(k/8), 8 halves a lane; D lane =
// col + 16*(row/4), 4 floats a lane (item = row % 4). Only the pairing of A and B k-slots matters
// for the kernels below: a lane's 8 A halves and the same lane group's 8 B halves are one k-range.
__device__ __forceinline__ f4_t mfma16(h8_t a, h8_t b, f4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4_t mfma16bf(b8_t a, b8_t b, f4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

/// 16x16x32 on 16-byte operands holding fp16 (BF = false) or bf16 (BF = true) values.
template <bool BF>
__device__ __forceinline__ f4_t mfma16x(u4_t a, u4_t b, f4_t c) {
    if constexpr (BF) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------ loads
__device__ __forceinline__ u4_t ld16(const void* p) { return *reinterpret_cast<const u4_t*>(p); }
__device__ __forceinline__ u2_t ld8(const void* p) { return *reinterpret_cast<const u2_t*>(p); }
/// Streaming loads for data read once (KV caches): no reuse, keep them out of the way.
__device__ __forceinline__ u4_t ld16_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p));
}

// ------------------------------------------------------------------ wave helpers (wave64)
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
/// Maxima on v_maximum3_f32 (IEEE 754-2019 maximum: NaN-propagating, so the compiler quiets no
/// input first; fmaxf's maxNum made it canonicalise each MFMA result, one more VALU a value). The
/// compiler sees these operations, so it also keeps the wait states a VALU read of an MFMA result
/// needs (inline asm here went without them).
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float vmax2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
/// max(v, v of lane xor 32) in every lane, on v_permlane32_swap (VALU, no LDS round trip).
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return vmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
/// v and v of lane xor 16 (r[0], r[1] in some order a lane), on v_permlane16_swap: with both
/// operands v, rows 0 and 2 keep their own values in one output and take rows 1 and 3 in the
/// other, and the other way round for rows 1 and 3. A commutative op of the pair gives the
/// shfl_xor result bit for bit, with no LDS round trip.
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
/// v of lane xor 16 (exactly shfl_xor(v, 16)): from the swap's pair, the half that is not the
/// lane's own (rows 0 and 2 find their partner's in r[1], rows 1 and 3 in r[0]).
__device__ __forceinline__ float xchg_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
/// The same over lane xor 32 (v_permlane32_swap); fmaxf, as the shfl_xor reductions it replaces.
__device__ __forceinline__ float fmax_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
/// max / sum over the four 16-lane rows (xor 16, then xor 32)
__device__ __forceinline__ float max_rows(float v) { return fmax_xor32(max_xor16(v)); }
__device__ __forceinline__ float sum_rows(float v) { return sum_xor32(sum_xor16(v)); }
/// DPP moves (VALU, no LDS round trip); CTRL: quad_perm 0xB1 (lane xor 1), 0x4E (xor 2),
/// row_half_mirror 0x141 (lane 7 - i of its 8), row_mirror 0x140, row_shr:n 0x110 + n, row_ror:n
/// 0x120 + n, row_bcast:15 0x142, row_bcast:31 0x143. Lanes with no source (bound_ctrl) and rows
/// off in ROW_MASK read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
/// Inclusive prefix sums within each 16-lane row (every lane of the wave active).
__device__ __forceinline__ uint32_t row_scan_incl(uint32_t v) {
    v += dpp_u32<0x111>(v);
    v += dpp_u32<0x112>(v);
    v += dpp_u32<0x114>(v);
    v += dpp_u32<0x118>(v);
    return v;
}
/// Inclusive prefix sum over the wave's 64 lanes (every lane active): the rows' scans, then row
/// 0's total into row 1 and row 2's into row 3 (row_bcast:15), then lane 31's into rows 2 and 3
/// (row_bcast:31). Exact for integers, as the shfl_up ladder it replaces.
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    v = row_scan_incl(v);
    v += dpp_u32<0x142, 0xA>(v);
    v += dpp_u32<0x143, 0xC>(v);
    return v;
}
/// op over the wave's 64 lanes, in every lane, bit for bit as the xor butterfly 32, 16, 8, 4, 2, 1
/// (v = op(v, v of lane xor m)) gives it, for a commutative op: the permlane swaps hand each lane
/// the pair for xor 32 and 16; row_ror:8 is xor 8 within a 16-lane row; row_ror:4 reads lane
/// i + 4 mod 16, which is i ^ 4 or i ^ 4 ^ 8, and lanes i and i ^ 8 agree after the xor-8 level;
/// then quad_perm for xor 2 and xor 1. No LDS round trips.
template <class Op>
__device__ __forceinline__ float wave_bfly(float v, Op op) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    v = op(v, dpp_f32<0x128>(v));
    v = op(v, dpp_f32<0x124>(v));
    v = op(v, dpp_f32<0x4E>(v));
    v = op(v, dpp_f32<0xB1>(v));
    return v;
}
/// A lane's O^T block of a 16x16 MFMA output (O[u][i]: dim 8n + u, head 4g + i) into LDS rows
/// om[head][128], for the heads below GQ (a multiple of 4): one branch, two 16-byte stores a head
/// (a store a value under its own condition compiled to a branch each).
template <int GQ>
__device__ __forceinline__ void store_o_rows(float (*om)[128], const f4_t* O, int n, int g) {
    if (4 * g < GQ) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *(f4_t*)&om[4 * g + i][8 * n] = (f4_t){O[0][i], O[1][i], O[2][i], O[3][i]};
            *(f4_t*)&om[4 * g + i][8 * n + 4] = (f4_t){O[4][i], O[5][i], O[6][i], O[7][i]};
        }
    }
}
/// LDS stores of a wave's lanes visible to the wave's other lanes (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
/// A 32-key tile's per-key scores from lane n = 0 of each row (lane group g): items e = 4t + i are
/// keys 16t + 4g + i, i.e. at dst[16t + i] (dst: the tile's first key plus 4g). A full tile is two
/// 16-byte stores; a partial one stores its valid keys one by one.
__device__ __forceinline__ void store_scores(float* dst, const float* smx, const bool* valid, bool full, int n) {
    if (n != 0) return;
    if (full) {
        *(f4_t*)dst = (f4_t){smx[0], smx[1], smx[2], smx[3]};
        *(f4_t*)(dst + 16) = (f4_t){smx[4], smx[5], smx[6], smx[7]};
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (valid[e]) dst[16 * (e >> 2) + (e & 3)] = smx[e];
    }
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ float readlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

/// Byte offset of element (key j, dim d) of kv head h in a K tile region of element size ES.
__host__ __device__ __forceinline__ size_t kt_off(int h, int max_s, int j, int d, int es) {
    const int k = j & 31, t = k >> 4, m = k & 15, l = m + 16 * (d >> 5), p = (d & 31) * es;
    const int jj = t * 2 * es + (p >> 4);
    return (((size_t)h * (max_s >> 5) + (j >> 5)) * 4096 * es) + (size_t)(jj * 64 + l) * 16 + (p & 15);
}
/// Byte offset of element (key j, dim d) of kv head h in a V tile region of element size ES.
__host__ __device__ __forceinline__ size_t vt_off(int h, int max_s, int j, int d, int es) {
    const int k = j & 31, t = k >> 4, g = (k >> 2) & 3, i = k & 3, n = d >> 3, u = d & 7;
    const int l = n + 16 * g, p = (8 * u + 4 * t + i) * es;
    return (((size_t)h * (max_s >> 5) + (j >> 5)) * 4096 * es) + (size_t)((p >> 4) * 64 + l) * 16 + (p & 15);
}
/// Start of the 32-key tile holding key j.
__host__ __device__ __forceinline__ size_t tile_base(int h, int max_s, int j, int es) {
    return ((size_t)h * (max_s >> 5) + (j >> 5)) * 4096 * es;
}

}  // namespace embla
