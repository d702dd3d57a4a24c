// Batched prefill attention over an int8 KV cache: T new tokens at positions p0 .. p0+T-1 attend
// keys 0 .. their own position (causal; optionally only the last `window` positions).
//
// Follows relu2_prefill_nax and attn_full_b (Sources/EmblaMetal/Kernels/attn_nax.metal:61-364,
// prefill.metal:214-282): ReLU² with sink (p = relu(s·scale)², out = Σp·v / (√128 + Σp)) for the
// reference's full layer, softmax (scale 1/√128) for the BASELINE configs; the int8 rows are
// staged once a workgroup as exact 16-bit integers (attn_nax.metal:26-56), each key's scale
// multiplies its score and each value row's scale its weight (attn_nax.metal:231-246, 294).
//
// MI355X design: a workgroup is (32 tokens, kv head) with one wave a query head (GQ waves), so the
// staged K/V tiles serve GQ * 32 query rows. S^T = K·Q^T runs on v_mfma_f32_32x32x16_f16 with the
// query rows as MFMA columns: lane (row r = l % 32, half h = l / 32) then holds one query row's 16
// scores a 32-key block, so the online softmax state (m, l) and the output O^T rows live in that
// lane: the row maximum needs one cross-lane step (xor 32) and rescaling O needs none. O^T += V^T·P^T
// takes P^T straight from the score registers (its k-slots are chosen to match the score items)
// and V^T from LDS, where V is staged as an fp16 copy of its global lane-order tile, which already
// holds 8 keys of one dim contiguous. K and V tiles are double-buffered in LDS: the next 64 keys'
// global loads are in flight while the current ones are multiplied.
#include "common.hpp"
#include "embla_internal.hpp"
#include "kv_row.hpp"

#include <type_traits>

namespace embla {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int PBK = 128;           // keys a staged tile
constexpr int NSUB = PBK / 32;     // 32-key global tiles (and MFMA key blocks) a staged tile
constexpr int KROW = HD + 8;       // LDS row stride of K (fp16 elements): conflict-free 16 B reads
// V is staged as an fp16 copy of its global tile order: a 32-key tile is 8 rows u (dim % 8) of 64
// lane slots (n + 16g) of 16 bytes, each slot the 8 keys {16t + 4g + i} of dim 8n + u. Rows are
// padded by 32 bytes: a 128-bit LDS read is served 16 lanes a pass over 64 banks, and the A-operand
// reads of 16 lanes (rows u = 0..7, slots n and n + 1) then sit at 16-byte offsets distinct mod 16.
constexpr int VUROW = 64 * 8 + 16; // fp16 elements a padded row u
constexpr int VTILE = 8 * VUROW;   // fp16 elements a staged 32-key V tile

__device__ __forceinline__ f16_t mfma32(h8v a, h8v b, f16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
/// 32x32x16 on 16-byte operands holding fp16 (BF = false) or bf16 (BF = true) values.
template <bool BF>
__device__ __forceinline__ f16_t mfma32x(u4_t a, u4_t b, f16_t c) {
    if constexpr (BF) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
}

struct __attribute__((aligned(16))) PrefillSmem {
    _Float16 k[2][PBK * KROW];
    _Float16 vt[2][NSUB * VTILE];
};

// a split's partial record (floats): O / l as 128 fp16, then m and l in fp32, padded to 16 bytes:
// half the bytes of an fp32 O for the split pass to write and the merge to read. O / l is a convex
// combination of V rows (l is the split's own weight sum, the sink is added by the merge), and
// every instance's P·V product already takes V as fp16: int8 V exactly, 16-bit ring V as a copy
// (fp16 rings) or widened to fp16 in staging (bf16 rings, bf8_to_h8: exact for |v| in
// [2^-14, 65504]). So the fp16 record loses no range that the product keeps.
constexpr int PPH = 68;
#ifndef PF_PRIO
// wave priority raised over the score chains (1), the P·V products (2): with two waves a SIMD
// entering each tile together, the raised one issues its chain first and the two drift into
// alternating MFMA and softmax phases (C5 full: 0.561 -> 0.555 ms with 1, 0.580 with 2, 0.570 with 3)
#define PF_PRIO 1
#endif
constexpr int PF_WAVES = 8;        // waves a workgroup: GQ query heads x (8 / GQ) 32-row blocks
#ifndef PF_XCD
#ifndef PF_FOLD
#define PF_FOLD 1
#endif
#define PF_XCD 1                   // workgroups of one (kv head, split) spread over one XCD
#endif
int launch_prefill_tail(const PrefillArgs& a, hipStream_t st);

/// Scales of the four keys kt + 4g .. + 3 (fp16 pair or fp32 quad) as fp32.
template <bool SCALE32>
__device__ __forceinline__ void scales4(const char* base, size_t idx, float* out) {
    if constexpr (SCALE32) {
        const u4_t r = ld16(base + idx * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = __uint_as_float(r[i]);
    } else {
        const u2_t r = ld8(base + idx * 2);
        out[0] = h2f((uint16_t)(r[0] & 0xFFFF));
        out[1] = h2f((uint16_t)(r[0] >> 16));
        out[2] = h2f((uint16_t)(r[1] & 0xFFFF));
        out[3] = h2f((uint16_t)(r[1] >> 16));
    }
}
/// 16 int8 as fp16, each times its scale (pairs of fp16 scales), into two 16-byte halves.
__device__ __forceinline__ h8_t i8x8_scaled(uint32_t a, uint32_t b, h2_t s01, h2_t s23, h2_t s45, h2_t s67) {
    h8_t x = i8x8_to_h8(a, b);
    h2_t* p = (h2_t*)&x;
    p[0] = p[0] * s01;
    p[1] = p[1] * s23;
    p[2] = p[2] * s45;
    p[3] = p[3] * s67;
    return x;
}

// RING: K/V from a 16-bit ring (no scales; S = K·Q^T on the MFMA in the ring's type, BF = bf16;
// V staged as fp16); else from an int8 region (fp16 MFMA), each key's K scale (with 1/√128, and
// log2 e for softmax) and V scale multiplied into its staged fp16 row. PRE: q normed with gains,
// rotated, bf16-rounded in-kernel. LIN (with RING): the "ring" is an int8 region staged to fp16 by
// prestage_kernel (slots = positions, no wrap; K rows already carry their scale and the score
// scale, V rows their scale), which the int8 path would otherwise convert in every workgroup.
template <int GQ, bool RELU2, bool SCALE32, bool QBF, bool OBF, bool RING = false, bool BF = false, bool PRE = false,
          bool LIN = false>
__global__ __launch_bounds__(64 * PF_WAVES, 1) void prefill_int8_kernel(PrefillArgs a) {
    constexpr int NT = 64 * PF_WAVES;
    constexpr int RB = PF_WAVES / GQ;                       // 32-row blocks a workgroup
    __shared__ PrefillSmem sm;
    // full caches: consecutive workgroup ids go to consecutive XCDs, and id % (n_kv * nsplit)
    // picks the (kv head, split), so that each XCD streams as few key ranges as possible and its L2
    // holds them (C5 full: -2%); a ring's windows differ from row block to row block (no gain)
    int tb = blockIdx.x, kvh = blockIdx.y, zz = blockIdx.z;
    if constexpr (PF_XCD && (!RING || LIN)) {
        const int nc = gridDim.y * gridDim.z;
        const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const int combo = lin % nc;
        tb = lin / nc;
        kvh = combo % gridDim.y;
        zz = combo / gridDim.y;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, h = lane >> 5;
    const int hq = kvh * GQ + w % GQ;
    const int wt0 = tb * 32 * RB;                             // the workgroup's first token
    const int tok0 = wt0 + 32 * (w / GQ), tok = tok0 + r;     // this wave's rows, this lane's row
    const bool row_ok = tok < a.T;
    const int pos = a.p0 + min(tok, a.T - 1);                  // its position
    const int last_tok = min(tok0 + 31, a.T - 1);              // the wave's last row
    const int hi = a.p0 + min(wt0 + 32 * RB - 1, a.T - 1);     // last key the workgroup needs
    int lo = 0;
    if (a.window > 0) lo = max(0, a.p0 + wt0 - a.window + 1);
    const int kfirst = lo & ~(PBK - 1);
    const int ntot = (hi - kfirst) / PBK + 1;
    // split z of nsplit takes an equal share of the block's key tiles (the prefix splits evenly)
    const int z = zz, t_lo = ntot * z / a.nsplit, t_hi = ntot * (z + 1) / a.nsplit;
    const int kstart = kfirst + t_lo * PBK;
    const int ntiles = t_hi - t_lo;

    // score scale: folded into the staged K rows for int8, applied to S for a ring
    const float c = RELU2 ? 0.08838834764831845f : 0.08838834764831845f * 1.4426950408889634f;
    const float cr = LIN ? 1.0f : c;   // the scale a ring's scores still need
    const size_t nrow = (size_t)a.n_kv * a.max_s * HD;
    const char* ksb = (const char*)(a.kc + nrow);
    const char* vsb = (const char*)(a.vc + nrow);
    constexpr int ES = SCALE32 ? 4 : 2;

    // ---- staging: each thread moves 16-byte pieces of the two 32-key global tiles of a 64-key tile
    constexpr int EB = RING ? 2 : 1;
    constexpr int PIECES = NSUB * 256 * EB;       // 16-byte pieces a staged tile, K (same for V)
    constexpr int PER = PIECES / NT;              // pieces a thread
    static_assert(PER >= 1, "a piece a thread at least");
    struct Stage {
        u4_t kr[PER], vr[PER];
        float ksr[PER];                           // int8: the K pieces' scales
        uint32_t vsh[PER][4];                     // int8: the V pieces' 8 scales, fp16 pairs
    };
    Stage SA;                                     // the next tile's loads
    auto tile_key = [&](int key) -> int {         // the 32-key tile's first key, clamped in range
        // a 64-key tile's second half may lie past max_s (max_s % 64 == 32): read the first half
        // again; those keys are past every row's position and masked
        return RING ? key : min(key, a.max_s - 32);
    };
    auto gload = [&](int k0, Stage& S) {
        u4_t* kr = S.kr;
        u4_t* vr = S.vr;
        float* ksr = S.ksr;
        uint32_t (*vsh)[4] = S.vsh;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int qw = 64 * w + NT * i, gt = qw / (256 * EB), jl = qw % (256 * EB) + lane;
            if constexpr (RING) {
                const size_t off = tile_base(kvh, a.R, LIN ? k0 + 32 * gt : (k0 + 32 * gt) % a.R, 2) + (size_t)jl * 16;
                kr[i] = ld16((const char*)a.kring + off);
                vr[i] = ld16((const char*)a.vring + off);
                // V piece (row jl / 64, slot l = jl % 64): keys 16 (e / 4) + 4 (l / 16) + e % 4 of
                // the tile; those past the last key the workgroup needs (slots maybe never written)
                // are zeroed so that their weight 0 adds exactly 0
                const int lk = k0 + 32 * gt, l = jl & 63;
                if (lk + 31 > hi) {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int e = 2 * k, key = lk + 16 * (e >> 2) + 4 * (l >> 4) + (e & 3);
                        vr[i][k] &= (key <= hi ? 0xFFFFu : 0u) | (key + 1 <= hi ? 0xFFFF0000u : 0u);
                    }
                }
            } else {
                // the piece's tile and row j are the wave's (uniform: scalar base addresses, the
                // lane's part a 32-bit offset)
                const int j = (qw % 256) >> 6, l = lane;
                const int kt = tile_key(k0 + 32 * gt);
                const size_t tb0 = tile_base(kvh, a.max_s, kt, 1) + (size_t)(qw % 256) * 16;
                kr[i] = ld16(a.kc + tb0 + 16 * l);
                vr[i] = ld16(a.vc + tb0 + 16 * l);
                // K piece: key kt + 16 (j / 2) + l % 16; V piece: keys kt + 16t + 4 (l / 16) + i
                const size_t kbase = (size_t)kvh * a.max_s + kt + 16 * (j >> 1);
                ksr[i] = SCALE32 ? *(const float*)(ksb + kbase * 4 + 4 * (l & 15))
                                 : h2f(*(const uint16_t*)(ksb + kbase * 2 + 2 * (l & 15)));
                const size_t vidx = (size_t)kvh * a.max_s + kt + 4 * (l >> 4);
                if constexpr (SCALE32) {
                    float t[8];
                    scales4<true>(vsb, vidx, t);
                    scales4<true>(vsb, vidx + 16, t + 4);
#pragma unroll
                    for (int k = 0; k < 4; k++) vsh[i][k] = (uint32_t)f2h(t[2 * k]) | ((uint32_t)f2h(t[2 * k + 1]) << 16);
                } else {   // fp16 scales stay fp16 pairs: the staging multiplies in fp16 anyway
                    const u2_t s0 = ld8(vsb + vidx * 2), s1 = ld8(vsb + (vidx + 16) * 2);
                    vsh[i][0] = s0[0];
                    vsh[i][1] = s0[1];
                    vsh[i][2] = s1[0];
                    vsh[i][3] = s1[1];
                }
                // keys past the last one the workgroup needs (the last staged tile; maybe never
                // written) are staged as zero rows: masked keys then add exactly 0 to P·V
                const int lk = k0 + 32 * gt;   // the tile's logical first key (kt may be clamped)
                if (lk + 31 > hi) {
                    if (lk + 16 * (j >> 1) + (l & 15) > hi) ksr[i] = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        if (lk + 16 * (e >> 2) + 4 * (l >> 4) + (e & 3) > hi) vsh[i][e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                }
            }
        }
    };
    auto sstore = [&](int b, const Stage& S) {
        const u4_t* kr = S.kr;
        const u4_t* vr = S.vr;
        const float* ksr = S.ksr;
        const uint32_t (*vsh)[4] = S.vsh;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            // piece q = 64 w + NT i + lane: its tile gt and row j are the wave's
            const int qw = 64 * w + NT * i, gt = qw / (256 * EB), j = (qw % (256 * EB)) >> 6, l = lane;
            if constexpr (RING) {
                // K piece (j, l): key 16 (j / 4) + l % 16, dims 32 (l / 16) + 8 (j % 4) .. + 7
                const int key = 32 * gt + 16 * (j >> 2) + (l & 15), d0 = 32 * (l >> 4) + 8 * (j & 3);
                *(u4_t*)(sm.k[b] + key * KROW + d0) = kr[i];
                // V piece (j = u, l): row u of slot l, 8 keys: a copy (bf16 widened to fp16, so P
                // keeps fp16's 11-bit significand in the P·V product)
                u4_t vv = vr[i];
                if constexpr (BF) vv = __builtin_bit_cast(u4_t, bf8_to_h8(vv));
                *(u4_t*)(sm.vt[b] + gt * VTILE + j * VUROW + l * 8) = vv;
            } else {
                // K piece (j, l): key 16 (j / 2) + l % 16, dims 32 (l / 16) + 16 (j % 2) .. + 15,
                // times its scale · c
                const int key = 32 * gt + 16 * (j >> 1) + (l & 15), d0 = 32 * (l >> 4) + 16 * (j & 1);
                const _Float16 sk = (_Float16)(ksr[i] * c);
                const h2_t s2 = {sk, sk};
                *(h8_t*)(sm.k[b] + key * KROW + d0) = i8x8_scaled(kr[i][0], kr[i][1], s2, s2, s2, s2);
                *(h8_t*)(sm.k[b] + key * KROW + d0 + 8) = i8x8_scaled(kr[i][2], kr[i][3], s2, s2, s2, s2);
                // V piece (j, l): rows u = 2j, 2j + 1 of slot l, 8 keys {16t + 4g + i} each (item
                // 4t + i), times their scales
                const h2_t v01 = __builtin_bit_cast(h2_t, vsh[i][0]), v23 = __builtin_bit_cast(h2_t, vsh[i][1]);
                const h2_t v45 = __builtin_bit_cast(h2_t, vsh[i][2]), v67 = __builtin_bit_cast(h2_t, vsh[i][3]);
                _Float16* base = sm.vt[b] + gt * VTILE + l * 8;
                *(h8_t*)(base + (2 * j) * VUROW) = i8x8_scaled(vr[i][0], vr[i][1], v01, v23, v45, v67);
                *(h8_t*)(base + (2 * j + 1) * VUROW) = i8x8_scaled(vr[i][2], vr[i][3], v01, v23, v45, v67);
            }
        }
    };

    // ---- Q^T as the B operand: lane (row r, half h), k-step s: dims 16s + 8h .. + 7 (16-bit,
    // in the MFMA's type)
    u4_t qb[8];
    {
        const uint16_t* qr = a.q + (size_t)min(tok, a.T - 1) * a.q_tok_stride + (size_t)hq * a.q_head_stride;
#pragma unroll
        for (int s = 0; s < 8; s++) qb[s] = ld16(qr + 16 * s + 8 * h);
        if constexpr (PRE) {
#pragma clang fp contract(off)
            // head_norm with the q gains, RoPE at the row's position, bf16 (attn_sliding8_b,
            // prefill.metal:450-456): the row's dims are split over lanes h = 0, 1 (xor 32); the
            // rotation pairs d and d + 32 (d < 32) sit in the same lane (k-steps s and s + 2)
            float x[64];
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    x[8 * s + 2 * i] = bf2f(qb[s][i] & 0xFFFF);
                    x[8 * s + 2 * i + 1] = bf2f(qb[s][i] >> 16);
                }
            // Σx² in rms_factor's butterfly over dim pairs (2l, 2l + 1): pair l = 8s + 4h + i
            // is this lane's (s, i); level 4 (h) crosses to lane xor 32, the others stay here
            float v[32];
#pragma unroll
            for (int e = 0; e < 32; e++) {
                const float p0 = x[2 * e] * x[2 * e], p1 = x[2 * e + 1] * x[2 * e + 1];
                v[e] = p0 + p1;
            }
#pragma unroll
            for (int m = 16; m >= 4; m >>= 1)   // pair levels 32, 16, 8: s ^ 4, s ^ 2, s ^ 1
#pragma unroll
                for (int e = 0; e < m; e++) v[e] = v[e] + v[e + m];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = sum_xor32(v[e]);
            v[0] = v[0] + v[2];
            v[1] = v[1] + v[3];
            v[0] = v[0] + v[1];
            const float rn = 1.0f / sqrtf(v[0] / 128.0f + EPS32);
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) x[8 * s + e] = x[8 * s + e] * (rn * (1.0f + bf2f(a.qg[16 * s + 8 * h + e])));
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int d = 16 * s + 8 * h + e;   // < 32, partner d + 32 at k-step s + 2
                    float sn, cs;
                    rope_cs(pos, d, cs, sn);
                    const float x1 = x[8 * s + e], x2 = x[8 * (s + 2) + e];
                    x[8 * s + e] = x1 * cs - x2 * sn;
                    x[8 * (s + 2) + e] = x1 * sn + x2 * cs;
                }
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    qb[s][i] = (uint32_t)f2bf(x[8 * s + 2 * i]) | ((uint32_t)f2bf(x[8 * s + 2 * i + 1]) << 16);
        } else if constexpr ((!RING || LIN) && QBF) {
#pragma unroll
            for (int s = 0; s < 8; s++) qb[s] = __builtin_bit_cast(u4_t, bf8_to_h8(qb[s]));
        }
    }

    float m = NEG_INF, lsum = 0.0f;
    // FOLD: the score chains subtract the running maximum themselves, by a ninth k-step of a ones
    // column (A) against -m (B, lane half 0, k 0), so the weights need no v_sub. m is then kept
    // exactly representable in fp16 (any shift of a row's scores leaves its softmax unchanged).
    // Its range is fp16's: scores up to 65504 in log2 units (about 45,400 before the 1/sqrt(d)
    // scale); the layers' q and k are RMS-normed a head, which keeps scores far below that.
    constexpr bool FOLD = PF_FOLD && !RELU2 && !BF && (!RING || LIN);
    const u4_t kone = {h ? 0u : 0x3C00u, 0u, 0u, 0u};   // fp16 1.0 at k 0
    u4_t qm = {0u, 0u, 0u, 0u};                          // -m (0 while the row has no key)
    f16_t O[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) O[i][e] = 0.0f;

    if (ntiles > 0) {
        gload(kstart, SA);
        sstore(0, SA);
    }
    __syncthreads();
    // tile it: products from LDS buffer it % 2 while tile it + 1's loads are in flight; tile it + 1
    // is staged into the other buffer at the end
    auto iteration = [&](int it, Stage& ld_set, const Stage& st_set) {
        const int b = it & 1, k0 = kstart + it * PBK;
        if (it + 1 < ntiles) gload(k0 + PBK, ld_set);
        const bool full_tile = k0 + PBK - 1 <= a.p0 + tok0 && (a.window == 0 || k0 >= a.p0 + last_tok - a.window + 1);
        const bool dead = k0 > a.p0 + last_tok;   // past every row of this wave: nothing to add
        // keys above kmax or at/below kmin are masked; a tile every row sees whole masks nothing
        const int kmax = full_tile ? 0x7FFFFFFF : pos;
        const int kmin = (full_tile || a.window == 0) ? -0x7FFFFFFF : pos - a.window;
        // S^T for keys k0 + 32kb + {8b + 4h + i}: the lane's 16 items e = 4b + i. Both blocks'
        // products are issued before either block's softmax, so one chain runs under the other's
        // VALU work.
        // P^T B operands (fp16) of a block's two 16-key k-steps: step s = items b = s (slots
        // 0..3) and b = 2 + s (slots 4..7)
        auto pack = [&](const float* pw, u4_t* pb) {
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int q2 = 0; q2 < 4; q2++) {
                    const int e0 = (q2 < 2 ? 4 * s : 4 * (2 + s)) + 2 * (q2 & 1);
                    pb[s][q2] = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)pw[e0], (_Float16)pw[e0 + 1]});
                }
        };
        // O^T (dims 32i + {8b + 4h + i}) += V^T P^T over two 16-key k-steps: in step s lane
        // (dim 32i + r, h) takes slot (n = dim / 8, g = 2s + h) of row u = dim % 8, whose 8 keys
        // {8s + 4h + i, 16 + 8s + 4h + i} are the P^T items b = s and b = 2 + s
        auto pv = [&](int kb, const u4_t* pb) {
            const u4_t* vt = (const u4_t*)(sm.vt[b] + kb * VTILE);
            if (PF_PRIO & 2) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int dim = 32 * i + r;
                    O[i] = mfma32x<false>(vt[(dim & 7) * (VUROW / 8) + (dim >> 3) + 16 * (2 * s + h)], pb[s], O[i]);
                }
            if (PF_PRIO & 2) __builtin_amdgcn_s_setprio(0);
        };
        // two 32-key blocks kb0, kb0 + 1 of the staged tile: one max and rescale decision
        auto pair = [&](int kb0) {
            // the two blocks' score chains interleaved (one chain's MFMA under the other's latency)
            f16_t s0, s1;
            if (PF_PRIO & 1) __builtin_amdgcn_s_setprio(1);
            {
                const u4_t* k0r = (const u4_t*)(sm.k[b] + (32 * kb0 + r) * KROW) + h;
                const u4_t* k1r = k0r + 32 * KROW / 8;
                if constexpr (FOLD) {
                    s0 = mfma32x<false>(kone, qm, (f16_t){});
                    s1 = mfma32x<false>(kone, qm, (f16_t){});
                    s0 = mfma32x<BF>(k0r[0], qb[0], s0);
                    s1 = mfma32x<BF>(k1r[0], qb[0], s1);
                } else {
                    s0 = mfma32x<BF>(k0r[0], qb[0], (f16_t){});
                    s1 = mfma32x<BF>(k1r[0], qb[0], (f16_t){});
                }
#pragma unroll
                for (int s = 1; s < 8; s++) {
                    s0 = mfma32x<BF>(k0r[2 * s], qb[s], s0);
                    s1 = mfma32x<BF>(k1r[2 * s], qb[s], s1);
                }
            }
            if (PF_PRIO & 1) __builtin_amdgcn_s_setprio(0);
            // scores of the tile's 64 keys: item e of block kb is x[16 kb + e]
            float x[32];
            // a ring's scores are unscaled (x c): ReLU² scales them here, softmax in the exponent
#pragma unroll
            for (int e = 0; e < 16; e++) {
                x[e] = RING && RELU2 ? s0[e] * cr : s0[e];
                x[16 + e] = RING && RELU2 ? s1[e] * cr : s1[e];
            }
            if (!full_tile) {   // uniform: only the diagonal (and window-edge) tiles
#pragma unroll
                for (int e = 0; e < 32; e++) {
                    const int key = k0 + 32 * (kb0 + (e >> 4)) + 8 * ((e & 15) >> 2) + 4 * h + (e & 3);
                    x[e] = key <= kmax && key > kmin ? x[e] : (RELU2 ? 0.0f : NEG_INF);
                }
            }
            float msub = 0.0f;
            if constexpr (FOLD) {
                // x = score - m already (m = 0 for a row with no key yet)
                float ma = vmax3(x[0], x[1], x[2]), mb = vmax3(x[16], x[17], x[18]);
#pragma unroll
                for (int e = 3; e < 15; e += 2) {
                    ma = vmax3(ma, x[e], x[e + 1]);
                    mb = vmax3(mb, x[16 + e], x[17 + e]);
                }
                const float mt = max_xor32(vmax3(vmax3(ma, mb, x[15]), x[31], x[31]));
                const bool fresh = m == NEG_INF;
                // a row's first keys set m; later, m moves only when a row's scores exceed it by
                // more than 2^8: weights stay <= 256 (fp16-safe), O and l share the stale m
                if (__any(mt > 8.0f || (fresh && mt > NEG_INF))) {
                    const float meff = fresh ? 0.0f : m;
                    const float top = meff + mt;   // the row's largest score of the pair
                    float mn = fresh ? top : fmaxf(m, top);
                    mn = mn == NEG_INF ? NEG_INF : (float)(_Float16)mn;
                    const float corr = fresh ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                    lsum *= corr;
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) O[i][e] *= corr;
                    const float d = mn == NEG_INF ? 0.0f : mn - meff;   // re-base this pair's x
#pragma unroll
                    for (int e = 0; e < 32; e++) x[e] -= d;
                    m = mn;
                    const _Float16 nm = (_Float16)(mn == NEG_INF ? 0.0f : -mn);
                    qm[0] = h ? 0u : (uint32_t)__builtin_bit_cast(uint16_t, nm);
                }
            } else if constexpr (!RELU2) {
                // two max3 chains over the 32 scores, then across the row's two lanes
                float ma = vmax3(x[0], x[1], x[2]), mb = vmax3(x[16], x[17], x[18]);
#pragma unroll
                for (int e = 3; e < 15; e += 2) {
                    ma = vmax3(ma, x[e], x[e + 1]);
                    mb = vmax3(mb, x[16 + e], x[17 + e]);
                }
                const float mt = max_xor32(vmax3(vmax3(ma, mb, x[15]), x[31], x[31])) * (RING ? cr : 1.0f);
                // the running maximum moves only when a row's grows by more than 2^8: weights stay
                // <= 256 (fp16-safe), O and l share the stale m
                if (__any(mt > m + 8.0f)) {
                    const float mn = fmaxf(m, mt);
                    const float corr = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                    lsum *= corr;
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) O[i][e] *= corr;
                    m = mn;
                }
                // a masked key gives exp2(-inf) = 0; a row whose every key so far is masked keeps
                // m = -inf: subtracting +inf instead keeps its weights 0 (not exp2(-inf + inf))
                msub = m == NEG_INF ? -NEG_INF : m;
            }
            auto weight = [&](float v) -> float {
                if constexpr (RELU2) {
                    const float t = fmaxf(v, 0.0f);
                    return t * t;
                } else {
                    if constexpr (FOLD) return __builtin_amdgcn_exp2f(v);
                    else return __builtin_amdgcn_exp2f(RING && !LIN ? __builtin_fmaf(v, c, -msub) : v - msub);
                }
            };
            float pw[16];
            u4_t pb0[2], pb1[2];
#pragma unroll
            for (int e = 0; e < 16; e++) { pw[e] = weight(x[e]); lsum += pw[e]; }
            pack(pw, pb0);
            // block 0's products run while block 1's weights are computed (the compiler's own
            // interleave: a pinned read/MFMA/6-VALU pattern here measured 1-2% slower)
            pv(kb0, pb0);
#pragma unroll
            for (int e = 0; e < 16; e++) { pw[e] = weight(x[16 + e]); lsum += pw[e]; }
            pack(pw, pb1);
            pv(kb0 + 1, pb1);
        };
        if (!dead) {   // uniform a wave
#pragma unroll
            for (int kb0 = 0; kb0 < NSUB; kb0 += 2) pair(kb0);
        }
        if (it + 1 < ntiles) {
            // buffer b ^ 1 was last read in the previous iteration, which every wave finished
            // before that iteration's barrier: one barrier a tile
            sstore(b ^ 1, st_set);
            __syncthreads();
        }
    };
    for (int it = 0; it < ntiles; it++) iteration(it, SA, SA);

    // ---- normalise and store: lane (row r, half h) holds dims 32i + 8b + 4h .. + 3. The
    // workgroup's rows are staged in LDS (the tile buffers are free once every wave is past the
    // loop) and written coalesced: a token's GQ heads are one contiguous run, GQ partial records
    // (PPH floats each) or GQ output rows. Each lane holding one row, 32 rows 4 KB apart a store
    // instruction, cost 4.2 µs a call on the sliding layer's 8.4 MB output.
    lsum = sum_xor32(lsum);
    const float inv = RELU2 ? 1.0f / (11.313708498984761f + lsum) : 1.0f / lsum;
    const int tl = 32 * (w / GQ) + r, hl = w % GQ;   // the lane's token and head in the workgroup
    const int ntok = min(32 * RB, a.T - wt0);
    const bool coalesced = ((uintptr_t)a.o % 16) == 0 && a.o_tok_stride % 8 == 0 && a.o_head_stride % 8 == 0;
    __syncthreads();
    float* stg = (float*)&sm;
    if (a.nsplit > 1) {   // this split's partial records: O / l (fp16), m, l
        constexpr int TS = GQ * PPH + 4;   // floats a token: the 8-byte writes of 16 rows on distinct banks
        float* rec = stg + tl * TS + hl * PPH;
        const float il = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        uint16_t* r16 = (uint16_t*)rec;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                u2_t pk;
                pk[0] = (uint32_t)f2h(O[i][4 * bb] * il) | ((uint32_t)f2h(O[i][4 * bb + 1] * il) << 16);
                pk[1] = (uint32_t)f2h(O[i][4 * bb + 2] * il) | ((uint32_t)f2h(O[i][4 * bb + 3] * il) << 16);
                *(u2_t*)(r16 + 32 * i + 8 * bb + 4 * h) = pk;
            }
        if (h == 0) *(f4_t*)(rec + HD / 2) = (f4_t){m, lsum, 0.0f, 0.0f};
        __syncthreads();
        constexpr int CPT = GQ * PPH / 4;   // 16-byte chunks a token
        float* pz = a.part + ((size_t)z * a.T + wt0) * a.n_q * PPH + (size_t)kvh * GQ * PPH;
        for (int cidx = tid; cidx < ntok * CPT; cidx += NT) {
            const int t = cidx / CPT, off = 4 * (cidx % CPT);
            *(f4_t*)(pz + (size_t)t * a.n_q * PPH + off) = *(const f4_t*)(stg + t * TS + off);
        }
        return;
    }
    if (!coalesced) {   // (uniform) strides that a 16-byte store cannot take: one row a lane
        if (!row_ok) return;
        uint16_t* orow = a.o + (size_t)tok * a.o_tok_stride + (size_t)hq * a.o_head_stride;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const int d = 32 * i + 8 * bb + 4 * h;
                u2_t pk;
                pk[0] = (uint32_t)f2a<OBF>(O[i][4 * bb] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 1] * inv) << 16);
                pk[1] = (uint32_t)f2a<OBF>(O[i][4 * bb + 2] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 3] * inv) << 16);
                *(u2_t*)(orow + d) = pk;
            }
        return;
    }
    constexpr int TS16 = GQ * HD + 8;   // 16-bit elements a token (+16 bytes: distinct banks)
    uint16_t* st16 = (uint16_t*)stg;
    uint16_t* rec16 = st16 + tl * TS16 + hl * HD;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            u2_t pk;
            pk[0] = (uint32_t)f2a<OBF>(O[i][4 * bb] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 1] * inv) << 16);
            pk[1] = (uint32_t)f2a<OBF>(O[i][4 * bb + 2] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 3] * inv) << 16);
            *(u2_t*)(rec16 + 32 * i + 8 * bb + 4 * h) = pk;
        }
    __syncthreads();
    constexpr int CPR = HD / 8;   // 16-byte chunks a (token, head) row
    for (int cidx = tid; cidx < ntok * GQ * CPR; cidx += NT) {
        const int t = cidx / (GQ * CPR), hh = (cidx / CPR) % GQ, off = 8 * (cidx % CPR);
        uint16_t* dst = a.o + (size_t)(wt0 + t) * a.o_tok_stride + (size_t)(kvh * GQ + hh) * a.o_head_stride + off;
        *(u4_t*)dst = *(const u4_t*)(st16 + t * TS16 + hh * HD + off);
    }
}

/// Merges the nsplit partial records of (token, head): 32 lanes a row, 4 dims a lane (8-byte loads),
/// 8 rows a workgroup: rows (blockIdx.x * 8 + tid / 32) of head blockIdx.y.
template <bool RELU2, bool OBF>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
    // 16 lanes a (token, head): 8 dims a lane, one 16-byte load of a split's O / l record
    const int lane = threadIdx.x & 15, tok = blockIdx.x * 16 + (threadIdx.x >> 4), hq = blockIdx.y;
    if (tok >= a.T) return;
    float M = RELU2 ? 0.0f : NEG_INF, mz[4], lz[4];
    u4_t v[4];
#pragma unroll
    for (int z = 0; z < 4; z++) {
        if (z < a.nsplit) {
            const float* pp = a.part + (((size_t)z * a.T + tok) * a.n_q + hq) * PPH;
            v[z] = ld16((const uint16_t*)pp + 8 * lane);   // O / l, fp16
            const u2_t ml = ld8(pp + HD / 2);
            mz[z] = __uint_as_float(ml[0]);
            lz[z] = __uint_as_float(ml[1]);
            if constexpr (!RELU2) M = fmaxf(M, mz[z]);
        }
    }
    float L = 0.0f, acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int z = 0; z < 4; z++) {
        if (z < a.nsplit) {
            // split z's share: its l, rescaled to the common maximum
            const float f = lz[z] * (RELU2 ? 1.0f : (mz[z] == NEG_INF ? 0.0f : exp2f(mz[z] - M)));
            L += f;
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] += h2f((uint16_t)(v[z][i / 2] >> (16 * (i & 1)))) * f;
        }
    }
    const float inv = RELU2 ? 1.0f / (11.313708498984761f + L) : 1.0f / L;
    uint16_t* orow = a.o + (size_t)tok * a.o_tok_stride + (size_t)hq * a.o_head_stride;
    u4_t pk;
#pragma unroll
    for (int i = 0; i < 4; i++)
        pk[i] = (uint32_t)f2a<OBF>(acc[2 * i] * inv) | ((uint32_t)f2a<OBF>(acc[2 * i + 1] * inv) << 16);
    if (((uintptr_t)orow & 15) == 0) {
        *(u4_t*)(orow + 8 * lane) = pk;
    } else {   // a token or head stride that breaks 16-byte alignment (4-byte aligned always)
        *(u2_t*)(orow + 8 * lane) = (u2_t){pk[0], pk[1]};
        *(u2_t*)(orow + 8 * lane + 4) = (u2_t){pk[2], pk[3]};
    }
}

int launch_prefill_int8(const PrefillArgs& a, hipStream_t st) {
    const int gq = a.n_q / a.n_kv;
    const dim3 grid((a.T + 32 * (PF_WAVES / gq) - 1) / (32 * (PF_WAVES / gq)), a.n_kv, a.nsplit);
#define EMBLA_PF(GQ, R, S32, QBF, OBF) \
    hipLaunchKernelGGL((prefill_int8_kernel<GQ, R, S32, QBF, OBF>), grid, dim3(64 * PF_WAVES), 0, st, a)
    if (gq == 4 && !a.relu2 && !a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(4, false, false, true, true);
    else if (gq == 4 && !a.relu2 && !a.scale32 && !a.q_bf16 && !a.out_bf16) EMBLA_PF(4, false, false, false, false);
    else if (gq == 8 && a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, true, true, true, true);
    else if (gq == 8 && !a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, false, true, true, true);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_PF
    return launch_prefill_tail(a, st);
}

int launch_prefill_ring(const PrefillArgs& a, hipStream_t st) {
    const int gq = a.n_q / a.n_kv;
    const dim3 grid((a.T + 32 * (PF_WAVES / gq) - 1) / (32 * (PF_WAVES / gq)), a.n_kv, a.nsplit);
#define EMBLA_PR(BF, PRE) \
    hipLaunchKernelGGL((prefill_int8_kernel<4, false, false, BF, BF, true, BF, PRE>), grid, dim3(64 * PF_WAVES), 0, st, a)
    if (gq == 8 && a.relu2 && a.q_bf16 && a.out_bf16 && !a.qg && a.window == 0) {
        // the reference's full layer over a bf16 cache (attn_full_b, prefill.metal:214-282)
        hipLaunchKernelGGL((prefill_int8_kernel<8, true, false, true, true, true, true, false>), grid, dim3(64 * PF_WAVES),
                           0, st, a);
        return launch_prefill_tail(a, st);
    }
    if (gq != 4 || a.relu2) return EMBLA_ERR_UNSUPPORTED;
    if (a.q_bf16 && a.out_bf16 && a.qg) EMBLA_PR(true, true);
    else if (a.q_bf16 && a.out_bf16) EMBLA_PR(true, false);
    else if (!a.q_bf16 && !a.out_bf16 && !a.qg) EMBLA_PR(false, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_PR
    return launch_prefill_tail(a, st);
}

/// Stages an int8 layer region's keys [0, n) (fp16 scales) as the 16-bit lane-order tiles the LIN
/// instance reads (R slots a kv head, R a multiple of 128 >= n): a thread a 16-byte int8 piece,
/// written as two 16-byte fp16 pieces with exactly the products prefill_int8_kernel's own staging
/// forms (K rows times fp16(scale · c), V rows times their fp16 scales, both in fp16). Keys
/// n .. R - 1 are staged as zeros (their cache bytes and scales may never have been written).
__global__ __launch_bounds__(256) void prestage_kernel(const int8_t* __restrict__ kc, const int8_t* __restrict__ vc,
                                                       uint16_t* __restrict__ k16, uint16_t* __restrict__ v16, int n,
                                                       int R, int max_s, float c) {
    const int tile = blockIdx.x, kvh = blockIdx.y, is_v = blockIdx.z;
    const int t0 = 32 * tile, j = threadIdx.x >> 6, l = threadIdx.x & 63;   // int8 piece (j, l)
    const int8_t* src = (is_v ? vc : kc);
    const uint16_t* sb = (const uint16_t*)(src + (size_t)max_s * HD * gridDim.y) + (size_t)kvh * max_s + t0;
    const bool live = t0 < n;   // uniform
    const u4_t r = live ? ld16(src + tile_base(kvh, max_s, t0, 1) + (size_t)(64 * j + l) * 16) : (u4_t){0, 0, 0, 0};
    auto sc = [&](int k) -> float { return t0 + k < n ? h2f(sb[k]) : 0.0f; };   // 0 past the keys staged
    uint16_t* dst = (is_v ? v16 : k16) + tile_base(kvh, R, t0, 2) / 2;
    h8_t a, b;
    if (!is_v) {   // K piece: key 16 (j / 2) + l % 16, dims 32 (l / 16) + 16 (j % 2) .. + 15
        const _Float16 sk = (_Float16)(sc(16 * (j >> 1) + (l & 15)) * c);
        const h2_t s2 = {sk, sk};
        a = i8x8_scaled(r[0], r[1], s2, s2, s2, s2);
        b = i8x8_scaled(r[2], r[3], s2, s2, s2, s2);
        // 16-bit tile: K load j16 = 4t + p / 16 with p = 2 (d % 32): pieces 2j and 2j + 1
        *(h8_t*)(dst + (size_t)(64 * (2 * j) + l) * 8) = a;
        *(h8_t*)(dst + (size_t)(64 * (2 * j + 1) + l) * 8) = b;
    } else {       // V piece: rows u = 2j, 2j + 1 of slot l, keys {16t + 4 (l / 16) + i}
        const int g = l >> 4;
        _Float16 v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            v[e] = (_Float16)sc(16 * (e >> 2) + 4 * g + (e & 3));   // an fp16 scale, exact
        }
        const h2_t v01 = {v[0], v[1]}, v23 = {v[2], v[3]}, v45 = {v[4], v[5]}, v67 = {v[6], v[7]};
        a = i8x8_scaled(r[0], r[1], v01, v23, v45, v67);
        b = i8x8_scaled(r[2], r[3], v01, v23, v45, v67);
        // 16-bit tile: V load j16 = u
        *(h8_t*)(dst + (size_t)(64 * (2 * j) + l) * 8) = a;
        *(h8_t*)(dst + (size_t)(64 * (2 * j + 1) + l) * 8) = b;
    }
}

/// Prefill over an int8 region through a staged fp16 copy (workspace k16, v16: n_kv * R * 128
/// elements each): the staging pass, then the LIN instance.
int launch_prefill_prestaged(const PrefillArgs& a0, uint16_t* k16, uint16_t* v16, int R, hipStream_t st) {
    const int gq = a0.n_q / a0.n_kv;
    const int n = a0.p0 + a0.T;
    if (!(gq == 4 && !a0.relu2 && !a0.scale32 && a0.q_bf16 && a0.out_bf16) || R % 128 || R < n) return EMBLA_ERR_UNSUPPORTED;
    const float c = 0.08838834764831845f * 1.4426950408889634f;
    hipLaunchKernelGGL(prestage_kernel, dim3(R / 32, a0.n_kv, 2), dim3(256), 0, st, a0.kc, a0.vc, k16, v16, n, R,
                       a0.max_s, c);
    PrefillArgs a = a0;
    a.kring = k16; a.vring = v16; a.R = R;
    const dim3 grid((a.T + 32 * (PF_WAVES / gq) - 1) / (32 * (PF_WAVES / gq)), a.n_kv, a.nsplit);
    hipLaunchKernelGGL((prefill_int8_kernel<4, false, false, true, true, true, false, false, true>), grid,
                       dim3(64 * PF_WAVES), 0, st, a);
    return launch_prefill_tail(a, st);
}

int launch_prefill_tail(const PrefillArgs& a, hipStream_t st) {
    if (a.nsplit > 1) {
        const dim3 mg((a.T + 15) / 16, a.n_q);
        if (a.relu2) hipLaunchKernelGGL((prefill_merge_kernel<true, true>), mg, dim3(256), 0, st, a);
        else if (a.out_bf16) hipLaunchKernelGGL((prefill_merge_kernel<false, true>), mg, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((prefill_merge_kernel<false, false>), mg, dim3(256), 0, st, a);
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
