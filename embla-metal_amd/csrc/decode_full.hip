// Split-K decode attention over an int8 KV cache (one query token), on gfx950 MFMA.
//
// Follows the reference's attn_full8 / attn_sparse8 (Sources/EmblaMetal/Kernels/attention.metal:
// 235-363, 448-584): a workgroup takes one (chunk of keys, kv head) and writes a partial; the
// partials are then merged (the reference's arrive_last step, common.metal:86-99, 209-220).
// Weights: softmax (config C1/C3 and the reference's sparse layers) or ReLU² with sink
// (`relu(q·k/√128)²`, `o = Σw·v / (√128 + Σw)`, attention.metal:143-145, 209-220).
//
// The MI355X design (not the reference's): a wave64 takes 32-key tiles. S^T = K·q^T runs on
// v_mfma_i32_16x16x64_i8 straight on the cache's int8 K bytes: q is held as a 15-bit fixed point
// per head (|error| <= absmax/64000) split exactly into two int8 halves, q = s·(256·hi + lo), each
// half its own B operand (column n = head n), so both partial sums land in the lane that combines
// them (two more MFMAs a tile instead of a cross-lane exchange a score: 10.50 against 10.69 us a
// launch at 32k). A lane (head n, lane group g) of the score tile then holds keys {16t + 4g + i},
// which is exactly the A-operand slice it needs for O += W·V (v_mfma_f32_16x16x32_f16, V bytes
// converted exactly to fp16), so the weights never move between lanes. K and V tiles are stored in MFMA lane order (common.hpp), so
// each of a wave's 8 loads a tile reads 1 KB contiguous. Scores and weights stay in fp32;
// W = p·scale_v is rounded to fp16 (with a power-of-two prescale) only as the MFMA operand.
// Chunk partials are merged by a second, wide kernel (a workgroup a (query head, 32 dims), one
// memory round) instead of the reference's last-arriving threadgroup: on MI355X a cross-XCD
// arrival protocol costs a chain of round trips through the coherence point (store completion,
// counter RMW, then the loads) of ~5 us, against ~2 us for a dependent launch; the split also
// needs no counters, so the path is graph-capturable and leaves no state behind.
#include "common.hpp"
#include "embla_internal.hpp"
#include "kv_row.hpp"

#include <type_traits>

namespace embla {

typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr float WSCALE = 64.0f;   // prescale of W into fp16's normal range; divided out at the end
constexpr float LOG2E = 1.4426950408889634f;
constexpr float QFIX = 32000.0f;  // q's fixed-point range: |q_int| <= 32000, so |hi| <= 125
// A (chunk, query head) partial record, PH floats: O / (l · WSCALE) as 128 fp16 (a convex
// combination of the dequantised V rows: fp16 holds it to |v| <= 65504, the range the P·V operand
// gives V anyway), then m and l in fp32, padded to 16 bytes. Half the bytes of an fp32 O, for the
// merge to read (it multiplies each record by its l and the softmax correction).
constexpr int PH = HD / 2 + 4;

/// One 32-key tile's raw bytes for a lane.
struct Tile8 {
    u4_t k[4];    // K: [2t + h] = half t, dims 32g + 16h .. + 15 of key 16t + n
    u4_t v[4];    // V: [u / 2], dwords (u % 2) * 2 .. = dim 8n + u for keys {16t + 4g + i}
    u4_t ks[2];   // scales of keys 16t + 4g .. + 3: fp16 in .xy of [t]; fp32 in [t]
    u4_t vs[2];
};

/// The 8 scales of a lane's keys, item e = 4t + i <-> key 16t + 4g + i.
template <bool SCALE32>
__device__ __forceinline__ void scales8(const u4_t* r, float* out) {
#pragma unroll
    for (int t = 0; t < 2; t++) {
        if constexpr (SCALE32) {
#pragma unroll
            for (int i = 0; i < 4; i++) out[4 * t + i] = __uint_as_float(r[t][i]);
        } else {
            out[4 * t + 0] = h2f((uint16_t)(r[t][0] & 0xFFFF));
            out[4 * t + 1] = h2f((uint16_t)(r[t][0] >> 16));
            out[4 * t + 2] = h2f((uint16_t)(r[t][1] & 0xFFFF));
            out[4 * t + 3] = h2f((uint16_t)(r[t][1] >> 16));
        }
    }
}

// K and V tile rows are read once: nontemporal loads (9.86 -> 9.40 us a split-K launch at 32k,
// 14.17 -> 13.55 us a layer, two A/B pairs on one box)
#define TLD(p) ld16_stream(p)

constexpr int DW = 8;            // waves a workgroup: one 32-key tile each a round

/// The decode step's own append (workgroup C of each kv head): waves 0 and 1 quantise the new
/// token's k and v rows exactly as kv_quant_kernel does and store them at position pos; then wave
/// h < GQ adds the new key as one more partial of query head kvh GQ + h: its score in the log2
/// domain as the maximum, weight 1, and vs v WSCALE as the sums, the chunk partials' conventions.
template <int GQ, bool SCALE32, bool QR>
__device__ __forceinline__ void decode_append(const DecodeAppend& app, const uint16_t* __restrict__ q,
                                              float* __restrict__ part, int C, int max_s, int n_kv, int kvh,
                                              float sc, const uint16_t* __restrict__ g1,
                                              const uint16_t* __restrict__ g2, int ng) {
    __shared__ int8_t nk[HD], nv[HD];
    __shared__ float nsc[2];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (w < 2) {
        const bool is_v = w == 1;
        const uint32_t raw = *(const uint32_t*)((is_v ? app.v : app.k) + (size_t)kvh * HD + 2 * lane);
        int q0, q1;
        const float am = quant_pair(bf2f(raw & 0xFFFF), bf2f(raw >> 16), !is_v && app.norm_k, true, q0, q1);
        store_pair8(is_v ? app.vc : app.kc, n_kv, max_s, kvh, app.pos, is_v, false, SCALE32, q0, q1, am, lane);
        int8_t* dst = is_v ? nv : nk;
        dst[2 * lane] = (int8_t)q0;
        dst[2 * lane + 1] = (int8_t)q1;
        if (lane == 0) nsc[w] = SCALE32 ? am / 127.0f : h2f(f2h(am / 127.0f));   // the stored scale
    }
    __syncthreads();
    if (w >= GQ) return;
    const int hq = kvh * GQ + w;
    const uint32_t qr = *(const uint32_t*)(q + (size_t)hq * HD + 2 * lane);
    float x0, x1;
    if constexpr (QR) {   // the head norm the chunk workgroups apply
        x0 = bf2f(qr & 0xFFFF);
        x1 = bf2f(qr >> 16);
        const float rf = rms_factor(x0, x1);
        float g0 = rf, gg1 = rf;
        if (ng >= 1) { g0 = g0 * (1.0f + bf2f(g1[2 * lane])); gg1 = gg1 * (1.0f + bf2f(g1[2 * lane + 1])); }
        if (ng >= 2) { g0 = g0 * (1.0f + bf2f(g2[2 * lane])); gg1 = gg1 * (1.0f + bf2f(g2[2 * lane + 1])); }
        x0 = bf2f(f2bf(x0 * g0));
        x1 = bf2f(f2bf(x1 * gg1));
    } else {
        x0 = h2f((uint16_t)(qr & 0xFFFF));
        x1 = h2f((uint16_t)(qr >> 16));
    }
    const float dot = wave_sum_bfly(x0 * (float)nk[2 * lane] + x1 * (float)nk[2 * lane + 1]);
    float* pp = part + ((size_t)C * n_kv * GQ + hq) * PH;   // weight 1: O / l is the dequantised row
    *(uint32_t*)((uint16_t*)pp + 2 * lane) =
        (uint32_t)f2h(nsc[1] * (float)nv[2 * lane]) | ((uint32_t)f2h(nsc[1] * (float)nv[2 * lane + 1]) << 16);
    if (lane == 0) { pp[HD / 2] = dot * nsc[0] * sc; pp[HD / 2 + 1] = 1.0f; }
}

template <int GQ, bool RELU2, bool SCALE32, bool OBF, bool SCORES, bool QR, bool APP>
__global__ __launch_bounds__(64 * DW, 2) void full_decode_kernel(
    const uint16_t* __restrict__ q,   // [n_kv * GQ][128]: fp16 prepared, or (QR) raw bf16
    const int8_t* __restrict__ kc, const int8_t* __restrict__ vc,
    float* __restrict__ part, float* __restrict__ scores, uint16_t* __restrict__ o, int S, int CH,
    int C, int max_s, int n_kv, float qk_scale, float sink, const uint16_t* __restrict__ g1,
    const uint16_t* __restrict__ g2, int ng, DecodeAppend app) {
    static_assert(GQ == 4 || GQ == 8, "4 or 8 query heads a kv head");
    static_assert(!APP || (!RELU2 && !SCORES), "the step's own append: softmax layers");
    // APP: a 1-D grid, the C * n_kv chunk workgroups first (chunk fastest) and the n_kv append
    // workgroups last, so that the chunks take one CU each and the short appends the spare slots
    int c = blockIdx.x, kvh = blockIdx.y;
    if constexpr (APP) {
        const int id = blockIdx.x;
        if (id >= C * n_kv) {   // uniform a workgroup
            decode_append<GQ, SCALE32, QR>(app, q, part, C, max_s, n_kv, id - C * n_kv, qk_scale * LOG2E, g1, g2, ng);
            return;
        }
        c = id % C;
        kvh = id / C;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;

    const size_t rows = (size_t)n_kv * max_s * HD;
    const char* ksb = (const char*)(kc + rows);
    const char* vsb = (const char*)(vc + rows);
    constexpr int ES = SCALE32 ? 4 : 2;
    const int j0 = c * CH, j1 = min(S, j0 + CH);
    const float sc = RELU2 ? qk_scale : qk_scale * LOG2E;

    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};

    i4_t qb[2], ql[2];
    float qsc = 0.0f;   // the fixed point's step, per head
    // SCORES (the reference's full layer, whose scores feed select_keys): q stays a 16-bit float
    // and S^T runs on v_mfma_f32_16x16x32_f16 with K widened exactly to fp16, so every product is
    // exact and the sums are fp32 (the fixed point's 2^-16 relative error would move near-ties in
    // or out of the top 1024). MFMA j: lane (n, g) dims 32g + 8j .. + 7, column n = head n.
    h8_t qh[SCORES ? 4 : 1];
    // q as a 15-bit fixed point split into int8 halves, hi in qb and lo in ql: column n < GQ holds
    // head n (other columns 0); lane (n, g), MFMA b: dims 32g + 16b .. + 15 (the K slice's dims).
    // Separate operands put both halves' products in the lane that uses them (no cross-lane step).
    // q's rows are requested before the first tile (loads complete in order: requested after the
    // tile, q's wait would also wait for the tile, and the set-up would start only once the tile
    // had arrived from HBM). The set-up splits the kv head's GQ rows over the wave: lane L takes
    // head L / LPH, dims d0 .. d0 + VPL - 1 (a quarter of what a lane of the operand layout holds,
    // where 16 lanes of a row repeat 4 heads), and hands the operands over through the wave's own
    // slot of the merge LDS (free until its tiles are done).
    constexpr int VPL = 2 * GQ, LPH = 64 / GQ, NQ = VPL / 8;
    const int qhd = lane / LPH, d0 = VPL * (lane % LPH);
    __shared__ __attribute__((aligned(16))) float om[DW][GQ][HD];
    char* const qa = (char*)&om[w][0][0];
    u4_t qraw[NQ], ga[QR ? NQ : 1], gb[QR ? NQ : 1];   // (QR: the head norm's gains)
    auto load_q = [&]() {
        const uint16_t* qr = q + ((size_t)kvh * GQ + qhd) * HD + d0;
#pragma unroll
        for (int u = 0; u < NQ; u++) qraw[u] = ld16(qr + 8 * u);
        if constexpr (QR) {   // no branch (a load under one made its join wait for every load)
            const uint16_t* p1 = ng >= 1 ? g1 + d0 : qr;   // (a gain not given reads q's row, unused)
            const uint16_t* p2 = ng >= 2 ? g2 + d0 : qr;
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                ga[u] = ld16(p1 + 8 * u);
                gb[u] = ld16(p2 + 8 * u);
            }
        }
    };
    // op over the LPH lanes of a head, as the butterfly over the head's dim pairs gives it: the
    // pair p = GQ k + j of lane k, slot j; levels xor 32 .. GQ cross lanes (k), xor GQ / 2 .. 1 stay
    // in the lane. The first cross-lane level exchanges exactly (GQ = 4: row_ror:8 is k ^ 8 in a
    // 16-lane row; GQ = 8: k ^ 4 from row_shl:4 or row_shr:4), after which the lanes a rotation or
    // quad_perm mixes agree, so every level pairs what the butterfly pairs.
    auto head_lanes = [&](float v, auto op) -> float {
        if constexpr (GQ == 4) {
            v = op(v, dpp_f32<0x128>(v));   // k ^ 8
            v = op(v, dpp_f32<0x124>(v));   // k ^ 4
        } else {
            const float up = dpp_f32<0x104>(v), dn = dpp_f32<0x114>(v);   // lane + 4, lane - 4
            v = op(v, (lane & 4) ? dn : up);                               // k ^ 4
        }
        v = op(v, dpp_f32<0x4E>(v));   // k ^ 2
        v = op(v, dpp_f32<0xB1>(v));   // k ^ 1
        return v;
    };
    auto setup_q = [&]() {
        float x[VPL];
#pragma unroll
        for (int u = 0; u < NQ; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t r = qraw[u][i];
                x[8 * u + 2 * i] = QR ? bf2f((uint16_t)(r & 0xFFFF)) : h2f((uint16_t)(r & 0xFFFF));
                x[8 * u + 2 * i + 1] = QR ? bf2f((uint16_t)(r >> 16)) : h2f((uint16_t)(r >> 16));
            }
        if constexpr (QR) {
            // the head norm of common.metal:13-26 (q_prep's): x * rms * (1 + g1) * (1 + g2),
            // rounded to bf16, Σx² in rms_factor's butterfly over the dim pairs (2p, 2p + 1)
#pragma clang fp contract(off)
            float sp[GQ];
#pragma unroll
            for (int j = 0; j < GQ; j++) {
                const float a = x[2 * j] * x[2 * j], b = x[2 * j + 1] * x[2 * j + 1];
                sp[j] = head_lanes(a + b, [](float u, float v) { return u + v; });
            }
#pragma unroll
            for (int m = GQ / 2; m >= 1; m >>= 1)
#pragma unroll
                for (int j = 0; j < m; j++) sp[j] = sp[j] + sp[j + m];
            const float rf = 1.0f / sqrtf(sp[0] / 128.0f + EPS32);
#pragma unroll
            for (int d = 0; d < VPL; d++) {
                const uint32_t wa = ga[d / 8][(d % 8) / 2], wb = gb[d / 8][(d % 8) / 2];
                float gf = rf;
                if (ng >= 1) gf = gf * (1.0f + bf2f((uint16_t)(d & 1 ? wa >> 16 : wa & 0xFFFF)));
                if (ng >= 2) gf = gf * (1.0f + bf2f((uint16_t)(d & 1 ? wb >> 16 : wb & 0xFFFF)));
                x[d] = bf2f(f2bf(x[d] * gf));
            }
        }
        const bool live = n < GQ;
        if constexpr (SCORES) {   // bf16 / fp16 q as fp16 (bf16 exact down to 2^-17), [head][dim]
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                h8_t hv;
#pragma unroll
                for (int e = 0; e < 8; e++) hv[e] = (_Float16)x[8 * u + e];
                *(h8_t*)(qa + (qhd * HD + d0 + 8 * u) * 2) = hv;
            }
            wave_lds_sync();
#pragma unroll
            for (int j = 0; j < 4; j++)
                qh[j] = live ? *(const h8_t*)(qa + (n * HD + 32 * g + 8 * j) * 2) : (h8_t){};
            return;
        }
        float am = 0.0f;
#pragma unroll
        for (int d = 0; d < VPL; d++) am = fmaxf(am, fabsf(x[d]));
        am = head_lanes(am, [](float u, float v) { return fmaxf(u, v); });
        const float inv = am > 0.0f ? QFIX / am : 0.0f;
        // hi bytes [head][dim] at qa, lo bytes after them, then each head's step
        uint32_t wh[VPL / 4], wl[VPL / 4];
#pragma unroll
        for (int k = 0; k < VPL / 4; k++) {
            wh[k] = 0;
            wl[k] = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int qi = (int)rintf(x[4 * k + e] * inv);
                const int hi = (qi + 128) >> 8, lo = qi - hi * 256;
                wh[k] |= (uint32_t)(hi & 0xFF) << (8 * e);
                wl[k] |= (uint32_t)(lo & 0xFF) << (8 * e);
            }
        }
#pragma unroll
        for (int k = 0; k < VPL / 4; k += 2) {
            *(u2_t*)(qa + qhd * HD + d0 + 4 * k) = (u2_t){wh[k], wh[k + 1]};
            *(u2_t*)(qa + GQ * HD + qhd * HD + d0 + 4 * k) = (u2_t){wl[k], wl[k + 1]};
        }
        float* const qs = (float*)(qa + 2 * GQ * HD);
        if (lane % LPH == 0) qs[qhd] = am / QFIX;
        wave_lds_sync();
#pragma unroll
        for (int b = 0; b < 2; b++) {
            qb[b] = live ? *(const i4_t*)(qa + n * HD + 32 * g + 16 * b) : (i4_t){0, 0, 0, 0};
            ql[b] = live ? *(const i4_t*)(qa + GQ * HD + n * HD + 32 * g + 16 * b) : (i4_t){0, 0, 0, 0};
        }
        qsc = qs[n % GQ];
        wave_lds_sync();   // (the slot is the merge's again only after every lane's reads)
    };

    auto load_k_scales = [&](int t0, Tile8& T) {
        const int8_t* pk = kc + tile_base(kvh, max_s, t0, 1) + lane * 16;
#pragma unroll
        for (int j = 0; j < 4; j++) T.k[j] = TLD(pk + 1024 * j);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const size_t si = ((size_t)kvh * max_s + t0 + 16 * t + 4 * g) * ES;
            if constexpr (SCALE32) { T.ks[t] = ld16(ksb + si); T.vs[t] = ld16(vsb + si); }
            else {
                const u2_t a2 = ld8(ksb + si), b2 = ld8(vsb + si);
                T.ks[t] = (u4_t){a2[0], a2[1], 0, 0};
                T.vs[t] = (u4_t){b2[0], b2[1], 0, 0};
            }
        }
    };
    auto compute_tile = [&](int t0, Tile8& T, int nxt) {
        const bool full = t0 + 32 <= j1;
        float ks[8], vs[8];
        scales8<SCALE32>(T.ks, ks);
        scales8<SCALE32>(T.vs, vs);
        // S^T (int32) of the two 16-key halves: lane (n, g) item i of half t = key t0 + 16t + 4g + i
        float x[8];
#pragma unroll
        for (int t = 0; t < 2 && SCORES; t++) {
            f4_t sf = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const u4_t r = T.k[2 * t + j / 2];
                const h8_t a = (j & 1) ? i8x8_to_h8(r[2], r[3]) : i8x8_to_h8(r[0], r[1]);
                sf = mfma16(a, qh[j], sf);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) x[4 * t + i] = sf[i] * ks[4 * t + i];
        }
#pragma unroll
        for (int t = 0; t < 2 && !SCORES; t++) {
            i4_t st = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
            st = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, T.k[2 * t]), qb[0], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, T.k[2 * t + 1]), qb[1], st, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, T.k[2 * t]), ql[0], sl, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, T.k[2 * t + 1]), ql[1], sl, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) x[4 * t + i] = (float)(st[i] * 256 + sl[i]) * qsc * ks[4 * t + i];
        }
        if (nxt >= 0) {   // K is consumed: the next tile's K rows and scales go out now
            const int8_t* pk = kc + tile_base(kvh, max_s, nxt, 1) + lane * 16;
#pragma unroll
            for (int j = 0; j < 4; j++) T.k[j] = TLD(pk + 1024 * j);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const size_t si = ((size_t)kvh * max_s + nxt + 16 * t + 4 * g) * ES;
                if constexpr (SCALE32) T.ks[t] = ld16(ksb + si);
                else { const u2_t a2 = ld8(ksb + si); T.ks[t] = (u4_t){a2[0], a2[1], 0, 0}; }
            }
        }
        bool valid[8];
#pragma unroll
        for (int e = 0; e < 8; e++) valid[e] = full || t0 + 16 * (e >> 2) + 4 * g + (e & 3) < j1;
        if constexpr (SCORES) {
            // max over the kv head's query heads of the dequantised q·k (attention.metal:295-305)
            // (lane n = 0 of each row takes it: lane xor 1, xor 2 by quad_perm, then lane + 4 by
            // row_shl, no LDS round trip; heads n >= GQ hold -inf)
            float smx[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = n < GQ ? x[e] : NEG_INF;
                v = fmaxf(v, dpp_f32<0xB1>(v));
                v = fmaxf(v, dpp_f32<0x4E>(v));
                smx[e] = fmaxf(v, dpp_f32<0x104>(v));
            }
            store_scores(scores + (size_t)kvh * max_s + t0 + 4 * g, smx, valid, full, n);
        }
        h8_t wa;
        if constexpr (RELU2) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float a = fmaxf(x[e] * sc, 0.0f);
                const float wt = valid[e] ? a * a : 0.0f;
                l += wt;
                wa[e] = (_Float16)(wt * vs[e] * WSCALE);
            }
        } else {
            float mt = NEG_INF;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                x[e] = valid[e] ? x[e] * sc : NEG_INF;
                mt = fmaxf(mt, x[e]);
            }
            mt = max_rows(mt);
            const float mn = fmaxf(m, mt);
            // rescale only when some head's maximum grew (rare once the maxima settle); nothing to
            // rescale while m is still -inf
            if (__any(n < GQ && mn > m)) {
                if (__any(n < GQ && m != NEG_INF)) {
                    const float corr = m == NEG_INF ? 0.0f : exp2f(m - mn);
                    l *= corr;
                    float cf[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float c0 = readlane(corr, i);
                        if constexpr (GQ == 8) {
                            const float c1 = readlane(corr, 4 + i);
                            cf[i] = g == 1 ? c1 : c0;
                        } else {
                            cf[i] = c0;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 8; u++)
#pragma unroll
                        for (int i = 0; i < 4; i++) O[u][i] *= cf[i];
                }
                m = mn;
            }
            const float mr = m == NEG_INF ? 0.0f : m;   // no valid key yet (a wave with no tile): every p 0
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float p = __builtin_amdgcn_exp2f(x[e] - mr);   // x = -inf -> 0
                l += p;
                wa[e] = (_Float16)(p * vs[e] * WSCALE);
            }
        }
        if (!full) {   // uniform: a masked key's weight is 0 whatever its scale holds (past S: maybe never written)
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (!valid[e]) wa[e] = (_Float16)0.0f;
        }
        // O += W V: MFMA u covers dims 8n + u (column n), rows = heads 4g + i
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const u4_t r = T.v[u >> 1];
            const h8_t b = (u & 1) ? i8x8_to_h8(r[2], r[3]) : i8x8_to_h8(r[0], r[1]);
            O[u] = mfma16(wa, b, O[u]);
        }
        if (nxt >= 0) {   // V and its scales are consumed: the next tile's go out now
            const int8_t* pv = vc + tile_base(kvh, max_s, nxt, 1) + lane * 16;
#pragma unroll
            for (int j = 0; j < 4; j++) T.v[j] = TLD(pv + 1024 * j);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const size_t si = ((size_t)kvh * max_s + nxt + 16 * t + 4 * g) * ES;
                if constexpr (SCALE32) T.vs[t] = ld16(vsb + si);
                else { const u2_t b2 = ld8(vsb + si); T.vs[t] = (u4_t){b2[0], b2[1], 0, 0}; }
            }
        }
    };

    // one tile a wave a round, its registers reloaded with the next tile's as soon as each part
    // is consumed. The host's chunk gives a wave two tiles at 32k (256 workgroups, one a CU).
    {
        constexpr int step = 32 * DW;
        const int t0 = j0 + 32 * w;
        Tile8 A;
        // the first tile: K and the scales, then V only after the q math. A thinner first burst
        // of requests measured faster than issuing the whole tile at once (10.49 against 11.15 µs
        // a launch at 32k)
        // The first tile's loads take no branch (a wave without a tile reads the chunk's first,
        // unused): under a branch, the compiler's wait for q at the join also waited for the tile
        // (loads complete in order), and the q set-up ran only after the tile had arrived.
        const int tf = t0 < j1 ? t0 : j0;
        load_q();
        __builtin_amdgcn_sched_barrier(0);   // q's requests first
        load_k_scales(tf, A);
        __builtin_amdgcn_sched_barrier(0);   // the scheduler keeps the tile's requests ahead of the set-up
        // q's registers pass through an empty statement here, so no part of the set-up is hoisted
        // above the tile's requests (its wait for q would then come first)
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            asm volatile("" : "+v"(qraw[u]));
            if constexpr (QR) asm volatile("" : "+v"(ga[u]), "+v"(gb[u]));
        }
        setup_q();
        {
            const int8_t* pv = vc + tile_base(kvh, max_s, tf, 1) + lane * 16;
#pragma unroll
            for (int j = 0; j < 4; j++) A.v[j] = TLD(pv + 1024 * j);
        }
        // each tile's K (and K scales) for the next tile go out as soon as the score MFMAs have
        // consumed them, its V (and V scales) after the P·V MFMAs: 10.41 -> 9.92 µs a launch at 32k.
        // The first tile runs outside the loop, whether or not the wave has one (t0 >= j1: every
        // key masked): inside the loop's guard, the compiler sank the first tile's loads below the
        // q set-up.
        compute_tile(t0, A, t0 + step < j1 ? t0 + step : -1);
        for (int t = t0 + step; t < j1; t += step) compute_tile(t, A, t + step < j1 ? t + step : -1);
    }

    // ---- merge the waves (LDS)
    __shared__ float mm[DW][GQ], ll[DW][GQ];
    l = sum_rows(l);
    if (g == 0 && n < GQ) { mm[w][n] = m; ll[w][n] = l; }
    store_o_rows<GQ>(om[w], O, n, g);
    __syncthreads();

    constexpr int PER = GQ * HD / (64 * DW);   // outputs a thread: 1 or 2 (one head, consecutive dims)
    const int oh = tid * PER / HD, od = tid * PER % HD;
    float acc[PER], M, L;
    if constexpr (RELU2) {
        M = 0.0f;
        L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < DW; ww++) L += ll[ww][oh];
#pragma unroll
        for (int e = 0; e < PER; e++) {
            float a = 0.0f;
#pragma unroll
            for (int ww = 0; ww < DW; ww++) a += om[ww][oh][od + e];
            acc[e] = a;
        }
    } else {
        M = NEG_INF;
#pragma unroll
        for (int ww = 0; ww < DW; ww++) M = fmaxf(M, mm[ww][oh]);
        float f[DW];
        L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < DW; ww++) {
            f[ww] = mm[ww][oh] == NEG_INF ? 0.0f : exp2f(mm[ww][oh] - M);
            L += ll[ww][oh] * f[ww];
        }
#pragma unroll
        for (int e = 0; e < PER; e++) {
            float a = 0.0f;
#pragma unroll
            for (int ww = 0; ww < DW; ww++) a += om[ww][oh][od + e] * f[ww];
            acc[e] = a;
        }
    }
    const int hq = kvh * GQ + oh;
    if (!APP && C == 1) {
        const float rr = RELU2 ? 1.0f / (WSCALE * (sink + L)) : 1.0f / (WSCALE * L);
#pragma unroll
        for (int e = 0; e < PER; e++) o[(size_t)hq * HD + od + e] = f2a<OBF>(acc[e] * rr);
        return;
    }
    float* pp = part + ((size_t)c * n_kv * GQ + hq) * PH;
    const float il = L > 0.0f ? 1.0f / (WSCALE * L) : 0.0f;   // ReLU²: every weight of a chunk may be 0
    uint16_t* p16 = (uint16_t*)pp + od;
    if constexpr (PER == 2) *(uint32_t*)p16 = (uint32_t)f2h(acc[0] * il) | ((uint32_t)f2h(acc[1] * il) << 16);
    else p16[0] = f2h(acc[0] * il);
    if (od == 0) { pp[HD / 2] = M; pp[HD / 2 + 1] = L; }
}

/// Merges the C chunk partials of query head blockIdx.x, dims 32 * blockIdx.y .. + 31: thread
/// (slice s of 4 dims, chunk group r) loads its chunks' slices, maxima and sums in one round.
#ifndef MERGE_DPW
#define MERGE_DPW 8   // C3 layer: 13.52 us with the LDS-loop merge, 12.98 (32 dims), 12.30 (16), 12.22-12.27 (8), 12.58 (4)
#endif
constexpr int MDPW = MERGE_DPW;   // dims a merge workgroup

/// op over the lanes of the wave with the same lane % G (G = 1, 2, 4 or 8), in every lane: DPP
/// within 16-lane rows (quad xor 1, xor 2, then row rotations by 4 and 8, which reach every lane
/// of the row with the same lane % 4 once the quads agree), then the rows by permlane swaps. No
/// LDS round trips (a shfl_xor chain waits on LDS at each of its 6 - log2 G steps).
template <int G, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    auto dpp = [](float x, auto ctrl) {
        const int xi = __builtin_bit_cast(int, x);
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, decltype(ctrl)::value, 0xF, 0xF, false));
    };
    if constexpr (G < 2) v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1, 0, 3, 2]
    if constexpr (G < 4) v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2, 3, 0, 1]
    if constexpr (G < 8) v = op(v, dpp(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
    v = op(v, dpp(v, std::integral_constant<int, 0x128>{}));                        // row_ror:8
    return MAX ? max_rows(v) : sum_rows(v);
}

/// Records: fp32 (H16 false: acc[128], m, l, pad: the sparse, ring and 16-bit cache decodes) or
/// the int8 decode's PH-float records (O / l as fp16, then m, l).
template <bool RELU2, bool OBF, bool H16>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part, uint16_t* __restrict__ o,
                                                           int C, int n_q, float sink, float oscale) {
    constexpr int RS = H16 ? PH : HD + 4;   // floats a record
    // thread (slice sl of 4 dims, chunk group r); the chunk groups of a wave reduce by shuffles, the
    // 4 waves through LDS
    constexpr int SLC = MDPW / 4, NR = 256 / SLC, MAXK = 256 / NR;   // C <= 256
    const int h = blockIdx.x, d0 = MDPW * blockIdx.y;
    const int tid = threadIdx.x, sl = tid % SLC, r = tid / SLC, w = tid >> 6;
    const int d = d0 + 4 * sl;
    u4_t v[MAXK];
    float mk[MAXK], lk[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; k++) {
        const int cc = r + NR * k;
        if (cc < C) {
            const float* p = part + ((size_t)cc * n_q + h) * RS;
            if constexpr (H16) {
                const u2_t x = ld8((const uint16_t*)p + d);
                v[k] = (u4_t){x[0], x[1], 0, 0};
            } else {
                v[k] = ld16(p + d);
            }
            const u2_t ml = ld8(p + (H16 ? HD / 2 : HD));
            mk[k] = __uint_as_float(ml[0]);
            lk[k] = __uint_as_float(ml[1]);
        }
    }
    __shared__ float sm[4], sl_[4][SLC];
    __shared__ f4_t sa[4][SLC];
    float M = RELU2 ? 0.0f : NEG_INF;
    if constexpr (!RELU2) {
#pragma unroll
        for (int k = 0; k < MAXK; k++)
            if (r + NR * k < C) M = fmaxf(M, mk[k]);
        M = group_reduce<SLC, true>(M);
        if ((tid & 63) == 0) sm[w] = M;
        __syncthreads();
        M = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    }
    f4_t A = {0, 0, 0, 0};
    float Lr = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXK; k++) {
        if (r + NR * k < C) {
            const float f = RELU2 ? 1.0f : (mk[k] == NEG_INF ? 0.0f : exp2f(mk[k] - M));
            Lr += lk[k] * f;
            if constexpr (H16) {   // O / l: the record's share is its l times the correction
                const float fl = f * lk[k];
#pragma unroll
                for (int i = 0; i < 4; i++) A[i] += h2f((uint16_t)(v[k][i / 2] >> (16 * (i & 1)))) * fl;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) A[i] += __uint_as_float(v[k][i]) * f;
            }
        }
    }
    Lr = group_reduce<SLC, false>(Lr);
#pragma unroll
    for (int i = 0; i < 4; i++) A[i] = group_reduce<SLC, false>(A[i]);
    if ((tid & 63) < SLC) { sa[w][sl] = A; sl_[w][sl] = Lr; }
    __syncthreads();
    if (tid >= SLC) return;
    const f4_t T = sa[0][sl] + sa[1][sl] + sa[2][sl] + sa[3][sl];
    const float L = sl_[0][sl] + sl_[1][sl] + sl_[2][sl] + sl_[3][sl];
    const float inv = 1.0f / (RELU2 ? oscale * (sink + L) : oscale * L);
#pragma unroll
    for (int i = 0; i < 4; i++) o[(size_t)h * HD + d + i] = f2a<OBF>(T[i] * inv);
}

// ------------------------------------------------------------------ host launch
int launch_full_decode(const FullDecodeArgs& a, hipStream_t st) {
    const dim3 grid(a.C, a.n_kv), block(64 * DW);
    const DecodeAppend app{a.knew, a.vnew, a.kcw, a.vcw, a.pos, a.norm_k};
    const float qs = 0.08838834764831845f;   // 1/sqrt(128)
    const float sink = 11.313708498984761f;   // sqrt(128)
#define EMBLA_FD(GQ, R, S32, OBF, SC)                                                              \
    hipLaunchKernelGGL((full_decode_kernel<GQ, R, S32, OBF, SC, false, false>), grid, block, 0, st, a.q, a.kc, a.vc, \
                       a.part, a.scores, a.o, a.S, a.CH, a.C, a.max_s, a.n_kv, qs, sink, nullptr, nullptr, 0, app)
#define EMBLA_FDR(GQ, R, S32, OBF, SC)                                                             \
    hipLaunchKernelGGL((full_decode_kernel<GQ, R, S32, OBF, SC, true, false>), grid, block, 0, st, a.q, a.kc, a.vc, \
                       a.part, a.scores, a.o, a.S, a.CH, a.C, a.max_s, a.n_kv, qs, sink, a.g1, a.g2, a.ng, app)
    const int gq = a.n_q / a.n_kv;
    if (a.append) {   // the decode step with its own append: raw queries, softmax, fp16 scales, bf16 out
        if (!(gq == 4 && a.ng >= 0 && !a.relu2 && !a.scale32 && a.out_bf16 && !a.scores)) return EMBLA_ERR_UNSUPPORTED;
        hipLaunchKernelGGL((full_decode_kernel<4, false, false, true, false, true, true>), dim3((a.C + 1) * a.n_kv),
                           block, 0, st, a.q, a.kc,
                           a.vc, a.part, a.scores, a.o, a.S, a.CH, a.C, a.max_s, a.n_kv, qs, sink, a.g1, a.g2, a.ng, app);
        return launch_decode_merge(a.part, a.o, a.C + 1, a.n_q, false, true, 1.0f, st, true);
    }
    if (a.ng >= 0) {   // raw queries: the reference's full and sparse layers, and the decode step
        if (gq == 8 && a.relu2 && a.scale32 && a.out_bf16 && !a.scores) EMBLA_FDR(8, true, true, true, false);
        else if (gq == 8 && a.relu2 && a.scale32 && a.out_bf16 && a.scores) EMBLA_FDR(8, true, true, true, true);
        else if (gq == 8 && !a.relu2 && a.scale32 && a.out_bf16 && !a.scores) EMBLA_FDR(8, false, true, true, false);
        else if (gq == 4 && !a.relu2 && !a.scale32 && a.out_bf16 && !a.scores) EMBLA_FDR(4, false, false, true, false);
        else return EMBLA_ERR_UNSUPPORTED;
    } else if (gq == 4 && !a.relu2 && !a.scale32 && !a.out_bf16 && !a.scores) EMBLA_FD(4, false, false, false, false);
    else if (gq == 4 && !a.relu2 && a.scale32 && a.out_bf16 && !a.scores) EMBLA_FD(4, false, true, true, false);
    else if (gq == 4 && !a.relu2 && !a.scale32 && a.out_bf16 && !a.scores) EMBLA_FD(4, false, false, true, false);
    else if (gq == 8 && a.relu2 && a.scale32 && a.out_bf16 && !a.scores) EMBLA_FD(8, true, true, true, false);
    else if (gq == 8 && a.relu2 && a.scale32 && a.out_bf16 && a.scores) EMBLA_FD(8, true, true, true, true);
    else if (gq == 8 && !a.relu2 && a.scale32 && a.out_bf16 && !a.scores) EMBLA_FD(8, false, true, true, false);
    else if (gq == 8 && !a.relu2 && !a.scale32 && !a.out_bf16 && !a.scores) EMBLA_FD(8, false, false, false, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_FD
#undef EMBLA_FDR
    if (a.C > 1 && a.merge) return launch_decode_merge(a.part, a.o, a.C, a.n_q, a.relu2, a.out_bf16, 1.0f, st, true);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

int launch_full_decode_merge(const FullDecodeArgs& a, hipStream_t st) {
    return launch_decode_merge(a.part, a.o, a.C, a.n_q, a.relu2, a.out_bf16, 1.0f, st, true);
}

int launch_decode_merge(const float* part, uint16_t* o, int C, int n_q, bool relu2, bool out_bf16, float oscale,
                        hipStream_t st, bool h16) {
    const dim3 mg(n_q, HD / MDPW), block(256);
    const float sink = 11.313708498984761f;   // sqrt(128)
#define EMBLA_MG(R, B)                                                                                               \
    do {                                                                                                             \
        if (h16) hipLaunchKernelGGL((decode_merge_kernel<R, B, true>), mg, block, 0, st, part, o, C, n_q, sink, oscale); \
        else hipLaunchKernelGGL((decode_merge_kernel<R, B, false>), mg, block, 0, st, part, o, C, n_q, sink, oscale);    \
    } while (0)
    if (relu2 && out_bf16) EMBLA_MG(true, true);
    else if (!relu2 && out_bf16) EMBLA_MG(false, true);
    else if (!relu2) EMBLA_MG(false, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_MG
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
