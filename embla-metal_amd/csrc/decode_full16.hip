// Decode over a bf16 full-layer cache (the reference without KV8): ReLU² with sink and the
// optional key scores (attn_full, Sources/EmblaMetal/Kernels/attention.metal:148-220), or softmax
// over every key or the selected rows (attn_sparse, attention.metal:370-441). q is the raw bf16 q of
// the q/k/v projection, head-normed with ng gains and rounded to bf16 in the kernel as the
// reference's kernels do (common.metal:13-26).
//
// MI355X design: the cache holds bf16 K and V in the 16-bit MFMA lane-order tiles the rings use
// (common.hpp, ES = 2), so S^T = K q^T and O += W V run on v_mfma_f32_16x16x32_bf16 with no
// conversion. A workgroup is (chunk of keys, kv head), 4 waves taking 32-key tiles with the next
// tile's loads in flight; q's query heads are the MFMA's columns (n < GQ live), so a lane (head n,
// lane group g) holds keys {16t + 4g + i} of a tile, exactly its A-operand slice of W V. With SEL,
// a wave first gathers its tile's 32 selected rows from the cache into a tile of its own in LDS
// (each row's K pairs and V elements at their tile places), then computes as on a cache tile.
// Chunk partials are merged by decode_merge_kernel (decode_full.hip).
#include "common.hpp"
#include "embla_internal.hpp"
#include "kv_row.hpp"

namespace embla {

namespace {

constexpr float LOG2E16 = 1.4426950408889634f;
constexpr int PS16 = HD + 4;   // floats a partial record: acc[128], m, l, pad (decode_merge_kernel's)

template <int GQ, bool RELU2, bool SCORES, bool SEL>
__global__ __launch_bounds__(256) void full16_decode_kernel(Full16Args a) {
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int j0 = c * a.CH, j1 = min(a.S, j0 + a.CH);
    const uint16_t* kbase = a.kc + (size_t)kvh * (a.max_s >> 5) * 4096;
    const uint16_t* vbase = a.vc + (size_t)kvh * (a.max_s >> 5) * 4096;

    // ---- q^T, B operand: lane (head n, group g), MFMA u: dims 32g + 8u .. + 7, bf16; head norm
    // with the gains in the oracle's summation order, then bf16 rounding
    u4_t qb[4];
    {
#pragma clang fp contract(off)
        const uint16_t* qr = a.q + (size_t)(kvh * GQ + (n < GQ ? n : 0)) * HD + 32 * g;
        float x[32];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const u4_t r = ld16(qr + 8 * u);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[8 * u + 2 * i] = bf2f((uint16_t)(r[i] & 0xFFFF));
                x[8 * u + 2 * i + 1] = bf2f((uint16_t)(r[i] >> 16));
            }
        }
        const float rf = 1.0f / sqrtf(sumsq_grouped32(x) / 128.0f + EPS32);
#pragma unroll
        for (int d = 0; d < 32; d++) {
            float gf = rf;
            if (a.ng >= 1) gf = gf * (1.0f + bf2f(a.g1[32 * g + d]));
            if (a.ng >= 2) gf = gf * (1.0f + bf2f(a.g2[32 * g + d]));
            x[d] = bf2f(f2bf(x[d] * gf));
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            u4_t r;
#pragma unroll
            for (int i = 0; i < 4; i++) r[i] = (uint32_t)f2bf(x[8 * u + 2 * i]) | ((uint32_t)f2bf(x[8 * u + 2 * i + 1]) << 16);
            qb[u] = n < GQ ? r : (u4_t){0, 0, 0, 0};
        }
    }

    // ---- tiles: a cache tile's lane slices, or (SEL) the wave's gathered tile in LDS
    __shared__ uint16_t gk[SEL ? 4 : 1][SEL ? 4096 : 8], gv[SEL ? 4 : 1][SEL ? 4096 : 8];
    u4_t Kt[2][8], Vt[2][8];
    auto load = [&](int t0, int b) {
        if constexpr (SEL) {
            // slot s <- row idx[kvh][t0 + s]: lane l moves dims 2l, 2l + 1 of every slot; slots
            // past j1 become zero rows
            const uint32_t* ix = a.idx + (size_t)kvh * a.S;
            for (int s = 0; s < 32; s++) {
                const int j = t0 + s;
                uint32_t kp = 0;
                uint16_t v0 = 0, v1 = 0;
                if (j < j1) {
                    const int r = (int)min(ix[j], (uint32_t)(a.max_s - 1));   // a stray index reads a real row
                    kp = *(const uint32_t*)(a.kc + kt_off(kvh, a.max_s, r, 2 * lane, 2) / 2);
                    v0 = a.vc[vt_off(kvh, a.max_s, r, 2 * lane, 2) / 2];
                    v1 = a.vc[vt_off(kvh, a.max_s, r, 2 * lane + 1, 2) / 2];
                }
                *(uint32_t*)(gk[w] + kt_off(0, 32, s, 2 * lane, 2) / 2) = kp;
                gv[w][vt_off(0, 32, s, 2 * lane, 2) / 2] = v0;
                gv[w][vt_off(0, 32, s, 2 * lane + 1, 2) / 2] = v1;
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int j = 0; j < 8; j++) { Kt[b][j] = ld16(gk[w] + lane * 8 + 512 * j); Vt[b][j] = ld16(gv[w] + lane * 8 + 512 * j); }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();   // the next gather rewrites the tile
        } else {
            const uint16_t* pk = kbase + (size_t)(t0 >> 5) * 4096 + lane * 8;
            const uint16_t* pv = vbase + (size_t)(t0 >> 5) * 4096 + lane * 8;
#pragma unroll
            for (int j = 0; j < 8; j++) { Kt[b][j] = ld16_stream(pk + 512 * j); Vt[b][j] = ld16_stream(pv + 512 * j); }
        }
    };
    constexpr int step = 32 * 4;
    const int tw = j0 + 32 * w;

    const float qs = 0.08838834764831845f;   // 1/sqrt(128)
    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};

    auto compute = [&](int t0, int b) {
        float x[8];
        bool valid[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f4_t st = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++) st = mfma16x<true>(Kt[b][4 * t + u], qb[u], st);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[4 * t + i] = st[i];
                valid[4 * t + i] = t0 + 16 * t + 4 * g + i < j1;
            }
        }
        if constexpr (SCORES) {   // max over the kv head's query heads of the raw q·k
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
            store_scores(a.scores + (size_t)kvh * a.max_s + t0 + 4 * g, smx, valid, t0 + 32 <= j1, n);
        }
        float p[8];
        if constexpr (RELU2) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float r = fmaxf(x[e] * qs, 0.0f);
                p[e] = valid[e] ? r * r : 0.0f;
                l += p[e];
            }
        } else {
            float mt = NEG_INF;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                x[e] = valid[e] ? x[e] * (qs * LOG2E16) : NEG_INF;
                mt = fmaxf(mt, x[e]);
            }
            mt = max_rows(mt);
            const float mn = fmaxf(m, mt);
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
#pragma unroll
            for (int e = 0; e < 8; e++) {
                p[e] = exp2f(x[e] - m);
                l += p[e];
            }
        }
        u4_t wb;
#pragma unroll
        for (int e = 0; e < 8; e += 2) wb[e / 2] = (uint32_t)f2bf(p[e]) | ((uint32_t)f2bf(p[e + 1]) << 16);
        if (t0 + 32 > j1) {
            // uniform: a partial tile; its masked keys' V elements (two a word, paired as the
            // weights) are zeroed so slots never written (NaN bits) add exactly 0
            u4_t mk;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int p0 = t0 + 16 * (k >> 1) + 4 * g + 2 * (k & 1);
                mk[k] = (p0 < j1 ? 0xFFFFu : 0u) | (p0 + 1 < j1 ? 0xFFFF0000u : 0u);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) Vt[b][u] &= mk;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) O[u] = mfma16x<true>(wb, Vt[b][u], O[u]);
    };

    if constexpr (SEL) {
        for (int t = tw; t < j1; t += step) {
            load(t, 0);
            compute(t, 0);
        }
    } else {
        if (tw < j1) load(tw, 0);
        if (tw + step < j1) load(tw + step, 1);
        for (int t = tw; t < j1; t += 2 * step) {
            compute(t, 0);
            if (t + 2 * step < j1) load(t + 2 * step, 0);
            if (t + step < j1) {
                compute(t + step, 1);
                if (t + 3 * step < j1) load(t + 3 * step, 1);
            }
        }
    }

    // ---- merge the 4 waves (LDS), then this chunk's partial (or o with one chunk)
    __shared__ __attribute__((aligned(16))) float om[4][GQ][HD];
    __shared__ float mm[4][GQ], ll[4][GQ];
    l = sum_rows(l);
    if (g == 0 && n < GQ) { mm[w][n] = m; ll[w][n] = l; }
    store_o_rows<GQ>(om[w], O, n, g);
    __syncthreads();
    constexpr int PER = GQ * HD / 256;
    const int oh = tid * PER / HD, od = tid * PER % HD;
    float f[4], L = 0.0f, M;
    if constexpr (RELU2) {
        M = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) { f[ww] = 1.0f; L += ll[ww][oh]; }
    } else {
        M = fmaxf(fmaxf(mm[0][oh], mm[1][oh]), fmaxf(mm[2][oh], mm[3][oh]));
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            f[ww] = mm[ww][oh] == NEG_INF ? 0.0f : exp2f(mm[ww][oh] - M);
            L += ll[ww][oh] * f[ww];
        }
    }
    float acc[PER];
#pragma unroll
    for (int e = 0; e < PER; e++) {
        float s = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) s += om[ww][oh][od + e] * f[ww];
        acc[e] = s;
    }
    const int hq = kvh * GQ + oh;
    if (a.C == 1) {
        const float inv = RELU2 ? 1.0f / (11.313708498984761f + L) : 1.0f / L;
#pragma unroll
        for (int e = 0; e < PER; e++) a.o[(size_t)hq * HD + od + e] = f2bf(acc[e] * inv);
        return;
    }
    float* pp = a.part + ((size_t)c * a.n_q + hq) * PS16;
#pragma unroll
    for (int e = 0; e < PER; e++) pp[od + e] = acc[e];
    if (od == 0) { pp[HD] = M; pp[HD + 1] = L; }
}

}  // namespace

int launch_full16_decode(const Full16Args& a, hipStream_t st) {
    const dim3 grid(a.C, a.n_kv), block(256);
    const int gq = a.n_q / a.n_kv;
    const bool sc = a.scores != nullptr, sel = a.idx != nullptr;
#define EMBLA_F16D(GQ, R, SC, SL) hipLaunchKernelGGL((full16_decode_kernel<GQ, R, SC, SL>), grid, block, 0, st, a)
    if (gq == 8 && a.relu2 && !sel && sc) EMBLA_F16D(8, true, true, false);
    else if (gq == 8 && a.relu2 && !sel && !sc) EMBLA_F16D(8, true, false, false);
    else if (gq == 8 && !a.relu2 && !sel && !sc) EMBLA_F16D(8, false, false, false);
    else if (gq == 8 && !a.relu2 && sel && !sc) EMBLA_F16D(8, false, false, true);
    else if (gq == 4 && a.relu2 && !sel && !sc) EMBLA_F16D(4, true, false, false);
    else if (gq == 4 && !a.relu2 && !sel && !sc) EMBLA_F16D(4, false, false, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_F16D
    if (a.C > 1) return launch_decode_merge(a.part, a.o, a.C, a.n_q, a.relu2, true, 1.0f, st);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
