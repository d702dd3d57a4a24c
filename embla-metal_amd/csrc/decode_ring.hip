// Sliding-window decode over a 16-bit ring (fp16 or bf16), one query token.
//
// Follows attn_sliding (Sources/EmblaMetal/Kernels/attention.metal:26-102): softmax over the last
// min(pos + 1, W) positions, the current one included; the current k, v are written into the ring
// slot pos % R. With pre-ops (the reference's sliding layers) q and k are RMS-normed with their
// gains and rotated (head_norm + rope, common.metal:13-51) and rounded to bf16 first.
//
// MI355X design: the ring holds K and V in the MFMA lane-order 32-key tiles (common.hpp, ES = 2), so
// S^T = K q^T and O += W V run on v_mfma_f32_16x16x32_{f16,bf16} with no conversion of K or V.
// Workgroups split the window's ring part (positions lo .. pos-1) into chunks; the current key is
// one extra row taken from the inputs by the last chunk's workgroup (its wave with the fewest
// tiles: C2 7.87 -> 7.18 us a step against its first wave after that wave's tiles), which also
// writes it into the ring (no other workgroup reads that slot in this launch, W <= R). Chunk partials are merged by
// decode_merge_kernel (decode_full.hip).
#include "common.hpp"
#include "embla_internal.hpp"
#include "kv_row.hpp"

namespace embla {

constexpr float RLOG2E = 1.4426950408889634f;
constexpr int RPS = HD + 4;   // partial record stride, as decode_full.hip

/// Prepared row (norm with gains, RoPE, bf16 rounding when PREOPS), dims 32g .. 32g + 31 of a head
/// held by the 4 lanes n, n+16, n+32, n+48 (lane group g), as fp32 in x[32].
template <bool BF, bool PREOPS>
__device__ __forceinline__ void prep_row(const u4_t* raw, const uint16_t* gain, int g, int pos, float* x) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const u4_t r = raw[u];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[8 * u + 2 * i] = a2f<BF>((uint16_t)(r[i] & 0xFFFF));
            x[8 * u + 2 * i + 1] = a2f<BF>((uint16_t)(r[i] >> 16));
        }
    }
    if constexpr (PREOPS) {
#pragma clang fp contract(off)
        const float r = 1.0f / sqrtf(sumsq_grouped32(x) / 128.0f + EPS32);
#pragma unroll
        for (int d = 0; d < 32; d++) x[d] = x[d] * (r * (1.0f + bf2f(gain[32 * g + d])));
        // rotate dims (d, d + 32), d < 32: lane group 0 holds d, group 1 holds d + 32
#pragma unroll
        for (int d = 0; d < 32; d++) {
            const float other = xchg_xor16(x[d]);
            if (g < 2) {
                float cs, sn;
                rope_cs(pos, d, cs, sn);
                x[d] = g == 0 ? x[d] * cs - other * sn : other * sn + x[d] * cs;
            }
        }
#pragma unroll
        for (int d = 0; d < 32; d++) x[d] = bf2f(f2bf(x[d]));
    }
}

template <int GQ, bool BF, bool PREOPS>
__global__ __launch_bounds__(256) void ring_decode_kernel(RingArgs a) {
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int pos = a.pos, R = a.R;
    const int lo = max(0, pos - a.W + 1);           // first position of the window
    const int t_first = lo & ~31;                   // first tile (position space)
    const int j0 = t_first + c * a.CH, j1 = min(pos, t_first + (c + 1) * a.CH);   // ring part [.., pos)

    // tile loads: position p lives at ring slot p % R (R % 32 == 0, so a tile never wraps)
    auto tbase = [&](int p) { return (size_t)(kvh * (R >> 5) + ((p % R) >> 5)) * 4096; };
    u4_t Kt[2][8], Vt[2][8];
    auto load = [&](int p, int b) {
        const uint16_t* pk = a.kring + tbase(p) + lane * 8;
        const uint16_t* pv = a.vring + tbase(p) + lane * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) { Kt[b][j] = ld16(pk + 512 * j); Vt[b][j] = ld16(pv + 512 * j); }
    };
    constexpr int step = 32 * 4;
    const int tw = j0 + 32 * w;
    // q's row is requested before the tiles (loads complete in order: after them, its wait would
    // also wait for the tiles)
    u4_t qraw[4];
    {
        const uint16_t* qr = a.q + (size_t)(kvh * GQ + (n < GQ ? n : 0)) * a.q_stride + 32 * g;
#pragma unroll
        for (int u = 0; u < 4; u++) qraw[u] = ld16(qr + 8 * u);
    }
    if (tw < j1) load(tw, 0);
    if (tw + step < j1) load(tw + step, 1);

    // q^T, B operand: lane (head n, group g), MFMA u: dims 32g + 8u .. + 7
    u4_t qb[4];
    if constexpr (PREOPS) {
        float x[32];
        prep_row<BF, PREOPS>(qraw, a.qg, g, pos, x);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            u4_t r;
#pragma unroll
            for (int i = 0; i < 4; i++)
                r[i] = (uint32_t)f2a<BF>(x[8 * u + 2 * i]) | ((uint32_t)f2a<BF>(x[8 * u + 2 * i + 1]) << 16);
            qb[u] = n < GQ ? r : (u4_t){0, 0, 0, 0};
        }
    } else {
        // the row's 16-bit values are the operand as they are; columns n >= GQ repeat head 0
        // (finite, and no result reads them: heads are the rows below GQ)
#pragma unroll
        for (int u = 0; u < 4; u++) qb[u] = qraw[u];
    }
    const float sc = 0.08838834764831845f * RLOG2E;
    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};

    // one softmax step for scores x[8] (item e = 4t + i <-> key 16t + 4g + i) and A operand rows
    auto softmax_step = [&](float* x, h8_t& wa_bits) {
        float mt = NEG_INF;
#pragma unroll
        for (int e = 0; e < 8; e++) mt = fmaxf(mt, x[e]);
        mt = max_rows(mt);
        const float mn = fmaxf(m, mt);
        if (__any(n < GQ && mn > m)) {
            if (__any(n < GQ && m != NEG_INF)) {
                const float corr = m == NEG_INF ? 0.0f : exp2f(m - mn);
                l *= corr;
                float cf[4];
#pragma unroll
                for (int i = 0; i < 4; i++) cf[i] = readlane(corr, i);
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 4; i++) O[u][i] *= cf[i];
            }
            m = mn;
        }
        u4_t wb;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float p0 = exp2f(x[e] - m), p1 = exp2f(x[e + 1] - m);
            l += p0 + p1;
            wb[e / 2] = (uint32_t)f2a<BF>(p0) | ((uint32_t)f2a<BF>(p1) << 16);
        }
        wa_bits = __builtin_bit_cast(h8_t, wb);
    };

    auto compute = [&](int t0, int b) {
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f4_t st = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++) st = mfma16x<BF>(Kt[b][4 * t + u], qb[u], st);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = t0 + 16 * t + 4 * g + i;
                x[4 * t + i] = p >= lo && p < j1 ? st[i] * sc : NEG_INF;
            }
        }
        h8_t wa;
        softmax_step(x, wa);
        const u4_t wu = __builtin_bit_cast(u4_t, wa);
        if (!(t0 >= lo && t0 + 32 <= j1)) {
            // uniform: a partial tile. The masked keys' V elements (the same 8 key items as the
            // weights, two a word) are zeroed, so slots never written (NaN bits) add exactly 0.
            u4_t mk;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int p0 = t0 + 16 * (k >> 1) + 4 * g + 2 * (k & 1);
                mk[k] = (p0 >= lo && p0 < j1 ? 0xFFFFu : 0u) | (p0 + 1 >= lo && p0 + 1 < j1 ? 0xFFFF0000u : 0u);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) Vt[b][u] &= mk;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) O[u] = mfma16x<BF>(wu, Vt[b][u], O[u]);
    };

    for (int t = tw; t < j1; t += 2 * step) {
        compute(t, 0);
        if (t + 2 * step < j1) load(t + 2 * step, 0);
        if (t + step < j1) {
            compute(t + step, 1);
            if (t + 3 * step < j1) load(t + 3 * step, 1);
        }
    }

    // the current key: one extra row, taken by wave 3 of the last chunk's workgroup (tiles are
    // dealt to waves 0, 1, 2, 3 in turn, so wave 3 has the fewest, none in a chunk of up to 3
    // tiles, and its loads of the new rows overlap the other waves' tiles)
    if (c == a.C - 1 && w == 3) {
        float kx[32], vx[32];
        u4_t kr[4], vr[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            kr[u] = ld16(a.k_new + (size_t)kvh * HD + 32 * g + 8 * u);
            vr[u] = ld16(a.v_new + (size_t)kvh * HD + 32 * g + 8 * u);
        }
        prep_row<BF, PREOPS>(kr, a.kg, g, pos, kx);
        prep_row<BF, false>(vr, nullptr, g, pos, vx);
        // q·k for head n: this lane's 32 dims, then the 4 lane groups
        float dot = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                dot += a2f<BF>((uint16_t)(qb[u][i] & 0xFFFF)) * kx[8 * u + 2 * i];
                dot += a2f<BF>((uint16_t)(qb[u][i] >> 16)) * kx[8 * u + 2 * i + 1];
            }
        dot = sum_rows(dot);
        float x[8];
        x[0] = dot * sc;
#pragma unroll
        for (int e = 1; e < 8; e++) x[e] = NEG_INF;
        // softmax_step's rescale and sums, with this lane's key slot 0 live only in group 0
        if (g != 0) x[0] = NEG_INF;
        h8_t wa;
        softmax_step(x, wa);
        // O[u][i] (head 4g + i, dim 8n + u) += p_(head) * v[8n + u]: p of head h is in lane h
        const float p = exp2f(x[0] - m);   // lanes n: head n (group 0)
        float ph[4];
#pragma unroll
        for (int i = 0; i < 4; i++) ph[i] = readlane(p, i);
        // v dims 8n .. 8n + 7 sit in lane group (8n) / 32 = n / 4, items 8 (n % 4) ..
        float vd[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int src = (n >> 2) * 16;   // a lane of group n / 4 (any n' holds the same dims)
            vd[u] = __shfl(vx[8 * (n & 3) + u], src + n, 64);
        }
        if (g == 0) {
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int i = 0; i < 4; i++) O[u][i] += ph[i] * vd[u];
        }
        // the ring slot of pos: K and V rows at their tile places (ES = 2)
        if (n == 0) {
#pragma unroll
            for (int d = 0; d < 32; d++) {
                a.kring[kt_off(kvh, R, pos % R, 32 * g + d, 2) / 2] = f2a<BF>(kx[d]);
                a.vring[vt_off(kvh, R, pos % R, 32 * g + d, 2) / 2] = f2a<BF>(vx[d]);
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
    const float M = fmaxf(fmaxf(mm[0][oh], mm[1][oh]), fmaxf(mm[2][oh], mm[3][oh]));
    float f[4], L = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++) {
        f[ww] = mm[ww][oh] == NEG_INF ? 0.0f : exp2f(mm[ww][oh] - M);
        L += ll[ww][oh] * f[ww];
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
#pragma unroll
        for (int e = 0; e < PER; e++) a.o[(size_t)hq * HD + od + e] = f2a<BF>(acc[e] / L);
        return;
    }
    float* pp = a.part + ((size_t)c * a.n_kv * GQ + hq) * RPS;
#pragma unroll
    for (int e = 0; e < PER; e++) pp[od + e] = acc[e];
    if (od == 0) { pp[HD] = M; pp[HD + 1] = L; }
}

int launch_ring_decode(const RingArgs& a, hipStream_t st) {
    const dim3 grid(a.C, a.n_kv), block(256);
    const int gq = a.n_q / a.n_kv;
    if (gq != 4) return EMBLA_ERR_UNSUPPORTED;
    if (a.bf16 && a.preops) hipLaunchKernelGGL((ring_decode_kernel<4, true, true>), grid, block, 0, st, a);
    else if (a.bf16) hipLaunchKernelGGL((ring_decode_kernel<4, true, false>), grid, block, 0, st, a);
    else if (!a.preops) hipLaunchKernelGGL((ring_decode_kernel<4, false, false>), grid, block, 0, st, a);
    else return EMBLA_ERR_UNSUPPORTED;
    if (a.C > 1) return launch_decode_merge(a.part, a.o, a.C, a.n_q, false, a.bf16, 1.0f, st);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
