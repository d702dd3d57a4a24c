// Sparse-layer decode: softmax attention over a gathered set of cache rows (16-bit K/V), one query.
//
// Follows attn_sparse / attn_sparse8 with SEL (Sources/EmblaMetal/Kernels/attention.metal:370-441,
// 448-584): keys are the rows idx[kv head][j] (or one set shared by every kv head, as the BASELINE
// config C4's selection), split into chunks whose partials are merged afterwards
// (decode_merge_kernel, decode_full.hip).
//
// MI355X design: the rows are gathered by a wave 32 at a time (each 16-byte load of the wave covers
// four whole 256-byte rows) into a wave-private LDS tile with a padded row stride; the MFMA A
// operand of S^T = K q^T is read back from it as 16-byte rows, and the V operand of O += W V is
// assembled from eight 16-byte row reads a lane (a register transpose), so both products run on
// v_mfma_f32_16x16x32_{f16,bf16}.
//
// In the sparse-layer step (embla_sparse_layer_decode) the rows come straight from the wide select:
// each workgroup runs the select's last step for the ranks it attends (wsel_slice, wsel.hpp) in
// its staging LDS before the first gather, so the selection needs no launch of its own and no
// round trip through the index list; kv head 0's workgroups still write the list.
#include "common.hpp"
#include "embla_internal.hpp"
#include "wsel.hpp"

namespace embla {

constexpr int SROW = HD + 8;   // LDS row stride in 16-bit elements (272 bytes: conflict-free rows)
constexpr int SPS = HD + 4;    // partial record stride, as decode_full.hip
constexpr int SPR_MAXSEL = 1152;   // keys a row of the batched gathered attention (top-k + recent)

template <bool BF>
__device__ __forceinline__ f4_t mfma16s(u4_t a, u4_t b, f4_t c) {
    if constexpr (BF) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}


constexpr int SPD_FS_MAXCH = kSparseFusedMaxCh;

template <int GQ, bool BF, bool FS>
__global__ __launch_bounds__(256) void sparse_decode_kernel(SparseArgs a) {
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int j0 = c * a.CH, j1 = min(a.nsel, j0 + a.CH);
    const uint32_t* rows = a.idx ? a.idx + (size_t)kvh * a.idx_stride : nullptr;   // null: rows 0 .. nsel-1
    const uint16_t* kb = a.kc + (size_t)kvh * a.max_s * HD;
    const uint16_t* vb = a.vc + (size_t)kvh * a.max_s * HD;

    __shared__ __attribute__((aligned(16))) uint16_t stage[4][2][32 * SROW];
    uint16_t* Ks = stage[w][0];
    uint16_t* Vs = stage[w][1];
    __shared__ uint32_t srows[FS ? SPD_FS_MAXCH : 1];   // FS: the chunk's selected rows
    static_assert(sizeof(stage) / 4 >= WSL_FIXED + 2, "the staging LDS holds the select's last step");
    if constexpr (FS) {
        // ranks j0 .. ts - 1 of the selection, from the wide select's last step (its scratch is
        // the staging LDS, free until the first gather); the rows go to the output at the end
        const int ts = min(j1, a.sel_topk);
        if (j0 < ts)   // uniform
            wsel_slice<256>(a.sel_n, a.sel_topk, a.sel_ws, (uint32_t*)&stage[0][0][0], (int)(sizeof(stage) / 4),
                            (uint32_t)j0, (uint32_t)(ts - j0), srows, nullptr);
        __syncthreads();
    }

    // q^T, B operand: lane (head n, group g), MFMA u: dims 32g + 8u .. + 7
    u4_t qb[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const u4_t r = ld16(a.q + (size_t)(kvh * GQ + (n < GQ ? n : 0)) * HD + 32 * g + 8 * u);
        qb[u] = n < GQ ? r : (u4_t){0, 0, 0, 0};
    }
    const float sc = 0.08838834764831845f * 1.4426950408889634f;
    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};

    for (int t0 = j0 + 32 * w; t0 < j1; t0 += 128) {
        // gather: load j covers rows 4j .. 4j + 3, lane l: row 4j + l / 16, dims 8 (l % 16) ..
        // the 8 row indices first, with no branch (an index read a row behind its own wait put 8
        // round trips before the last load): keys past the chunk's last (p >= j1) take row 0,
        // their index reads clamped in range and discarded
        int r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = t0 + 4 * j + (lane >> 4);
            if constexpr (FS) {
                const int sr = (int)srows[min(p - j0, SPD_FS_MAXCH - 1)];
                r[j] = p < j1 ? (p < a.sel_topk ? sr : a.sel_n + p - a.sel_topk) : 0;
            } else {
                r[j] = rows ? (int)rows[min(p, j1 - 1)] : p;
                r[j] = p < j1 ? r[j] : 0;
            }
        }
        u4_t kr[8], vr[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const size_t row = (size_t)min(r[j], a.max_s - 1);   // rows clamped in range
            kr[j] = ld16(kb + row * HD + 8 * n);
            vr[j] = ld16(vb + row * HD + 8 * n);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int r = 4 * j + (lane >> 4);
            *(u4_t*)(Ks + r * SROW + 8 * n) = kr[j];
            *(u4_t*)(Vs + r * SROW + 8 * n) = vr[j];
        }
        wave_lds_sync();
        // S^T: lane (head n, group g) item i of half t = key 16t + 4g + i
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f4_t st = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++)
                st = mfma16s<BF>(*(const u4_t*)(Ks + (16 * t + n) * SROW + 32 * g + 8 * u), qb[u], st);
#pragma unroll
            for (int i = 0; i < 4; i++) x[4 * t + i] = t0 + 16 * t + 4 * g + i < j1 ? st[i] * sc : NEG_INF;
        }
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
                for (int i = 0; i < 4; i++) {
                    const float c0 = readlane(corr, i);
                    if constexpr (GQ == 8) cf[i] = g == 1 ? readlane(corr, 4 + i) : c0;
                    else cf[i] = c0;
                }
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
        // V operand: lane (dim column n, group g), MFMA u = dim 8n + u, item e = key 16t + 4g + i
        u4_t vrow[8];
#pragma unroll
        for (int e = 0; e < 8; e++) vrow[e] = *(const u4_t*)(Vs + (16 * (e >> 2) + 4 * g + (e & 3)) * SROW + 8 * n);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            u4_t b;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const uint32_t lo = (vrow[e][u >> 1] >> (16 * (u & 1))) & 0xFFFF;
                const uint32_t hi = (vrow[e + 1][u >> 1] >> (16 * (u & 1))) & 0xFFFF;
                b[e / 2] = lo | (hi << 16);
            }
            O[u] = mfma16s<BF>(wb, b, O[u]);
        }
        wave_lds_sync();   // the next tile's stores come after every lane's reads
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
    if constexpr (FS) {   // kv head 0's workgroups write the selection; one thread advances the epoch
        if (kvh == 0 && a.sel_out)
            for (int p = j0 + tid; p < j1; p += 256)
                a.sel_out[p] = p < a.sel_topk ? srows[p - j0] : (uint32_t)(a.sel_n + p - a.sel_topk);
        if (c == 0 && kvh == 0 && tid == 0) *a.sel_epoch += 1;   // the next call's histogram buffer
    }
    if (a.C == 1) {
#pragma unroll
        for (int e = 0; e < PER; e++) a.o[(size_t)hq * HD + od + e] = f2a<BF>(acc[e] / L);
        return;
    }
    float* pp = a.part + ((size_t)c * a.n_kv * GQ + hq) * SPS;
#pragma unroll
    for (int e = 0; e < PER; e++) pp[od + e] = acc[e];
    if (od == 0) { pp[HD] = M; pp[HD + 1] = L; }
}

int launch_sparse_decode(const SparseArgs& a, hipStream_t st) {
    const dim3 grid(a.C, a.n_kv), block(256);
    const int gq = a.n_q / a.n_kv;
    const bool fs = a.sel_ws != nullptr;
    if (fs && (a.CH > SPD_FS_MAXCH || !a.sel_epoch || a.sel_topk <= 0 || a.sel_n <= a.sel_topk ||
               a.sel_n > SEL_MAXN || a.nsel < a.sel_topk))
        return EMBLA_ERR_INVALID;
#define EMBLA_SPD(G, B)                                                                         \
    do {                                                                                        \
        if (fs) hipLaunchKernelGGL((sparse_decode_kernel<G, B, true>), grid, block, 0, st, a);  \
        else hipLaunchKernelGGL((sparse_decode_kernel<G, B, false>), grid, block, 0, st, a);    \
    } while (0)
    if (gq == 4 && !a.bf16) EMBLA_SPD(4, false);
    else if (gq == 4 && a.bf16) EMBLA_SPD(4, true);
    else if (gq == 8 && a.bf16) EMBLA_SPD(8, true);
    else if (gq == 8 && !a.bf16) EMBLA_SPD(8, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_SPD
    if (a.C > 1) return launch_decode_merge(a.part, a.o, a.C, a.n_q, false, a.bf16, 1.0f, st);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

/// Gathered attention over an int8 cache: one workgroup a (key chunk, kv head, query row), its 4
/// waves taking interleaved 32-key steps of the chunk's key list (held in LDS, so gathers need no
/// dependent load). A wave gathers 32 keys of K and V, widens them to fp16 (exact) into its LDS
/// stage, and runs the same MFMA scheme as sparse_decode_kernel; each key's scale multiplies its
/// score, each value row's scale (x 64, into fp16's normal range) its weight.
///  - row-major cache (the sparse prefill's): each 16-byte load covers eight 128-byte rows, and the
///    next step's gather is in flight during this step's products;
///  - MFMA tile cache (the full layer's, for the reference's attn_sparse8 with SEL,
///    attention.metal:448-584): a key's K row is 8 whole 16-byte pieces of its tile; its V row is
///    interleaved with 7 other keys' (2 bytes of each of 64 pieces), so V is gathered 8x over.
template <int GQ, bool TILES, bool SCALE32>
__global__ __launch_bounds__(256) void sparse_rows8_kernel(SparseRows8Args a) {
    const int c = blockIdx.x, kvh = blockIdx.y, r = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int pos = a.p0 + r;
    const bool sel = a.idx && pos + 1 > a.nsel;
    const int nk_all = sel ? a.nsel : pos + 1;
    const int j0 = c * a.CH, nk = min(nk_all, j0 + a.CH) - j0;   // this chunk's keys
    const size_t nrow = (size_t)a.n_kv * a.max_s * HD;
    const int8_t* kb = TILES ? a.kc : a.kc + (size_t)kvh * a.max_s * HD;
    const int8_t* vb = TILES ? a.vc : a.vc + (size_t)kvh * a.max_s * HD;
    constexpr int ES = SCALE32 ? 4 : 2;
    const char* ksc = (const char*)(a.kc + nrow) + (size_t)kvh * a.max_s * ES;
    const char* vsc = (const char*)(a.vc + nrow) + (size_t)kvh * a.max_s * ES;
    auto scale_at = [&](const char* base, size_t row) -> float {
        if constexpr (SCALE32) return *(const float*)(base + row * 4);
        else return h2f(*(const uint16_t*)(base + row * 2));
    };

    // the stage (per wave: 32 K and 32 V rows as fp16) and, after the loop, the merge buffers
    constexpr int STAGE = 4 * 2 * 32 * SROW * 2;
    constexpr int MERGE = (4 * GQ * HD + 8 * GQ) * 4;
    __shared__ __attribute__((aligned(16))) char smem[STAGE > MERGE ? STAGE : MERGE];
    __shared__ uint32_t sidx[SPR_MAXSEL];
    __shared__ float sks[4][32], svs[4][32];
    uint16_t* Ks = (uint16_t*)smem + (2 * w) * 32 * SROW;
    uint16_t* Vs = Ks + 32 * SROW;

    // the chunk's key list into LDS (rows clamped in range)
    const uint32_t* rows = sel ? a.idx + (size_t)r * a.idx_row_stride + (size_t)kvh * a.idx_kv_stride : nullptr;
    for (int p = tid; p < nk; p += 256) sidx[p] = (uint32_t)min(rows ? (int)rows[j0 + p] : j0 + p, a.max_s - 1);
    __syncthreads();

    // q^T, B operand (fp16): lane (head n, group g), MFMA u: dims 32g + 8u .. + 7
    u4_t qb[4];
    {
        const uint16_t* qr = a.q + (size_t)r * a.q_row_stride + (size_t)(kvh * GQ + (n < GQ ? n : 0)) * HD;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            u4_t v = ld16(qr + 32 * g + 8 * u);
            if (a.q_bf16) v = __builtin_bit_cast(u4_t, bf8_to_h8(v));
            qb[u] = n < GQ ? v : (u4_t){0, 0, 0, 0};
        }
    }
    const float sc = 0.08838834764831845f * 1.4426950408889634f;
    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};

    // row-major gather of one 32-key step: load j covers keys t0 + 8j .. + 7, lane l: key
    // t0 + 8j + l / 8, dims 16 (l % 8) ..; lanes < 32 also fetch key t0 + l's two scales
    u4_t kr[4], vr[4];
    float s_k = 0.0f, s_v = 0.0f;
    auto gather_rows = [&](int t0) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int p = t0 + 8 * j + (lane >> 3);
            const size_t row = p < nk ? sidx[p] : 0;
            kr[j] = ld16(kb + row * HD + 16 * (lane & 7));
            vr[j] = ld16(vb + row * HD + 16 * (lane & 7));
        }
    };
    auto gather_scales = [&](int t0) {
        if (lane < 32) {
            const int p = t0 + lane;
            const size_t row = p < nk ? sidx[p] : 0;
            s_k = scale_at(ksc, row);
            s_v = scale_at(vsc, row);
        }
    };
    // tile gather straight into the stage: lane l takes key slot l / 2, half l % 2 (64 dims)
    auto gather_tiles = [&](int t0) {
        const int s = lane >> 1, hf = lane & 1, p = t0 + s;
        const int row = p < nk ? (int)sidx[p] : 0;
        const int m16 = row & 15, t = (row >> 4) & 1, gq = (row >> 2) & 3, i = row & 3;
        const int8_t* kt = kb + tile_base(kvh, a.max_s, row, 1);
        const int8_t* vt = vb + tile_base(kvh, a.max_s, row, 1);
        u4_t kp[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {   // dims 32 (2hf + e/2) + 16 (e%2) .. + 15
            const int gg = 2 * hf + (e >> 1), jj = e & 1;
            kp[e] = ld16(kt + ((2 * t + jj) * 64 + m16 + 16 * gg) * 16);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint16_t* kd = Ks + s * SROW + 32 * (2 * hf + (e >> 1)) + 16 * (e & 1);
            *(h8_t*)kd = i8x8_to_h8(kp[e][0], kp[e][1]);
            *(h8_t*)(kd + 8) = i8x8_to_h8(kp[e][2], kp[e][3]);
        }
#pragma unroll
        for (int nn = 0; nn < 8; nn++) {   // dims 8 (8hf + nn) + u, u = 0..7: 4 pieces, 2 bytes each
            const int n2 = 8 * hf + nn;
            u4_t vp[4];
#pragma unroll
            for (int j = 0; j < 4; j++) vp[j] = ld16(vt + (j * 64 + n2 + 16 * gq) * 16);
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t b0 = (vp[j][t] >> (8 * i)) & 0xFF, b1 = (vp[j][2 + t] >> (8 * i)) & 0xFF;
                const uint32_t pair = b0 | (b1 << 8);   // dims 2j, 2j + 1
                if (j < 2) lo |= pair << (16 * j);
                else hi |= pair << (16 * (j - 2));
            }
            *(h8_t*)(Vs + s * SROW + 8 * n2) = i8x8_to_h8(lo, hi);
        }
    };
    if constexpr (!TILES) {
        if (32 * w < nk) { gather_rows(32 * w); gather_scales(32 * w); }
    }
    for (int t0 = 32 * w; t0 < nk; t0 += 128) {
        if constexpr (TILES) {
            gather_scales(t0);
            gather_tiles(t0);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int rr = 8 * j + (lane >> 3);
                uint16_t* kd = Ks + rr * SROW + 16 * (lane & 7);
                uint16_t* vd = Vs + rr * SROW + 16 * (lane & 7);
                *(h8_t*)kd = i8x8_to_h8(kr[j][0], kr[j][1]);
                *(h8_t*)(kd + 8) = i8x8_to_h8(kr[j][2], kr[j][3]);
                *(h8_t*)vd = i8x8_to_h8(vr[j][0], vr[j][1]);
                *(h8_t*)(vd + 8) = i8x8_to_h8(vr[j][2], vr[j][3]);
            }
        }
        if (lane < 32) { sks[w][lane] = s_k * sc; svs[w][lane] = s_v * 64.0f; }
        if constexpr (!TILES) {
            if (t0 + 128 < nk) { gather_rows(t0 + 128); gather_scales(t0 + 128); }   // in flight during the products
        }
        wave_lds_sync();
        // S^T: lane (head n, group g) item i of half t = key 16t + 4g + i
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f4_t st = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++)
                st = mfma16s<false>(*(const u4_t*)(Ks + (16 * t + n) * SROW + 32 * g + 8 * u), qb[u], st);
            const f4_t kq = *(const f4_t*)(&sks[w][16 * t + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; i++) x[4 * t + i] = t0 + 16 * t + 4 * g + i < nk ? st[i] * kq[i] : NEG_INF;
        }
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
                for (int i = 0; i < 4; i++) {
                    const float c0 = readlane(corr, i);
                    if constexpr (GQ == 8) cf[i] = g == 1 ? readlane(corr, 4 + i) : c0;
                    else cf[i] = c0;
                }
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 4; i++) O[u][i] *= cf[i];
            }
            m = mn;
        }
        u4_t wb;
        const f4_t vq0 = *(const f4_t*)(&svs[w][4 * g]), vq1 = *(const f4_t*)(&svs[w][16 + 4 * g]);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float p0 = exp2f(x[e] - m), p1 = exp2f(x[e + 1] - m);
            l += p0 + p1;
            const float s0 = e < 4 ? vq0[e & 3] : vq1[e & 3], s1 = e < 4 ? vq0[(e + 1) & 3] : vq1[(e + 1) & 3];
            wb[e / 2] = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)(p0 * s0), (_Float16)(p1 * s1)});
        }
        // V operand: lane (dim column n, group g), MFMA u = dim 8n + u, item e = key 16t + 4g + i
        u4_t vrow[8];
#pragma unroll
        for (int e = 0; e < 8; e++) vrow[e] = *(const u4_t*)(Vs + (16 * (e >> 2) + 4 * g + (e & 3)) * SROW + 8 * n);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            u4_t b;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const uint32_t lo = (vrow[e][u >> 1] >> (16 * (u & 1))) & 0xFFFF;
                const uint32_t hi = (vrow[e + 1][u >> 1] >> (16 * (u & 1))) & 0xFFFF;
                b[e / 2] = lo | (hi << 16);
            }
            O[u] = mfma16s<false>(wb, b, O[u]);
        }
        wave_lds_sync();   // the next step's stores come after every lane's reads
    }

    // ---- merge the 4 waves (LDS, over the stage), then the row's output or this chunk's partial
    __syncthreads();
    float (*om)[GQ][HD] = (float (*)[GQ][HD])smem;
    float (*mm)[GQ] = (float (*)[GQ])(smem + 4 * GQ * HD * 4);
    float (*ll)[GQ] = (float (*)[GQ])(smem + (4 * GQ * HD + 4 * GQ) * 4);
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
    const int hq = kvh * GQ + oh;
    if (a.C > 1) {   // partial: O x 64 unnormalised, m, l (decode_merge_kernel with oscale 64)
        float* pp = a.part + ((size_t)c * a.n_q + hq) * SPS;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            float s = 0.0f;
#pragma unroll
            for (int ww = 0; ww < 4; ww++) s += om[ww][oh][od + e] * f[ww];
            pp[od + e] = s;
        }
        if (od == 0) { pp[HD] = M; pp[HD + 1] = L; }
        return;
    }
    const float inv = 1.0f / (64.0f * L);
    uint16_t* orow = a.o + (size_t)r * a.o_row_stride + (size_t)hq * HD + od;
#pragma unroll
    for (int e = 0; e < PER; e++) {
        float s = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) s += om[ww][oh][od + e] * f[ww];
        orow[e] = a.o_bf16 ? f2bf(s * inv) : f2h(s * inv);
    }
}


/// Gathered attention over a row-major int8 cache held entirely in registers (the sparse prefill's
/// cache): one workgroup a (key chunk, kv head, query row), its 4 waves taking interleaved 32-key
/// steps of the chunk's key list (in LDS). No stage: S^T = K q^T runs on v_mfma_i32_16x16x64_i8
/// straight on the gathered K bytes, q being a 15-bit fixed point split exactly into int8 halves
/// (hi in column n, lo in column n + GQ of the B operand; the scheme of full_decode_kernel), so the
/// scores are exact integers times the fixed point's step. A lane (head n, group g) of the score
/// tile holds keys {16t + 4g + i}, the A-operand slice of O += W V; it reads those 8 keys' V
/// bytes for dims 8n .. 8n + 7 (8 bytes a key, a row's 128 bytes over 16 lanes) and transposes
/// them into the fp16 B operand in registers. K and V go through per-wave LDS tiles, gathered as
/// whole rows (each cache line once a load: the gathers' address work bounds this kernel); as soon
/// as a step's rows are in the tiles, the next step's K and V rows are requested, so they are in
/// flight through this whole step.
// three workgroups a CU (C5 sparse layer 0.403 ms at four with the V rows requested at a step's
// end in the A layout, 0.380 at three, 0.374 with them a step ahead, 0.361 through the tile)
#ifndef SPR_OCC
#define SPR_OCC 3
#endif

template <int GQ>
__global__ __launch_bounds__(256, SPR_OCC) void sparse_rows8_rm_kernel(SparseRows8Args a) {
    typedef int i4_t __attribute__((ext_vector_type(4)));
    constexpr float QFIX = 32000.0f;   // |q_int| <= 32000: |hi| <= 125
    const int c = blockIdx.x, kvh = blockIdx.y, r = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int pos = a.p0 + r;
    const bool sel = a.idx && pos + 1 > a.nsel;
    const int nk_all = sel ? a.nsel : pos + 1;
    const int j0 = c * a.CH, nk = min(nk_all, j0 + a.CH) - j0;   // this chunk's keys
    const size_t nrow = (size_t)a.n_kv * a.max_s * HD;
    const int8_t* kb = a.kc + (size_t)kvh * a.max_s * HD;
    const int8_t* vb = a.vc + (size_t)kvh * a.max_s * HD;
    const uint16_t* ksc = (const uint16_t*)(a.kc + nrow) + (size_t)kvh * a.max_s;
    const uint16_t* vsc = (const uint16_t*)(a.vc + nrow) + (size_t)kvh * a.max_s;

    constexpr int MERGE = (4 * GQ * HD + 8 * GQ) * 4;
    __shared__ __attribute__((aligned(16))) char smem[MERGE];
    __shared__ __attribute__((aligned(16))) uint32_t sidx[SPR_MAXSEL];   // the key list, padded with row 0
    __shared__ __attribute__((aligned(16))) float sks[4][2][32];   // per wave: k scales, v scales
    // a step's K rows, gathered whole (8 lanes a 128-byte row, 8 keys a load: each cache line once,
    // where the MFMA's A layout would touch each twice, 64 bytes at a time), in a per-wave tile:
    // 16-byte piece p of key j at slot p ^ ((j >> 1) & 7), so that the A-layout reads (16 lanes,
    // 16 keys, one piece) fall in distinct bank groups
    __shared__ __attribute__((aligned(16))) u4_t kt[4][32][8];
    // V rows the same way, in 32-bit words (lane (n, g) reads its 8 bytes of a key as two of them;
    // read as one 8-byte vector over a narrower type, the compiler has taken one word for both)
    __shared__ __attribute__((aligned(16))) uint32_t vt[4][32][32];

    // the key list: every load issued before the first store (rows clamped in range)
    const uint32_t* rows = sel ? a.idx + (size_t)r * a.idx_row_stride + (size_t)kvh * a.idx_kv_stride : nullptr;
    constexpr int LP = (SPR_MAXSEL + 255) / 256;
    int lr[LP];
#pragma unroll
    for (int i = 0; i < LP; i++) {
        const int p = tid + 256 * i;
        lr[i] = p < nk ? (rows ? (int)rows[j0 + p] : j0 + p) : 0;   // past nk: row 0 (masked by position)
    }

    // q^T as the B operand: column n < GQ hi of head n, column GQ + n lo; lane (n, g), MFMA h:
    // dims 64h + 16g .. + 15 (the K slice's dims)
    i4_t qb[2];
    float qsc;
    {
        const int hn = n % GQ;
        const bool live = n < 2 * GQ, is_lo = n >= GQ;
        const uint16_t* qr = a.q + (size_t)r * a.q_row_stride + (size_t)(kvh * GQ + hn) * HD + 16 * g;
        u4_t qv[4];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int u = 0; u < 2; u++) qv[2 * h + u] = ld16(qr + 64 * h + 8 * u);
        const int npad = (nk + 31) & ~31;   // whole 32-key steps
#pragma unroll
        for (int i = 0; i < LP; i++)
            if (tid + 256 * i < npad) sidx[tid + 256 * i] = (uint32_t)min(max(lr[i], 0), a.max_s - 1);
        float qf[32];
        const bool qbf = a.q_bf16;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t x = qv[j][i];
                const float bl = __uint_as_float(x << 16), bh = __uint_as_float(x & 0xFFFF0000u);
                const float hl = h2f((uint16_t)(x & 0xFFFF)), hh = h2f((uint16_t)(x >> 16));
                qf[8 * j + 2 * i] = qbf ? bl : hl;
                qf[8 * j + 2 * i + 1] = qbf ? bh : hh;
            }
        float am = 0.0f;
#pragma unroll
        for (int d = 0; d < 32; d++) am = fmaxf(am, fabsf(qf[d]));
        am = max_rows(am);
        const float inv = am > 0.0f ? QFIX / am : 0.0f;
        // step x 1/sqrt(128) x log2(e), applied in the exponent's fma (> 0, so -inf scores stay -inf)
        qsc = fmaxf(am / QFIX * (0.08838834764831845f * 1.4426950408889634f), 1e-30f);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t word = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int qi = (int)rintf(qf[16 * h + 4 * k + e] * inv);
                    const int hi = (qi + 128) >> 8, lo = qi - hi * 256;
                    const int byte = live ? (is_lo ? lo : hi) : 0;
                    word |= (uint32_t)(byte & 0xFF) << (8 * e);
                }
                qb[h][k] = (int)word;
            }
    }
    __syncthreads();   // the key list

    float m = NEG_INF, l = 0.0f;
    f4_t O[8];
#pragma unroll
    for (int u = 0; u < 8; u++) O[u] = (f4_t){0, 0, 0, 0};
    // V enters the P·V products as the fp16 subnormal (128 + v) 2^-24 (its bytes with 0x80
    // flipped, as whole raw words, under a zero high byte: one v_perm a dword of the operand and
    // no other VALU); OB accumulates 128 · 2^-24 · Σ w with one more MFMA against a constant
    // operand, and O - OB is scaled by 2^24 at the end. MFMA takes fp16 subnormals as they are;
    // the products are exact and the fp32 sums carry the bias' rounding at ~2^-24 of 128 · Σ w.
    // (Against the normal fp16 1152 + v, which needs an XOR a dword of the operand: 16 fewer VALU
    // a step, the C5 sparse layer unchanged at 0.411-0.413 ms, a 9x smaller bias.)
    f4_t OB = {0, 0, 0, 0};
    const h8_t c128 = __builtin_bit_cast(h8_t, (u4_t){0x00800080u, 0x00800080u, 0x00800080u, 0x00800080u});

    // one 32-key step's raw bytes: K[2t + h] = key 16t + n, dims 64h + 16g ..; V[e] = key
    // 16(e / 4) + 4g + e % 4, dims 8n .. 8n + 7; lanes < 32 hold key t0 + lane's two scales
    struct Raw { u4_t k[4]; u4_t v[4]; uint32_t s; };   // k, v: rows 8i + lane / 8, 16 bytes a lane
    // rows as 32-bit byte offsets from the kv head's base (< 2^31: max_s * 128 a head)
    auto gather_k = [&](int t0, Raw& R) {   // k[i]: key 8i + lane / 8, bytes 16 (lane % 8) .. + 15
#pragma unroll
        for (int i = 0; i < 4; i++)
            R.k[i] = ld16(kb + sidx[t0 + 8 * i + (lane >> 3)] * (uint32_t)HD + 16 * (lane & 7));
        const uint32_t row = sidx[t0 + (lane & 31)];
        R.s = lane < 32 ? ksc[row] : vsc[row];
    };
    auto gather_v = [&](int t0, Raw& R) {   // v[i]: key 8i + lane / 8, bytes 16 (lane % 8) .. + 15
#pragma unroll
        for (int i = 0; i < 4; i++)
            R.v[i] = ld16(vb + sidx[t0 + 8 * i + (lane >> 3)] * (uint32_t)HD + 16 * (lane & 7));
    };
    Raw A;
    if (32 * w < nk) { gather_k(32 * w, A); gather_v(32 * w, A); }
    for (int t0 = 32 * w; t0 < nk; t0 += 128) {
        // scales to LDS: k scale of key j at [0][j], v scale (x 64) at [1][j]
        sks[w][lane >> 5][lane & 31] = lane < 32 ? h2f((uint16_t)A.s) : 64.0f * h2f((uint16_t)A.s);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = 8 * i + (lane >> 3);
            kt[w][j][(lane & 7) ^ ((j >> 1) & 7)] = A.k[i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = 8 * i + (lane >> 3), sl = (lane & 7) ^ ((j >> 1) & 7);
#pragma unroll
            for (int q = 0; q < 4; q++) vt[w][j][4 * sl + q] = A.v[i][q];
        }
        // the registers are free again: the next step's K and V are requested now, a step ahead
        if (t0 + 128 < nk) {
            gather_k(t0 + 128, A);
            gather_v(t0 + 128, A);
        }
        wave_lds_sync();
        i4_t st[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            // A operands: key 16t + n, dims 64h + 16g .. + 15
            u4_t ka[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int j = 16 * t + n;
                ka[h] = kt[w][j][(4 * h + g) ^ ((j >> 1) & 7)];
            }
            st[t] = (i4_t){0, 0, 0, 0};
            st[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, ka[0]), qb[0], st[t], 0, 0, 0);
            st[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4_t, ka[1]), qb[1], st[t], 0, 0, 0);
        }
        const f4_t kq0 = *(const f4_t*)(&sks[w][0][4 * g]), kq1 = *(const f4_t*)(&sks[w][0][16 + 4 * g]);
        const f4_t vq0 = *(const f4_t*)(&sks[w][1][4 * g]), vq1 = *(const f4_t*)(&sks[w][1][16 + 4 * g]);
        float x[8];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // lo from lane n + GQ (DPP row_shl: lane i reads lane i + GQ of its row; only the
                // lanes n < GQ use x)
                const int lo = (int)dpp_u32<0x100 + GQ>((uint32_t)st[t][i]);
                const float kq = t == 0 ? kq0[i] : kq1[i];
                x[4 * t + i] = (float)(st[t][i] * 256 + lo) * kq;
            }
        if (t0 + 32 > nk) {   // uniform: the list's last, partial step
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (t0 + 16 * (e >> 2) + 4 * g + (e & 3) >= nk) x[e] = NEG_INF;
        }
        float mt = NEG_INF;
#pragma unroll
        for (int e = 0; e < 8; e++) mt = fmaxf(mt, x[e]);
        mt = max_rows(mt);
        const float mn = fmaxf(m, mt * qsc);
        if (__any(n < GQ && mn > m)) {
            if (__any(n < GQ && m != NEG_INF)) {
                const float corr = m == NEG_INF ? 0.0f : exp2f(m - mn);
                l *= corr;
                float cf[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float c0 = readlane(corr, i);
                    if constexpr (GQ == 8) cf[i] = g == 1 ? readlane(corr, 4 + i) : c0;
                    else cf[i] = c0;
                }
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 4; i++) O[u][i] *= cf[i];
#pragma unroll
                for (int i = 0; i < 4; i++) OB[i] *= cf[i];
            }
            m = mn;
        }
        h8_t wa;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], qsc, -m));   // x = -inf -> 0
            l += p;
            wa[e] = (_Float16)(p * (e < 4 ? vq0[e & 3] : vq1[e & 3]));
        }
        // B operand of MFMA u: halves (V[e][8n + u], V[e + 1][8n + u]) a dword: byte u of keys e
        // and e + 1 (0x80 flipped) into bytes 0 and 2, zero bytes 1 and 3: the fp16 subnormal pair
        // (128 + x) 2^-24
        OB = mfma16(wa, c128, OB);
        u2_t va[8];   // keys 4g + e and 16 + 4g + e - 4, dims 8n .. 8n + 7, with 0x80 flipped
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int j = 16 * (e >> 2) + 4 * g + (e & 3), sl = (n >> 1) ^ ((j >> 1) & 7);
            va[e] = (u2_t){vt[w][j][4 * sl + 2 * (n & 1)], vt[w][j][4 * sl + 2 * (n & 1) + 1]} ^
                    (u2_t){0x80808080u, 0x80808080u};
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            u4_t b;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const uint32_t sel = (u & 3) | (((u & 3) + 4) << 16) | 0x0C000C00u;
                b[e / 2] = __builtin_amdgcn_perm(va[e + 1][u >> 2], va[e][u >> 2], sel);
            }
            O[u] = mfma16(wa, __builtin_bit_cast(h8_t, b), O[u]);
        }
        wave_lds_sync();   // the next step's scale stores come after every lane's reads
    }

#pragma unroll
    for (int u = 0; u < 8; u++)
#pragma unroll
        for (int i = 0; i < 4; i++) O[u][i] = (O[u][i] - OB[i]) * 16777216.0f;   // the V bias and the 2^-24

    // ---- merge the 4 waves (LDS), then the row's output or this chunk's partial
    float (*om)[GQ][HD] = (float (*)[GQ][HD])smem;
    float (*mm)[GQ] = (float (*)[GQ])(smem + 4 * GQ * HD * 4);
    float (*ll)[GQ] = (float (*)[GQ])(smem + (4 * GQ * HD + 4 * GQ) * 4);
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
    const int hq = kvh * GQ + oh;
    if (a.C > 1) {   // partial: O x 64 unnormalised, m, l (decode_merge_kernel with oscale 64)
        float* pp = a.part + ((size_t)c * a.n_q + hq) * SPS;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            float s = 0.0f;
#pragma unroll
            for (int ww = 0; ww < 4; ww++) s += om[ww][oh][od + e] * f[ww];
            pp[od + e] = s;
        }
        if (od == 0) { pp[HD] = M; pp[HD + 1] = L; }
        return;
    }
    const float inv = 1.0f / (64.0f * L);
    uint16_t* orow = a.o + (size_t)r * a.o_row_stride + (size_t)hq * HD + od;
#pragma unroll
    for (int e = 0; e < PER; e++) {
        float s = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) s += om[ww][oh][od + e] * f[ww];
        orow[e] = a.o_bf16 ? f2bf(s * inv) : f2h(s * inv);
    }
}

int launch_sparse_rows8(const SparseRows8Args& a, hipStream_t st) {
    if (a.CH > SPR_MAXSEL || a.CH <= 0 || a.C <= 0) return EMBLA_ERR_UNSUPPORTED;   // a chunk's keys fit the list
    if (a.C > 1 && (a.R != 1 || !a.part)) return EMBLA_ERR_INVALID;
    const dim3 grid(a.C, a.n_kv, a.R), block(256);
    const int gq = a.n_q / a.n_kv;
#define EMBLA_SR(GQ, TL, S32) hipLaunchKernelGGL((sparse_rows8_kernel<GQ, TL, S32>), grid, block, 0, st, a)
    static const bool staged = getenv("EMBLA_SPR_STAGE") != nullptr;   // the LDS-staged variant (tuning)
    if (gq == 4 && !a.tiles && !a.scale32 && !staged)
        hipLaunchKernelGGL((sparse_rows8_rm_kernel<4>), grid, block, 0, st, a);
    else if (gq == 8 && !a.tiles && !a.scale32 && !staged)
        hipLaunchKernelGGL((sparse_rows8_rm_kernel<8>), grid, block, 0, st, a);
    else if (gq == 4 && !a.tiles && !a.scale32) EMBLA_SR(4, false, false);
    else if (gq == 8 && !a.tiles && !a.scale32) EMBLA_SR(8, false, false);
    else if (gq == 8 && a.tiles && a.scale32) EMBLA_SR(8, true, true);
    else if (gq == 4 && a.tiles && !a.scale32) EMBLA_SR(4, true, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_SR
    if (a.C > 1) return launch_decode_merge(a.part, a.o, a.C, a.n_q, false, a.o_bf16, 64.0f, st);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
