// Sparse-layer batched prefill: per query row, the ReLU² index scores of every earlier key, the
// exact top-k of them (+ the latest `recent` positions), then softmax attention over those rows.
//
// The selection must be bit-exact with the scorer's fp32 spec (index_scores_kernel, select.hip:
// 8 fma chains of 8 dims, a fixed combine tree, r = max(dot, 0), s = fma(w_h, r·r, s)) and with
// select_keys' order (Sources/EmblaMetal/Kernels/attention.metal:647-744). For a 2048-row chunk
// the scores are 2048 × ~32K × 4 heads × 64 dims (33 GFLOP), matrix-core work, but an MFMA's
// internal summation order is not the spec's. MI355X design, in three kernels:
//
//  1. index_mfma_kernel: approximate scores on v_mfma_f32_32x32x16_f16 (8 rows × 4 index heads as
//     an A tile, 32 keys as B; fp16 products are exact, the fp32 sums differ from the spec's by a
//     bounded amount), stored as the top 16 bits of their order bits (134 MB for C5 in place of
//     268), plus each key chunk's largest key norm for the error bound.
//  2. select_band_kernel, a workgroup a row: a 2-pass radix select on the 16-bit keys gives the
//     k-th largest truncated key T. With ε bounding |approximate − spec| for every key of the row
//     (from the row's query norms, weights and the key norm maximum), the spec's k-th largest
//     score E lies in [lo(T) − ε, hi(T) + ε]; keys whose 16-bit interval lies entirely above
//     hi(T) + 2ε are selected, entirely below lo(T) − 2ε rejected, and only the band between is
//     rescored with the spec itself (a handful of keys a row) and ranked exactly. Every decision
//     is therefore the spec's. The ordered compaction then writes the indices in select_keys'
//     order.
//  3. sparse_rows8_kernel (decode_sparse.hip): gathered attention over a row-major int8 cache.
#include "common.hpp"
#include "embla_internal.hpp"

#pragma clang fp contract(off)

namespace embla {

__device__ __forceinline__ uint32_t ob32(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ob_to_float(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ 1. approximate scores (MFMA)
/// Workgroup (64-row block rb, key chunk ch), 4 waves; wave w takes rows 64 rb + 16 w .. + 15 as
/// two A tiles (8 rows × 4 index heads each) and sweeps every key of the chunk 32 at a time, so a
/// key fragment feeds two MFMAs and the workgroup's waves read the same keys (L1 hits after the
/// first). A tile: A row R = 4ρ + h (row ρ, index head h), lane l: R = l % 32, dims 16 s + 8 (l / 32)
/// .. + 7 of k-step s. B: lane l: key l % 32, the same dims. D lane (key l % 32, half hh = l / 32)
/// item e: A row 8 (e / 4) + 4 hh + e % 4, i.e. row ρ = 2 (e / 4) + hh, head e % 4: the 4 heads of
/// a (row, key) score sit in one lane.
__global__ __launch_bounds__(256) void index_mfma_kernel(IndexMfmaArgs a) {
    const int rb = blockIdx.x, ch = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane & 31, hh = lane >> 5;
    const int r0 = 64 * rb + 16 * w;   // the wave's first row
    h8v_t qa[2][4];
    float wq[2][4][4];
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        const int R = lane & 31, row = min(r0 + 8 * rt + (R >> 2), a.T - 1), h = R & 3;
        const uint16_t* qr = a.qi + ((size_t)row * 4 + h) * 64;
#pragma unroll
        for (int s = 0; s < 4; s++) qa[rt][s] = __builtin_bit_cast(h8v_t, ld16(qr + 16 * s + 8 * hh));
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int rw = min(r0 + 8 * rt + 2 * b + hh, a.T - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) wq[rt][b][i] = a.w[rw * 4 + i];
        }
    }
    const int k0 = ch * a.kchunk, k1 = min(a.ld, k0 + a.kchunk);
    const bool norms = rb == 0 && w == 0;   // one wave a chunk takes the key norms
    float nmax = 0.0f;
    for (int kb = k0; kb < k1; kb += 32) {
        const int key = kb + c;
        u4_t kr[4];
#pragma unroll
        for (int s = 0; s < 4; s++) kr[s] = key < a.nk ? ld16(a.ki + (size_t)key * 64 + 16 * s + 8 * hh) : (u4_t){0, 0, 0, 0};
        f16_t d[2] = {};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
                d[rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa[rt][s], __builtin_bit_cast(h8v_t, kr[s]), d[rt], 0, 0, 0);
        if (norms) {   // this key's squared norm (half the dims a lane), for the chunk maximum
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float x0 = h2f(kr[s][i] & 0xFFFF), x1 = h2f(kr[s][i] >> 16);
                    ss = __builtin_fmaf(x0, x0, ss);
                    ss = __builtin_fmaf(x1, x1, ss);
                }
            ss += shfl_xor(ss, 32);
            nmax = fmaxf(nmax, ss);
        }
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                float sc = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float r = fmaxf(d[rt][4 * b + i], 0.0f);
                    sc = __builtin_fmaf(wq[rt][b][i], r * r, sc);
                }
                const int row = r0 + 8 * rt + 2 * b + hh;
                if (row < a.T) a.keys[(size_t)row * a.ld + key] = (uint16_t)(ob32(sc) >> 16);
            }
    }
    if (norms) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) nmax = fmaxf(nmax, shfl_xor(nmax, o));
        // the fp32 sum of 64 exact squares is within 64 units of 2^-24 of the true sum
        if (lane == 0) a.kmax[ch] = sqrtf(nmax * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-16f);
    }
}

int launch_index_mfma(const IndexMfmaArgs& a, hipStream_t st) {
    const dim3 grid((a.T + 63) / 64, (a.ld + a.kchunk - 1) / a.kchunk);
    hipLaunchKernelGGL(index_mfma_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// ------------------------------------------------------------------ 2. exact selection by band
constexpr int BS_T = 512;               // threads (8 waves)
constexpr int BS_MAXN = 32768;          // candidate keys a row
constexpr int BS_LB = 1024;             // band capacity (else the band is ranked from the keys)
constexpr int BS_HC = 4, BS_HS = 257;   // 256-bin histogram copies, stride
constexpr uint16_t K_GT = 0xFFFF, K_EQ = 0xFFFE;   // class marks (no finite score truncates to them)

struct BandSmem {
    uint16_t keys[BS_MAXN];
    uint32_t hist[BS_HC * BS_HS];
    uint32_t bj[BS_LB];      // band key indices; the staged output at the end
    uint32_t bx[BS_LB];      // their spec scores' order bits
    uint32_t tab[2][64];     // compaction: counts, then offsets, a (round, wave)
    float qf[4][64];
    float wq[4];
    uint32_t buf[9];
    uint32_t sel[2];
    uint32_t cnt[2];         // band size, keys surely above
    uint32_t kin, kout;
};

/// The spec score of key j (index_scores_kernel's order), the row's queries and weights in LDS:
/// chain k of head h is dims 8k .. 8k + 7, one 16-byte load of the key.
__device__ __noinline__ float spec_score(const BandSmem& sm, const uint16_t* __restrict__ ki, int j) {
    float cc[4][8];
    const u4_t* kr = (const u4_t*)(ki + (size_t)j * 64);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const u4_t v = kr[k];
        float kf[8];
#pragma unroll
        for (int i = 0; i < 4; i++) { kf[2 * i] = h2f(v[i] & 0xFFFF); kf[2 * i + 1] = h2f(v[i] >> 16); }
#pragma unroll
        for (int h = 0; h < 4; h++) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) acc = __builtin_fmaf(sm.qf[h][8 * k + d], kf[d], acc);
            cc[h][k] = acc;
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; h++) {
        const float dot = ((cc[h][0] + cc[h][1]) + (cc[h][2] + cc[h][3])) + ((cc[h][4] + cc[h][5]) + (cc[h][6] + cc[h][7]));
        const float r = fmaxf(dot, 0.0f);
        s = __builtin_fmaf(sm.wq[h], r * r, s);
    }
    return s;
}

/// Digit (of 256, histogram copies `nc` at stride BS_HS) holding the k-th largest: sel = {digit,
/// keys in digits above}. Wave 0, 4 digits a lane from the top.
__device__ void bs_pick(BandSmem& sm, int nc, uint32_t k) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        uint32_t cc[4], s = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int d = 255 - (4 * lane + i);
            uint32_t t = 0;
            for (int c = 0; c < nc; c++) t += sm.hist[c * BS_HS + d];
            cc[i] = t;
            s += t;
        }
        uint32_t above = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t x = __shfl_up(above, o, 64);
            if (lane >= o) above += x;
        }
        above -= s;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (above < k && above + cc[i] >= k) { sm.sel[0] = 255u - (4 * lane + i); sm.sel[1] = above; }
            above += cc[i];
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(BS_T) void select_band_kernel(BandSelectArgs a) {
    __shared__ BandSmem sm;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int S = a.p0 + t + 1;
    if (S <= a.topk + a.recent) return;   // a short row attends every key: no selection
    const int n = S - a.recent;
    uint32_t* out = a.idx + (size_t)t * a.idx_stride;
    const uint16_t* kr = a.keys + (size_t)t * a.ld;
    const int rounds = (n + 8 * BS_T - 1) / (8 * BS_T);   // 4096 keys a round, 8 a lane

    for (int q = tid; q < BS_HC * BS_HS; q += BS_T) sm.hist[q] = 0;
    if (tid < 2) sm.cnt[tid] = 0;
    if (tid < 256) sm.qf[tid >> 6][tid & 63] = h2f(a.qi[(size_t)t * 256 + tid]);
    if (tid < 4) sm.wq[tid] = a.w[t * 4 + tid];
    __syncthreads();
    // ---- load (every load in flight), top-byte histogram; keys past n are 0 and not counted
    {
        u4_t v[BS_MAXN / (8 * BS_T)];
#pragma unroll
        for (int r = 0; r < BS_MAXN / (8 * BS_T); r++) {
            const int j = 8 * tid + 8 * BS_T * r;
            v[r] = j < n ? ld16(kr + j) : (u4_t){0, 0, 0, 0};
        }
        uint32_t* hc = sm.hist + (lane & (BS_HC - 1)) * BS_HS;
#pragma unroll
        for (int r = 0; r < BS_MAXN / (8 * BS_T); r++) {
            const int j = 8 * tid + 8 * BS_T * r;
            if (r < rounds) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t key = (v[r][e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                    if (j + e < n) atomicAdd(&hc[key >> 8], 1u);
                    else v[r][e >> 1] &= ~(0xFFFFu << (16 * (e & 1)));
                }
                *(u4_t*)(sm.keys + j) = v[r];
            }
        }
    }
    __syncthreads();
    uint32_t k = (uint32_t)a.topk;
    bs_pick(sm, BS_HC, k);
    const uint32_t d1 = sm.sel[0];
    k -= sm.sel[1];
    __syncthreads();
    for (int q = tid; q < BS_HS; q += BS_T) sm.hist[q] = 0;
    __syncthreads();
    for (int r = 0; r < rounds; r++) {
        const int j = 8 * tid + 8 * BS_T * r;
        const u4_t v = *(const u4_t*)(sm.keys + j);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t key = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
            if ((key >> 8) == d1 && j + e < n) atomicAdd(&sm.hist[key & 255], 1u);
        }
    }
    __syncthreads();
    bs_pick(sm, 1, k);
    const uint32_t T16 = (d1 << 8) | sm.sel[0];

    // ---- the band: ε bounds |approximate − spec| for every key of this row
    if (tid == 0) {
        float km = 0.0f;
        for (int c = 0; c < a.nchunks; c++) km = fmaxf(km, a.kmax[c]);
        double eps = 0.0, mag = 0.0;
        for (int h = 0; h < 4; h++) {
            double qn = 0.0;
            for (int d = 0; d < 64; d++) qn += (double)sm.qf[h][d] * sm.qf[h][d];
            const double R = sqrt(qn) * km * (1.0 + 1e-6);   // |q·k| <= |q||k|
            const double del = R * 0x1p-16;                  // both fp32 sums of 64 exact products
            const double wa = fabs((double)sm.wq[h]);
            eps += wa * del * (2.0 * R + del);
            mag += wa * (R + del) * (R + del);
        }
        eps += mag * 0x1p-20;   // the fp32 squares, products and the sum over heads, both sides
        eps = eps * (1.0 + 0x1p-10) + 1e-30;
        const double lo = ob_to_float(T16 << 16), hi = ob_to_float((T16 << 16) | 0xFFFFu);
        const float fin = __double2float_rd(hi + 2.0 * eps);    // largest float <= hi(T) + 2ε
        const float fout = __double2float_ru(lo - 2.0 * eps);   // smallest float >= lo(T) - 2ε
        sm.kin = (ob32(fin) >> 16) + 1;   // keys >= kin: interval wholly above hi(T) + 2ε
        sm.kout = ob32(fout) >> 16;       // keys < kout: interval wholly below lo(T) - 2ε
    }
    __syncthreads();
    const uint32_t kin = sm.kin, kout = sm.kout;
    // ---- classify: count the keys surely above, list the band (one atomic a wave)
    for (int r = 0; r < rounds; r++) {
        const int j = 8 * tid + 8 * BS_T * r;
        const u4_t v = *(const u4_t*)(sm.keys + j);
        uint32_t nb = 0, na = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t key = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
            const bool real = j + e < n;
            na += real && key >= kin;
            nb += real && key >= kout && key < kin;
        }
        uint32_t incl = nb;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t x = __shfl_up(incl, o, 64);
            if (lane >= o) incl += x;
        }
        uint32_t sa = na;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sa += __shfl_xor(sa, o, 64);
        uint32_t base = 0;
        if (lane == 63) base = atomicAdd(&sm.cnt[0], incl);
        if (lane == 0) {   // the compaction's counts: sure-above keys now, the band's added later
            sm.tab[0][8 * r + w] = sa;
            sm.tab[1][8 * r + w] = 0;
            if (sa) atomicAdd(&sm.cnt[1], sa);
        }
        base = __shfl(base, 63, 64);
        if (nb) {
            uint32_t p = base + incl - nb;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t key = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                if (j + e < n && key >= kout && key < kin) {
                    if (p < BS_LB) sm.bj[p] = (uint32_t)(j + e);
                    p++;
                }
            }
        }
    }
    __syncthreads();
    const uint32_t nband = sm.cnt[0];
    k = (uint32_t)a.topk - sm.cnt[1];   // rank of the spec's k-th largest among the band
    const bool listed = nband <= BS_LB;
    if (listed)
        for (uint32_t q = tid; q < nband; q += BS_T) sm.bx[q] = ob32(spec_score(sm, a.ki, sm.bj[q]));
    __syncthreads();
    // ---- exact rank within the band: four 8-bit passes over the band's spec scores
    uint32_t pre = 0, msk = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int q = tid; q < BS_HS; q += BS_T) sm.hist[q] = 0;
        __syncthreads();
        if (listed) {
            for (uint32_t q = tid; q < nband; q += BS_T) {
                const uint32_t x = sm.bx[q];
                if ((x & msk) == pre) atomicAdd(&sm.hist[(x >> shift) & 255u], 1u);
            }
        } else {   // a band too large to list: rescore it from the keys on every pass
            for (int j = tid; j < n; j += BS_T) {
                const uint32_t key = sm.keys[j];
                if (key >= kout && key < kin) {
                    const uint32_t x = ob32(spec_score(sm, a.ki, j));
                    if ((x & msk) == pre) atomicAdd(&sm.hist[(x >> shift) & 255u], 1u);
                }
            }
        }
        __syncthreads();
        bs_pick(sm, 1, k);
        pre |= sm.sel[0] << shift;
        msk |= 255u << shift;
        k -= sm.sel[1];
        __syncthreads();
    }
    const uint32_t E = pre;   // the spec's k-th largest score; k = ties to take, first by index
    // ---- mark the band keys with their class
    // a band key's class into its slot and into the compaction count of its (round, wave): key j is
    // in round j / 4096, wave (j % 4096) / 512
    auto mark = [&](int j, uint32_t x) {
        const uint16_t cl = x > E ? K_GT : (x == E ? K_EQ : 0);
        sm.keys[j] = cl;
        if (cl) atomicAdd(&sm.tab[cl == K_GT ? 0 : 1][8 * (j >> 12) + ((j & 4095) >> 9)], 1u);
    };
    if (listed) {
        for (uint32_t q = tid; q < nband; q += BS_T) mark((int)sm.bj[q], sm.bx[q]);
    } else {
        for (int j = tid; j < n; j += BS_T) {
            const uint32_t key = sm.keys[j];
            if (key >= kout && key < kin) mark(j, ob32(spec_score(sm, a.ki, j)));
        }
    }
    __syncthreads();
    // ---- ordered compaction: above (sure or marked), then the first k equal, by index. Round r,
    // wave w holds keys 4096 r + 512 w .. + 511: table entry 8 r + w, counted above.
    auto cls = [&](uint32_t key, bool real, bool& g, bool& e) {
        g = real && (key == K_GT || (key >= kin && key < K_EQ));
        e = real && key == K_EQ;
    };
    if (w < 2) {
        uint32_t* tb = sm.tab[w];
        const int m = 8 * rounds;
        const uint32_t v = lane < m ? tb[lane] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t x = __shfl_up(incl, o, 64);
            if (lane >= o) incl += x;
        }
        if (lane < m) tb[lane] = incl - v;
        if (lane == 63) sm.sel[w] = incl;
    }
    __syncthreads();
    const uint32_t ngt = sm.sel[0];
    uint32_t* sout = a.topk <= BS_LB ? sm.bj : out;
    for (int r = 0; r < rounds; r++) {
        const int j = 8 * tid + 8 * BS_T * r;
        const u4_t v = *(const u4_t*)(sm.keys + j);
        bool g[8], q[8];
        uint32_t cg = 0, ce = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            cls((v[e >> 1] >> (16 * (e & 1))) & 0xFFFF, j + e < n, g[e], q[e]);
            cg += g[e];
            ce += q[e];
        }
        uint32_t ig = cg, ie = ce;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t xg = __shfl_up(ig, o, 64), xe = __shfl_up(ie, o, 64);
            if (lane >= o) { ig += xg; ie += xe; }
        }
        uint32_t pg = sm.tab[0][8 * r + w] + ig - cg, pe = sm.tab[1][8 * r + w] + ie - ce;
        if (cg | ce) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if (g[e]) {
                    if (pg < (uint32_t)a.topk) sout[pg] = (uint32_t)(j + e);
                    pg++;
                }
                if (q[e]) {
                    if (pe < k && ngt + pe < (uint32_t)a.topk) sout[ngt + pe] = (uint32_t)(j + e);
                    pe++;
                }
            }
        }
    }
    __syncthreads();
    if (sout != out)
        for (int j = tid; j < a.topk; j += BS_T) out[j] = sout[j];
    for (int j = tid; j < a.recent; j += BS_T) out[a.topk + j] = (uint32_t)(n + j);
}

int launch_select_band(const BandSelectArgs& a, hipStream_t st) {
    if (a.p0 + a.T - a.recent > BS_MAXN) return EMBLA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(select_band_kernel, dim3(a.T), dim3(BS_T), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
