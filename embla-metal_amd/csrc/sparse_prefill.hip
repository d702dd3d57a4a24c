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
//     order. A band too large to list (scores massed at the k-th value) is left to
//     band_overflow_kernel, which scores it once into LDS and ranks it there.
//  3. sparse_rows8_rm_kernel (decode_sparse.hip): gathered attention over a row-major int8 cache.
#include "common.hpp"
#include "embla_internal.hpp"

#pragma clang fp contract(off)

namespace embla {

__device__ __forceinline__ uint32_t ob32(float f) {
    // negative: every bit flipped; otherwise the sign bit set (an arithmetic shift, an or, a xor)
    const uint32_t u = __float_as_uint(f);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__device__ __forceinline__ float ob_to_float(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

typedef _Float16 h8v_t __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ 1. approximate scores (MFMA)
/// Workgroup (64-row block rb, key chunk ch), 4 waves; wave w takes rows 64 rb + 16 w .. + 15 as
/// two A tiles (8 rows × 4 index heads each) and sweeps every key of the chunk 32 at a time, so a
/// key fragment feeds two MFMAs; the workgroup's waves share each block's keys through an LDS
/// tile that they load together. A tile: A row R = 4ρ + h (row ρ, index head h), lane l: R = l % 32, dims 16 s + 8 (l / 32)
/// .. + 7 of k-step s. B: lane l: key l % 32, the same dims. D lane (key l % 32, half hh = l / 32)
/// item e: A row 8 (e / 4) + 4 hh + e % 4, i.e. row ρ = 2 (e / 4) + hh, head e % 4: the 4 heads of
/// a (row, key) score sit in one lane.
// 8-row MFMA row tiles a wave (8 rows x 4 heads each): 16 rows a wave. What bounded this kernel
// was the vector memory unit's address work (busy 61% of its cycles) on the key loads: each wave
// loaded its keys in the B layout, 16 bytes of a 128-byte row a lane, every row four times; loaded
// whole into the shared tile, each row is requested once a workgroup (90 -> 68 us a C5 chunk)
constexpr int IXRT = 2;
__global__ __launch_bounds__(256) void index_mfma_kernel(IndexMfmaArgs a) {
    const int rb = blockIdx.x, ch = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane & 31, hh = lane >> 5;
    const int r0 = 32 * IXRT * rb + 8 * IXRT * w;   // the wave's first row
    h8v_t qa[IXRT][4];
    // the 4 head weights of the workgroup's rows, in LDS (in registers, 16 a row tile: 148 against
    // 117 VGPRs, and 88-91 against 81-84 us a C5 chunk)
    __shared__ f4_t wl[32 * IXRT];
    // a block's 32 key rows (128 bytes each) in a workgroup tile, double-buffered: wave w loads
    // rows 8w .. 8w + 7 whole, 8 lanes a row (each cache line once a workgroup, where each wave's
    // B-layout loads touched it four times, 16 bytes at a time), the next block's rows in flight
    // during this block's products; one barrier a block. 16-byte piece p of key j sits at slot
    // p ^ ((j >> 1) & 7), so the B-layout reads (16 lanes, 16 keys, one piece) are conflict-free.
    __shared__ __attribute__((aligned(16))) u4_t kts[2][32][8];
    for (int i = tid; i < 32 * IXRT; i += 256) {
        const int rw = min(32 * IXRT * rb + i, a.T - 1);
        wl[i] = (f4_t){a.w[rw * 4], a.w[rw * 4 + 1], a.w[rw * 4 + 2], a.w[rw * 4 + 3]};
    }
#pragma unroll
    for (int rt = 0; rt < IXRT; rt++) {
        const int R = lane & 31, row = min(r0 + 8 * rt + (R >> 2), a.T - 1), h = R & 3;
        const uint16_t* qr = a.qi + ((size_t)row * 4 + h) * 64;
#pragma unroll
        for (int s = 0; s < 4; s++) qa[rt][s] = __builtin_bit_cast(h8v_t, ld16(qr + 16 * s + 8 * hh));
    }
    __syncthreads();
    const int k0 = ch * a.kchunk, k1 = min(a.ld, k0 + a.kchunk);
    const bool norms = rb == 0 && w == 0;   // one wave a chunk takes the key norms
    float nmax = 0.0f;
    auto load_rows = [&](int kb) {   // wave w's share of block kb: row 8w + lane / 8, piece lane % 8
        const int kj = kb + 8 * w + (lane >> 3);
        return kj < a.nk ? ld16(a.ki + (size_t)kj * 64 + 8 * (lane & 7)) : (u4_t){0, 0, 0, 0};
    };
    u4_t nx = {0, 0, 0, 0};
    if (k0 < k1) nx = load_rows(k0);
    int it = 0;
    for (int kb = k0; kb < k1; kb += 32, it++) {
        const int key = kb + c;
        u4_t kr[4];   // key c, dims 16s + 8hh .. + 7: the B operand of k-step s
        {
            const int j = 8 * w + (lane >> 3);
            kts[it & 1][j][(lane & 7) ^ ((j >> 1) & 7)] = nx;
            __syncthreads();
            if (kb + 32 < k1) nx = load_rows(kb + 32);
#pragma unroll
            for (int s = 0; s < 4; s++) kr[s] = kts[it & 1][c][(2 * s + hh) ^ ((c >> 1) & 7)];
        }
        f16_t d[IXRT] = {};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int rt = 0; rt < IXRT; rt++)
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
            ss = sum_xor32(ss);
            nmax = fmaxf(nmax, ss);
        }
        auto score = [&](int rt, int b) {
            float sc = 0.0f;
            const f4_t wv = wl[8 * IXRT * w + 8 * rt + 2 * b + hh];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float r = vmax2(d[rt][4 * b + i], 0.0f);
                sc = __builtin_fmaf(wv[i], r * r, sc);
            }
            return (uint16_t)(ob32(sc) >> 16);
        };
        // (uniform) every row of the wave exists and sees every key of the block: no per-key tests
        if (r0 + 8 * IXRT <= a.T && kb + 32 <= r0 + a.lim0) {
#pragma unroll
            for (int rt = 0; rt < IXRT; rt++)
#pragma unroll
                for (int b = 0; b < 4; b++) a.keys[(size_t)(r0 + 8 * rt + 2 * b + hh) * a.ld + key] = score(rt, b);
        } else {
#pragma unroll
            for (int rt = 0; rt < IXRT; rt++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int row = r0 + 8 * rt + 2 * b + hh;
                    const uint16_t v = score(rt, b);
                    if (row < a.T) a.keys[(size_t)row * a.ld + key] = key < row + a.lim0 ? v : 0;
                }
        }
    }
    if (norms) {
        nmax = wave_bfly(nmax, [](float x, float y) { return fmaxf(x, y); });
        // the fp32 sum of 64 exact squares is within 64 units of 2^-24 of the true sum
        if (lane == 0) a.kmax[ch] = sqrtf(nmax * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-16f);
    }
}

int launch_index_mfma(const IndexMfmaArgs& a, hipStream_t st) {
    const dim3 grid((a.T + 32 * IXRT - 1) / (32 * IXRT), (a.ld + a.kchunk - 1) / a.kchunk);
    hipLaunchKernelGGL(index_mfma_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// ------------------------------------------------------------------ 2. exact selection by band
constexpr int BS_T = 512;               // threads (8 waves)
constexpr int BS_MAXN = 32768;          // candidate keys a row
constexpr int BS_LB = 1024;             // band capacity (else the band is ranked from the keys)
constexpr int BS_HS = 257;              // band radix histogram (256 bins) stride
constexpr int BS_R = BS_MAXN / (8 * BS_T);   // rounds of 4096 keys, 8 a lane

struct BandSmem {
    uint32_t h1[2][4096];   // first digit (the key's top 12 bits), two copies (by lane parity)
    uint32_t bj[BS_LB];     // band key indices, in no order
    uint32_t bx[BS_LB];     // their spec scores' order bits
    uint32_t hist[BS_HS];
    uint32_t gt[BS_MAXN / 32];   // bitmap of the selected keys above the k-th's score
    uint32_t eq[BS_MAXN / 32];   // bitmap of the band keys whose spec score equals the k-th's
    float qf[4][64];
    float wq[4];
    double eps;
    uint32_t sel[2];
    uint32_t cnt[2];         // band size, keys surely above
    uint32_t wsum[8];        // the output scan's wave totals
    uint32_t kin, kout;
};

/// The spec score of key j (index_scores_kernel's order), the row's queries qf[4][64] and weights
/// wq[4] in LDS: chain k of head h is dims 8k .. 8k + 7, one 16-byte load of the key.
__device__ __forceinline__ float spec_score_q(const float (*qf)[64], const float* wq, const uint16_t* __restrict__ ki,
                                              int j) {
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
            for (int d = 0; d < 8; d++) acc = __builtin_fmaf(qf[h][8 * k + d], kf[d], acc);
            cc[h][k] = acc;
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; h++) {
        const float dot = ((cc[h][0] + cc[h][1]) + (cc[h][2] + cc[h][3])) + ((cc[h][4] + cc[h][5]) + (cc[h][6] + cc[h][7]));
        const float r = fmaxf(dot, 0.0f);
        s = __builtin_fmaf(wq[h], r * r, s);
    }
    return s;
}
__device__ __noinline__ float spec_score(const BandSmem& sm, const uint16_t* __restrict__ ki, int j) {
    return spec_score_q(sm.qf, sm.wq, ki, j);
}

/// Digit (of 256, histogram copies `nc` at stride BS_HS) holding the k-th largest: sel = {digit,
/// keys in digits above}. Wave 0, 4 digits a lane from the top.
template <class Sm>
__device__ void bs_pick(Sm& sm, int nc, uint32_t k) {
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
        above = wave_scan_incl(above);
        above -= s;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (above < k && above + cc[i] >= k) { sm.sel[0] = 255u - (4 * lane + i); sm.sel[1] = above; }
            above += cc[i];
        }
    }
    __syncthreads();
}

/// Bin (of 4096) holding the k-th largest key, from the first-digit counts: sel = {bin, keys in
/// bins above}. Wave 0: each lane sums 64 bins (both copies) from the top; the lane whose bins
/// hold the k-th is found by a scan and a ballot, then its 64 bins go one a lane through a second
/// scan.
__device__ void bs_pick1(BandSmem& sm, uint32_t k) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        const int b0 = 4032 - 64 * lane;   // the lane's bins b0 .. b0 + 63
        uint32_t s = 0;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const u4_t x = *(const u4_t*)(sm.h1[c] + b0 + 4 * i);
                s += (x[0] + x[1]) + (x[2] + x[3]);
            }
        uint32_t above = s;
        above = wave_scan_incl(above);
        above -= s;
        const int L = max(__ffsll((long long)__ballot(above < k && above + s >= k)) - 1, 0);
        const uint32_t base = readlane_u32(above, L);   // L is uniform
        const int d = 4095 - 64 * L - lane;   // bins of lane L, from the top
        const uint32_t c = sm.h1[0][d] + sm.h1[1][d];
        uint32_t incl = c;
        incl = wave_scan_incl(incl);
        if (base + incl - c < k && base + incl >= k) { sm.sel[0] = (uint32_t)d; sm.sel[1] = base + incl - c; }
    }
    __syncthreads();
}

/// The selection in select_keys' order from the bitmaps sm.gt (keys above the k-th's score) and
/// sm.eq (keys equal to it): the keys of gt by index, then the first k of eq by index, then the
/// latest positions n .. n + recent - 1. Thread i holds keys 64 i .. + 63 of each bitmap; a block
/// scan of the counts gives its first slot. BS_T threads.
template <class Sm>
__device__ void bs_emit(Sm& sm, uint32_t k, uint32_t* __restrict__ out, int n, int topk, int recent) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    auto block_scan = [&](uint32_t c, uint32_t& total) -> uint32_t {
        uint32_t incl = c;
        incl = wave_scan_incl(incl);
        if (lane == 63) sm.wsum[w] = incl;
        __syncthreads();
        uint32_t before = 0;
        total = 0;
#pragma unroll
        for (int i = 0; i < BS_T / 64; i++) {
            const uint32_t x = sm.wsum[i];
            before += i < w ? x : 0u;
            total += x;
        }
        __syncthreads();   // wsum is reused by the next scan
        return before + incl - c;
    };
    uint32_t ngt;
    {
        uint32_t g0 = sm.gt[2 * tid], g1 = sm.gt[2 * tid + 1];
        uint32_t p = block_scan(__popc(g0) + __popc(g1), ngt);
        for (; g0; g0 &= g0 - 1) out[p++] = 64u * tid + __ffs(g0) - 1;
        for (; g1; g1 &= g1 - 1) out[p++] = 64u * tid + 32u + __ffs(g1) - 1;
    }
    if (k > 0) {   // ties (k is uniform)
        uint32_t e0 = sm.eq[2 * tid], e1 = sm.eq[2 * tid + 1];
        uint32_t neq;
        uint32_t p = block_scan(__popc(e0) + __popc(e1), neq);
        for (; e0 && p < k; e0 &= e0 - 1) out[ngt + p++] = 64u * tid + __ffs(e0) - 1;
        for (; e1 && p < k; e1 &= e1 - 1) out[ngt + p++] = 64u * tid + 32u + __ffs(e1) - 1;
    }
    for (int j = tid; j < recent; j += BS_T) out[topk + j] = (uint32_t)(n + j);
}

__global__ __launch_bounds__(BS_T) __attribute__((amdgpu_waves_per_eu(6))) void select_band_kernel(BandSelectArgs a) {
    __shared__ BandSmem sm;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int S = a.p0 + t + 1;
    if (S <= a.topk + a.recent) return;   // a short row attends every key: no selection
    const int n = S - a.recent;
    uint32_t* out = a.idx + (size_t)t * a.idx_stride;
    const uint16_t* kr = a.keys + (size_t)t * a.ld;
    // 4096 keys a round, 8 a lane. The index kernel stores 0 for every key past n, and a real
    // score's key is >= 0x8000, so keys past n need no test anywhere below: they fall in bin 0 of
    // the first digit (never the k-th's bin), below kout and below kin.
    const int rounds = (n + 8 * BS_T - 1) / (8 * BS_T);

    for (int q = tid; q < 2 * 4096; q += BS_T) (&sm.h1[0][0])[q] = 0;
    for (int q = tid; q < BS_MAXN / 32; q += BS_T) sm.gt[q] = 0;
    for (int q = tid; q < BS_HS; q += BS_T) sm.hist[q] = 0;
    if (tid < 2) sm.cnt[tid] = 0;
    if (tid < 256) sm.qf[tid >> 6][tid & 63] = h2f(a.qi[(size_t)t * 256 + tid]);
    if (tid < 4) sm.wq[tid] = a.w[t * 4 + tid];
    __syncthreads();
    // ---- the row's keys, held in registers: v[r] = keys 8 tid + 4096 r .. + 7 (every load in
    // flight); first-digit histogram
    u4_t v[BS_R];
#pragma unroll
    for (int r = 0; r < BS_R; r++) {
        const int j = 8 * tid + 8 * BS_T * r;
        v[r] = j < n ? ld16(kr + j) : (u4_t){0, 0, 0, 0};   // j + 8 <= ld: ld, j multiples of 8
    }
    if (w == 1) {
        // ε, while the keys are in flight: it bounds |approximate − spec| for every key of this
        // row, from the row's query norms, weights and the key norm maximum
        float km = 0.0f;
        for (int c = lane; c < a.nchunks; c += 64) km = fmaxf(km, a.kmax[c]);
        km = wave_bfly(km, [](float x, float y) { return fmaxf(x, y); });
        double eps = 0.0, mag = 0.0;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            double qn = (double)sm.qf[h][lane] * sm.qf[h][lane];   // exact products
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) qn += __shfl_xor(qn, o, 64);
            const double R = sqrt(qn) * km * (1.0 + 1e-6);   // |q·k| <= |q||k|
            const double del = R * 0x1p-16;                  // both fp32 sums of 64 exact products
            const double wa = fabs((double)sm.wq[h]);
            eps += wa * del * (2.0 * R + del);
            mag += wa * (R + del) * (R + del);
        }
        eps += mag * 0x1p-20;   // the fp32 squares, products and the sum over heads, both sides
        if (lane == 0) sm.eps = eps * (1.0 + 0x1p-10) + 1e-30;
    }
    {
        uint32_t* hc = sm.h1[lane & 1];
#pragma unroll
        for (int r = 0; r < BS_R; r++) {
            if (r < rounds) {
#pragma unroll
                for (int e = 0; e < 8; e++) atomicAdd(&hc[((v[r][e >> 1] >> (16 * (e & 1))) & 0xFFFF) >> 4], 1u);
            }
        }
    }
    __syncthreads();
    uint32_t k = (uint32_t)a.topk;
    bs_pick1(sm, k);
    const uint32_t d1 = sm.sel[0];
    k -= sm.sel[1];
    // second digit: the low 4 bits of the keys in bin d1
    {
        const uint32_t base = d1 << 4;
#pragma unroll
        for (int r = 0; r < BS_R; r++) {
            if (r < rounds) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t x0 = (v[r][i] & 0xFFFF) - base, x1 = (v[r][i] >> 16) - base;
                    if (x0 < 16) atomicAdd(&sm.hist[x0], 1u);
                    if (x1 < 16) atomicAdd(&sm.hist[x1], 1u);
                }
            }
        }
    }
    __syncthreads();
    bs_pick(sm, 1, k);
    const uint32_t T16 = (d1 << 4) | sm.sel[0];

    // ---- the band: keys within 2ε of T's interval
    if (tid == 0) {
        const double eps = sm.eps;
        const double lo = ob_to_float(T16 << 16), hi = ob_to_float((T16 << 16) | 0xFFFFu);
        const float fin = __double2float_rd(hi + 2.0 * eps);    // largest float <= hi(T) + 2ε
        const float fout = __double2float_ru(lo - 2.0 * eps);   // smallest float >= lo(T) - 2ε
        sm.kin = (ob32(fin) >> 16) + 1;   // keys >= kin: interval wholly above hi(T) + 2ε
        sm.kout = ob32(fout) >> 16;       // keys < kout: interval wholly below lo(T) - 2ε
    }
    __syncthreads();
    const uint32_t kin = sm.kin, kout = sm.kout;
    // ---- classify: the keys surely above into the bitmap (a byte a lane) and their count (by
    // ballots); the band into a list (an LDS atomic a band key, in no order)
#pragma unroll
    for (int r = 0; r < BS_R; r++) {
        if (r < rounds) {
            const int j = 8 * tid + 8 * BS_T * r;
            uint32_t sa = 0, bits = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t key = (v[r][e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                const bool above = key >= kin;
                sa += (uint32_t)__popcll(__ballot(above));
                bits |= (uint32_t)above << e;
                const bool inb = key >= kout && !above;
                const uint64_t bm = __ballot(inb);
                if (bm) {   // one LDS atomic a wave (scores massed at the k-th value put every lane here)
                    uint32_t p0 = 0;
                    if (lane == __ffsll((long long)bm) - 1) p0 = atomicAdd(&sm.cnt[0], (uint32_t)__popcll(bm));
                    p0 = readlane_u32(p0, __ffsll((long long)bm) - 1);   // a uniform lane
                    const uint32_t p = p0 + (uint32_t)__popcll(bm & ((1ull << lane) - 1));
                    if (inb && p < BS_LB) sm.bj[p] = (uint32_t)(j + e);
                }
            }
            ((uint8_t*)sm.gt)[j >> 3] = (uint8_t)bits;
            if (lane == 0 && sa) atomicAdd(&sm.cnt[1], sa);
        }
    }
    __syncthreads();
    const uint32_t nband = sm.cnt[0];
    k = (uint32_t)a.topk - sm.cnt[1];   // rank of the spec's k-th largest among the band
    // a band too large to list goes to band_overflow_kernel, which ranks it from an LDS array of
    // every key's spec score: the row's bounds are its record there (kin = 0: no overflow)
    if (tid == 0) *(uint2*)(a.ovf + 2 * t) = nband <= BS_LB ? make_uint2(0u, 0u) : make_uint2(kin, kout);
    if (nband > BS_LB) return;   // uniform
    for (uint32_t q = tid; q < nband; q += BS_T) sm.bx[q] = ob32(spec_score(sm, a.ki, sm.bj[q]));
    __syncthreads();
    // ---- exact rank within the band: four 8-bit passes over the band's spec scores
    uint32_t pre = 0, msk = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int q = tid; q < BS_HS; q += BS_T) sm.hist[q] = 0;
        __syncthreads();
        for (uint32_t q = tid; q < nband; q += BS_T) {
            const uint32_t x = sm.bx[q];
            if ((x & msk) == pre) atomicAdd(&sm.hist[(x >> shift) & 255u], 1u);
        }
        __syncthreads();
        bs_pick(sm, 1, k);
        pre |= sm.sel[0] << shift;
        msk |= 255u << shift;
        k -= sm.sel[1];
        __syncthreads();
    }
    const uint32_t E = pre;   // the spec's k-th largest score; k = ties to take, first by index
    // ---- band keys above E into the selection bitmap, those equal to E into the tie bitmap
    for (int q = tid; q < BS_MAXN / 32; q += BS_T) sm.eq[q] = 0;
    __syncthreads();
    auto mark = [&](int j, uint32_t x) {
        if (x > E) atomicOr(&sm.gt[j >> 5], 1u << (j & 31));
        else if (x == E) atomicOr(&sm.eq[j >> 5], 1u << (j & 31));
    };
    for (uint32_t q = tid; q < nband; q += BS_T) mark((int)sm.bj[q], sm.bx[q]);
    __syncthreads();
    bs_emit(sm, k, out, n, a.topk, a.recent);
}

// ------------------------------------------------------------------ 2b. bands too large to list
// A row whose band holds more than BS_LB keys (scores massed at the k-th value, such as many exact
// zeros of ReLU²) is ranked here: each band key's spec score is computed once into an LDS array
// indexed by key (128 KB, one workgroup a CU), then the same four 8-bit rank passes and the same
// output as select_band_kernel run over that array. Persistent: workgroup b takes rows b, b +
// gridDim.x, ...; a row without an overflow record costs one 8-byte load.
struct OvfSmem {
    uint32_t xs[BS_MAXN];        // order bits of band key j's spec score (set for band keys only)
    uint32_t bd[BS_MAXN / 32];   // bitmap of the band keys
    uint32_t gt[BS_MAXN / 32];   // bitmap of the selected keys above the k-th's score
    uint32_t eq[BS_MAXN / 32];   // bitmap of the band keys whose spec score equals the k-th's
    uint32_t hist[BS_HS];
    float qf[4][64];
    float wq[4];
    uint32_t sel[2];
    uint32_t above;              // keys surely above (keys >= kin)
    uint32_t wsum[8];
};
constexpr int BO_GRID = 256;   // one workgroup a CU (fewer measured slower when many rows overflow)

constexpr int OV_NK = 2;   // band keys a thread scores at once (1 and 4 measured slower)
static_assert(BS_MAXN / 32 == 2 * BS_T, "two bitmap words a thread");

/// spec_score_q of the NK keys j[], their loads all in flight together. The queries are read from
/// LDS a chunk of 8 dims at a time; the arithmetic is spec_score_q's, operation for operation.
template <int NK>
__device__ __forceinline__ void spec_scores_n(const float (*qf)[64], const float* wq, const uint16_t* __restrict__ ki,
                                              const int (&j)[NK], float (&x)[NK]) {
    u4_t kv[NK][8];
#pragma unroll
    for (int n = 0; n < NK; n++)
#pragma unroll
        for (int k = 0; k < 8; k++) kv[n][k] = ((const u4_t*)(ki + (size_t)j[n] * 64))[k];
    float cc[NK][4][8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        // chunk k - 1's sums are done before chunk k's queries are read, which are read here and
        // not earlier: one chunk of queries in registers (else all 256 are hoisted and spill)
        if (k > 0)
#pragma unroll
            for (int n = 0; n < NK; n++)
#pragma unroll
                for (int h = 0; h < 4; h++) __asm__ volatile("" : : "v"(cc[n][h][k - 1]));
        int z = 0;
        __asm__ volatile("" : "+s"(z) : : "memory");
        float qv[4][8];
#pragma unroll
        for (int h = 0; h < 4; h++)
#pragma unroll
            for (int d = 0; d < 8; d++) qv[h][d] = qf[h][8 * k + d + z];
#pragma unroll
        for (int n = 0; n < NK; n++) {
            float kf[8];
#pragma unroll
            for (int i = 0; i < 4; i++) { kf[2 * i] = h2f(kv[n][k][i] & 0xFFFF); kf[2 * i + 1] = h2f(kv[n][k][i] >> 16); }
#pragma unroll
            for (int h = 0; h < 4; h++) {
                float acc = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) acc = __builtin_fmaf(qv[h][d], kf[d], acc);
                cc[n][h][k] = acc;
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NK; n++) {
        float s = 0.0f;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const float* c = cc[n][h];
            const float dot = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
            const float r = fmaxf(dot, 0.0f);
            s = __builtin_fmaf(wq[h], r * r, s);
        }
        x[n] = s;
    }
}

__global__ __launch_bounds__(BS_T) void band_overflow_kernel(BandSelectArgs a) {
    __shared__ OvfSmem sm;
    const int tid = threadIdx.x, lane = tid & 63;
    const int G = gridDim.x;
    for (int i0 = 0; (int)blockIdx.x + G * i0 < a.T; i0 += 64) {
      // the records of rows blockIdx.x + G (i0 + lane), read by every wave alike: a mask of the
      // rows that overflowed (select_band_kernel writes no record for a row without selection)
      const int tl = (int)blockIdx.x + G * (i0 + lane);
      const bool ov = tl < a.T && a.p0 + tl + 1 > a.topk + a.recent && a.ovf[2 * tl] != 0;
      for (uint64_t rows = __ballot(ov); rows; rows &= rows - 1) {
        const int t = (int)blockIdx.x + G * (i0 + __ffsll((long long)rows) - 1);
        const int S = a.p0 + t + 1;
        const uint2 rec = *(const uint2*)(a.ovf + 2 * t);
        const uint32_t kin = rec.x, kout = rec.y;
        const int n = S - a.recent;
        uint32_t* out = a.idx + (size_t)t * a.idx_stride;
        const uint16_t* kr = a.keys + (size_t)t * a.ld;
        __syncthreads();   // the previous row is done with sm
        if (tid < 256) sm.qf[tid >> 6][tid & 63] = h2f(a.qi[(size_t)t * 256 + tid]);
        if (tid < 4) sm.wq[tid] = a.w[t * 4 + tid];
        if (tid == 0) sm.above = 0;
        __syncthreads();
        // words tid and tid + BS_T: keys 32 wd .. + 31 (ld is a multiple of 32; the index kernel
        // stored 0, below kout, for keys past n); bit e of a word is key 32 wd + e, as bs_emit
        // reads the bitmaps
        uint32_t nab = 0;
        uint64_t band = 0;
#pragma unroll
        for (int hw = 0; hw < 2; hw++) {
            const int wd = tid + BS_T * hw;
            uint32_t ab = 0, bd = 0;
            if (32 * wd < n) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const u4_t v = ld16(kr + 32 * wd + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const uint32_t key = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                        ab |= (uint32_t)(key >= kin) << (8 * c + e);
                        bd |= (uint32_t)(key >= kout && key < kin) << (8 * c + e);
                    }
                }
            }
            sm.gt[wd] = ab;
            sm.bd[wd] = bd;
            nab += __popc(ab);
            band |= (uint64_t)bd << (32 * hw);
        }
        while (band) {   // the thread's band keys, OV_NK at a time (spare slots repeat the first)
            int jj[OV_NK];
            bool ok[OV_NK];
#pragma unroll
            for (int i = 0; i < OV_NK; i++) {
                ok[i] = band != 0;
                const int e = ok[i] ? __ffsll((long long)band) - 1 : 0;
                const int j = e < 32 ? 32 * tid + e : 32 * (tid + BS_T) + e - 32;
                jj[i] = i == 0 || ok[i] ? j : jj[0];
                band &= band - 1;
            }
            float x[OV_NK];
            spec_scores_n<OV_NK>(sm.qf, sm.wq, a.ki, jj, x);
#pragma unroll
            for (int i = 0; i < OV_NK; i++)
                if (ok[i]) sm.xs[jj[i]] = ob32(x[i]);
        }
        nab = readlane_u32(wave_scan_incl(nab), 63);   // the wave's total
        if (lane == 0 && nab) atomicAdd(&sm.above, nab);
        __syncthreads();
        uint32_t k = (uint32_t)a.topk - sm.above;   // rank of the spec's k-th largest in the band
        const int nw = (n + 31) / 32;
        uint32_t pre = 0, msk = 0;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int q = tid; q < BS_HS; q += BS_T) sm.hist[q] = 0;
            __syncthreads();
            for (int wd = tid; wd < nw; wd += BS_T) {
                uint32_t rd = 0, rc = 0;   // a run of equal digits: one atomic a run
                for (uint32_t b = sm.bd[wd]; b; b &= b - 1) {
                    const uint32_t x = sm.xs[32 * wd + __ffs(b) - 1];
                    if ((x & msk) != pre) continue;
                    const uint32_t d = (x >> shift) & 255u;
                    if (rc && d != rd) {
                        atomicAdd(&sm.hist[rd], rc);
                        rc = 0;
                    }
                    rd = d;
                    rc++;
                }
                if (rc) atomicAdd(&sm.hist[rd], rc);
            }
            __syncthreads();
            bs_pick(sm, 1, k);
            pre |= sm.sel[0] << shift;
            msk |= 255u << shift;
            k -= sm.sel[1];
            __syncthreads();
        }
        const uint32_t E = pre;   // the spec's k-th largest score; k = ties to take, first by index
        for (int wd = tid; wd < BS_MAXN / 32; wd += BS_T) {
            uint32_t g = 0, q = 0;
            for (uint32_t b = sm.bd[wd]; b; b &= b - 1) {
                const int e = __ffs(b) - 1;
                const uint32_t x = sm.xs[32 * wd + e];
                g |= (uint32_t)(x > E) << e;
                q |= (uint32_t)(x == E) << e;
            }
            sm.gt[wd] |= g;
            sm.eq[wd] = q;
        }
        __syncthreads();
        bs_emit(sm, k, out, n, a.topk, a.recent);
      }
    }
}

int launch_select_band(const BandSelectArgs& a, hipStream_t st) {
    if (a.p0 + a.T - a.recent > BS_MAXN || a.ld % 32 || !a.ovf) return EMBLA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(select_band_kernel, dim3(a.T), dim3(BS_T), 0, st, a);
    if (hipGetLastError() != hipSuccess) return EMBLA_ERR_HIP;
    hipLaunchKernelGGL(band_overflow_kernel, dim3(a.T < BO_GRID ? a.T : BO_GRID), dim3(BS_T), 0, st, a);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
