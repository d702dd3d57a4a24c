// Key selection for the sparse layers: the ReLU² index scorer and the exact radix top-k.
//
// select_topk_kernel restates select_keys (Sources/EmblaMetal/Kernels/attention.metal:647-744):
// among keys [0, n = S - recent) the topk with the largest order_bits(score) (order_bits,
// attention.metal:657-660), found by three MSB-first radix passes (11, 11, 10 bits), then an ordered
// compaction: keys above the topk-th value in index order, then the first keys equal to it in
// index order, then the recent keys n .. S-1. The output is bit-exact with the reference's
// definition (order included). MI355X design: one 1024-thread workgroup a set keeps all n scores
// order bits in LDS (gfx950 has 160 KB a CU; 32K scores take 128 KB), so the passes and
// the compaction read LDS, not HBM.
//
// index_scores_kernel computes score_j = Σ_h w_h relu(q_h·k_j)² (the BASELINE configs' indexer,
// 64-dim fp16 index heads). Its fp32 order is part of the spec, so the top-k is reproducible: lane
// k (0..7) of a key takes dims 8k .. 8k + 7 as an fma chain from 0 (fp16 products are exact in
// fp32); the 8 chains combine as ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)); then
// r = max(dot, 0), s = fma(w_h, r * r, s) over h = 0 .. from s = 0. oracle/oracle.c restates it.
#include "common.hpp"
#include "embla_internal.hpp"
#include "wsel.hpp"


#pragma clang fp contract(off)

namespace embla {

constexpr int SEL_T = 1024;                 // threads of the select workgroup (16 waves)
constexpr int HBINS = 2048;                 // 11-bit radix digits: bits 31..21, 20..10, 9..0
constexpr int HCOPIES = 2;                  // copies of the first pass's histogram
constexpr int HSTRIDE = HBINS + 1;          // words a copy (offset by one word: other banks)
constexpr int LCAP = 2048;                  // bucket list capacity (else passes 2-3 read every key)
constexpr int SEL_OUTCAP = HCOPIES * HSTRIDE + LCAP;   // topk indices staged in hist + list

__device__ __forceinline__ uint32_t order_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/// Exclusive prefix sum over the 1024 threads, and the total.
__device__ __forceinline__ uint32_t block_scan_excl(uint32_t v, uint32_t* buf, uint32_t& total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t incl = v;
    incl = wave_scan_incl(incl);
    if (lane == 63) buf[w] = incl;
    __syncthreads();
    if (w == 0) {
        uint32_t x = lane < 16 ? buf[lane] : 0u, xi = x;
        xi = row_scan_incl(xi);
        if (lane < 16) buf[lane] = xi - x;
        if (lane == 15) buf[16] = xi;
    }
    __syncthreads();
    const uint32_t r = buf[w] + incl - v;
    total = buf[16];
    __syncthreads();
    return r;
}

struct SelSmem {
    uint32_t keys[SEL_MAXN];            // order bits, in index order
    uint32_t hist[HCOPIES * HSTRIDE];   // histograms; with list: the staged output at the end
    uint32_t list[LCAP];                // low 21 bits of the keys in the first pass's bucket
    uint32_t tab[2][SEL_MAXN / 256];    // compaction: counts, then offsets, a (round, wave)
    uint32_t buf[17];
    uint32_t sel[3];
    uint32_t cnt;
};

/// The digit holding the k-th largest of a histogram (ncopies copies of HBINS bins, HSTRIDE
/// apart): sel = {digit, keys in digits above it, keys in it}. Thread t owns digits 2047 - 2t and
/// 2046 - 2t.
__device__ void pick_digit(SelSmem& sm, int ncopies, uint32_t k) {
    const int tid = threadIdx.x;
    uint32_t c0 = 0, c1 = 0;
    for (int i = 0; i < ncopies; i++) {
        c0 += sm.hist[i * HSTRIDE + HBINS - 1 - 2 * tid];
        c1 += sm.hist[i * HSTRIDE + HBINS - 2 - 2 * tid];
    }
    uint32_t tot;
    const uint32_t above = block_scan_excl(c0 + c1, sm.buf, tot);
    if (above < k && above + c0 >= k) { sm.sel[0] = HBINS - 1 - 2 * tid; sm.sel[1] = above; sm.sel[2] = c0; }
    if (above + c0 < k && above + c0 + c1 >= k) { sm.sel[0] = HBINS - 2 - 2 * tid; sm.sel[1] = above + c0; sm.sel[2] = c1; }
    __syncthreads();
}

/// One set a 1024-thread workgroup. The kernel runs once a launch and is bound by instruction
/// issue on its one CU, so every pass is a short rolled loop over the LDS-resident keys that takes
/// 4 keys a lane (round r: lane t of wave w holds keys 4096 r + 4 (64 w + t) + e), with compares
/// written as wave masks and counted by scalar popcounts. Phase 1 loads the scores (16-byte,
/// every load in flight at once), stores their order bits and histograms their top 11 bits into 2
/// copies (lane parity). The bucket holding the topk-th largest goes to an LDS list (when it
/// fits) and passes 2 and 3 histogram only the list. The compaction writes, in index order, every
/// key above the topk-th value and the first keys equal to it, at offsets from a scan of
/// per-(round, wave) counts, staged in LDS and stored as one coalesced run.
__global__ __launch_bounds__(SEL_T) void select_topk_kernel(const float* __restrict__ scores, int score_stride,
                                                            uint32_t* __restrict__ idx, int idx_stride, int S,
                                                            int topk, int recent) {
    __shared__ SelSmem sm;
    const int set = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* sc = scores + (size_t)set * score_stride;
    uint32_t* out = idx + (size_t)set * idx_stride;
    const int n = S - recent;
    const int rounds = (n + 4 * SEL_T - 1) / (4 * SEL_T);
    constexpr int NL = SEL_MAXN / (4 * SEL_T);   // rounds at most (8)

    for (int q = tid; q < HCOPIES * HSTRIDE; q += SEL_T) sm.hist[q] = 0;
    if (tid == 0) sm.cnt = 0;
    __syncthreads();
    // ---- phase 1: load, order bits (0 past n: below every real key and never counted), histogram
    {
        const bool al = ((uintptr_t)sc & 15) == 0;
        u4_t v[NL];
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int j = 4 * tid + 4 * SEL_T * i;
            v[i] = (u4_t){0, 0, 0, 0};
            if (al && j + 3 < n) v[i] = ld16(sc + j);
            else if (j < n)
                for (int e = 0; e < 4; e++) v[i][e] = j + e < n ? __float_as_uint(sc[j + e]) : 0u;
        }
        uint32_t* hc = sm.hist + (lane & 1) * HSTRIDE;
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int j = 4 * tid + 4 * SEL_T * i;
            if (i < rounds) {
                u4_t o;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    o[e] = j + e < n ? order_bits(__uint_as_float(v[i][e])) : 0u;
                    if (j + e < n) atomicAdd(&hc[o[e] >> 21], 1u);
                }
                *(u4_t*)(sm.keys + j) = o;
            }
        }
    }
    __syncthreads();
    uint32_t k = (uint32_t)topk;
    pick_digit(sm, HCOPIES, k);
    const uint32_t d1 = sm.sel[0], nb = sm.sel[2];
    k -= sm.sel[1];
    uint32_t kth;
    if (nb <= LCAP) {
        // ---- the bucket's keys (low 21 bits) to the list, then passes 2 and 3 over it
        const uint64_t below = (1ull << lane) - 1ull;
        for (int r = 0; r < rounds; r++) {
            const int j = 4 * tid + 4 * SEL_T * r;
            const u4_t v = *(const u4_t*)(sm.keys + j);
            // list slots: one atomic a wave, lanes below first (the list's order is free)
            bool h[4];
            uint32_t tot = 0, pos = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                h[e] = (v[e] >> 21) == d1;   // padding (0) is never in the bucket holding the k-th
                const uint64_t m = __ballot(h[e]);
                tot += __popcll(m);
                pos += __popcll(m & below);
            }
            if (tot) {
                uint32_t base = 0;
                if (lane == 0) base = atomicAdd(&sm.cnt, tot);
                pos += __shfl(base, 0, 64);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (h[e]) sm.list[pos++] = v[e] & 0x1FFFFFu;
            }
        }
        uint32_t pre = 0;
        for (int pass = 0; pass < 2; pass++) {
            const int shift = pass == 0 ? 10 : 0;
            sm.hist[tid] = 0;
            sm.hist[tid + SEL_T] = 0;
            __syncthreads();
            for (uint32_t q = tid; q < nb; q += SEL_T) {
                const uint32_t v = sm.list[q];
                if (pass == 0 || (v >> 10) == pre) atomicAdd(&sm.hist[(v >> shift) & 2047u], 1u);
            }
            __syncthreads();
            pick_digit(sm, 1, k);
            pre = pass == 0 ? sm.sel[0] : (pre << 10) | sm.sel[0];
            k -= sm.sel[1];
            __syncthreads();
        }
        kth = (d1 << 21) | pre;
    } else {
        // ---- a bucket too large for the list: passes 2 and 3 over every key
        uint32_t prefix = d1 << 21, mask = 0xFFE00000u;
        for (int pass = 0; pass < 2; pass++) {
            const int shift = pass == 0 ? 10 : 0;
            const uint32_t dm = pass == 0 ? 2047u : 1023u;
            for (int q = tid; q < HCOPIES * HSTRIDE; q += SEL_T) sm.hist[q] = 0;
            __syncthreads();
            uint32_t* hc = sm.hist + (lane & 1) * HSTRIDE;
            for (int r = 0; r < rounds; r++) {
                const int j = 4 * tid + 4 * SEL_T * r;
                const u4_t v = *(const u4_t*)(sm.keys + j);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if ((v[e] & mask) == prefix && j + e < n) atomicAdd(&hc[(v[e] >> shift) & dm], 1u);
            }
            __syncthreads();
            pick_digit(sm, HCOPIES, k);
            prefix |= sm.sel[0] << shift;
            mask |= dm << shift;
            k -= sm.sel[1];
            __syncthreads();
        }
        kth = prefix;
    }

    // ---- ordered compaction: keys above kth, then the first k equal to it, by index. Round r,
    // wave w holds keys 4096 r + 256 w .. + 255: table entry 16 r + w. Padding keys are 0, never
    // above kth, and equal to it only if kth is 0, which needs k > every real key's count: no.
    for (int r = 0; r < rounds; r++) {
        const int j = 4 * tid + 4 * SEL_T * r;
        const u4_t v = *(const u4_t*)(sm.keys + j);
        uint32_t cg = 0, ce = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            cg += __popcll(__ballot(v[e] > kth));
            ce += __popcll(__ballot(v[e] == kth && j + e < n));
        }
        if (lane == 0) { sm.tab[0][16 * r + w] = cg; sm.tab[1][16 * r + w] = ce; }
    }
    __syncthreads();
    if (w < 2) {   // wave 0 scans the "above" table, wave 1 the "equal" one (2 entries a lane)
        uint32_t* t = sm.tab[w];
        const int m = 16 * rounds;
        const uint32_t v0 = 2 * lane < m ? t[2 * lane] : 0u, v1 = 2 * lane + 1 < m ? t[2 * lane + 1] : 0u;
        const uint32_t s = v0 + v1;
        uint32_t incl = s;
        incl = wave_scan_incl(incl);
        if (2 * lane < m) t[2 * lane] = incl - s;
        if (2 * lane + 1 < m) t[2 * lane + 1] = incl - s + v0;
        if (lane == 63) sm.sel[w] = incl;   // totals: keys above kth, keys equal to it
    }
    __syncthreads();
    const uint32_t ngt = sm.sel[0];
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t* sout = topk <= SEL_OUTCAP ? sm.hist : out;   // hist and list are contiguous
    for (int r = 0; r < rounds; r++) {
        const int j = 4 * tid + 4 * SEL_T * r;
        const u4_t v = *(const u4_t*)(sm.keys + j);
        bool g[4], e[4];
        uint32_t pg = sm.tab[0][16 * r + w], pe = sm.tab[1][16 * r + w];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            g[u] = v[u] > kth;
            e[u] = v[u] == kth && j + u < n;
            pg += __popcll(__ballot(g[u]) & below);   // the keys of lanes below this one
            pe += __popcll(__ballot(e[u]) & below);
        }
        if (g[0] | g[1] | g[2] | g[3] | e[0] | e[1] | e[2] | e[3]) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (g[u]) sout[pg++] = (uint32_t)(j + u);
                if (e[u]) {
                    if (pe < k) sout[ngt + pe] = (uint32_t)(j + u);
                    pe++;
                }
            }
        }
    }
    __syncthreads();
    if (sout != out)
        for (int j = tid; j < topk; j += SEL_T) out[j] = sout[j];
    for (int j = tid; j < recent; j += SEL_T) out[topk + j] = (uint32_t)(n + j);
}

int launch_select_topk(const float* scores, int score_stride, uint32_t* idx, int idx_stride, int S, int n_sets,
                       int topk, int recent, hipStream_t st) {
    if (S - recent > SEL_MAXN) return EMBLA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(select_topk_kernel, dim3(n_sets), dim3(SEL_T), 0, st, scores, score_stride, idx, idx_stride,
                       S, topk, recent);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// ------------------------------------------------------------------ wide select (one set)
/// The wide select's second step, a 256-thread workgroup a 1024 keys. Every workgroup finds the
/// 12-bit first digit d1 holding the topk-th largest from the scorer's histograms: the coarse
/// digit from the 256 coarse bins (summed over the copies), then d1 among that digit's 16 fine
/// bins (workgroup 0 records d1 and the keys above it). For its keys j = base + t + 256 e it then
/// writes the bitmap of keys whose digit is above d1 (a ballot covers 64 consecutive keys: two
/// words, no atomics) and the keys in digit d1 (order bits, index) to its own candidate region
/// (slots from an LDS counter), whose count it stores for the last step.
__global__ __launch_bounds__(256) void wsel_classify_kernel(const float* __restrict__ scores, int n, int topk,
                                                            uint32_t* __restrict__ sw) {
    __shared__ uint32_t ch[CB], sel[2], lcnt, total;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t* meta = sw + 2 * HWORDS;
    uint32_t* cnts = meta + 64;
    uint32_t* gt = cnts + SEL_MAXN / 1024;
    uint32_t* cand = gt + SEL_MAXN / 32 + 2 * 1024 * blockIdx.x;
    const uint32_t* H = sw + (meta[3] & 1) * HWORDS;
    const int base = blockIdx.x * 1024;
    float sv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = base + tid + 256 * e;
        sv[e] = j < n ? scores[j] : 0.0f;
    }
    uint32_t c = 0;
#pragma unroll
    for (int cp = 0; cp < NCP; cp++) c += H[cp * CB + tid];
    ch[tid] = c;
    if (tid == 0) { sel[0] = 0; sel[1] = 0; lcnt = 0; }
    __shared__ uint32_t fp[8];   // the fine bins of cd, two a word
    if (tid < 8) fp[tid] = 0;
    __syncthreads();
    if (w == 0) pick256(ch, (uint32_t)topk, sel, &total);
    __syncthreads();
    if (total != (uint32_t)n) {
        // (uniform) The buffer held counts from before this call's scorer: a workspace that was
        // not zeroed, was overwritten, or saw a call stop between its scorer and its attention.
        // Its bins cannot be trusted, so this workgroup counts the coarse digits of all n scores
        // itself (exact, ~n / 256 loads a thread); the next call's buffer is clean again, as this
        // call's scorer cleared it. meta[4] counts such calls.
        ch[tid] = 0;
        if (tid == 0) { sel[0] = 0; sel[1] = 0; }
        __syncthreads();
        for (int j = tid; j < n; j += 256) atomicAdd(&ch[order_bits(scores[j]) >> 24], 1u);
        __syncthreads();
        if (w == 0) pick256(ch, (uint32_t)topk, sel);
        if (blockIdx.x == 0 && tid == 0) atomicAdd(&meta[4], 1u);
        __syncthreads();
    }
    const uint32_t cd = sel[0] & (CB - 1), above_c = sel[1];
    {   // the fine bins of cd: the sum of the scorer workgroups' rows (one a scorer workgroup)
        const int nsc = min(index_score_blocks(n), kWideSelectScorers);
        // (a row a thread, two bins a word; summed as packed 16-bit pairs across the wave by a
        // DPP scan, no bin's total or partial sum exceeding 32768, then one LDS atomic a word a
        // wave: LDS atomics of every lane on the same 16 words cost ~19 us)
        const uint32_t* F = sw + kWideSelectFine;
        uint32_t x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (tid < nsc) {
            const u4_t x0 = *(const u4_t*)(F + (size_t)tid * 2048 + 8 * cd), x1 = *(const u4_t*)(F + (size_t)tid * 2048 + 8 * cd + 4);
#pragma unroll
            for (int i = 0; i < 4; i++) { x[i] = x0[i]; x[4 + i] = x1[i]; }
        }
        if (tid < ((nsc + 63) & ~63)) {   // uniform a wave
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = readlane_u32(wave_scan_incl(x[i]), 63);   // the wave's totals
            if (lane == 0)
#pragma unroll
                for (int i = 0; i < 8; i++) atomicAdd(&fp[i], x[i]);
        }
    }
    if (tid == 0) sel[0] = 16 * cd;
    __syncthreads();
    if (w == 0) {   // lanes < 16: fine bins 16 cd + 15 - lane, from the top
        const uint32_t v = lane < 16 ? (fp[(15 - lane) >> 1] >> (16 * ((15 - lane) & 1))) & 0xFFFF : 0u;
        uint32_t incl = v;
        incl = row_scan_incl(incl);
        const uint32_t k1 = (uint32_t)topk - above_c;
        if (lane < 16 && incl - v < k1 && incl >= k1) { sel[0] = 16 * cd + 15 - lane; sel[1] = above_c + incl - v; }
    }
    __syncthreads();
    const uint32_t d1 = sel[0];
    if (blockIdx.x == 0 && tid == 0) { meta[1] = d1; meta[2] = sel[1]; }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = base + tid + 256 * e;
        const bool real = j < n;
        const uint32_t key = order_bits(sv[e]), dg = key >> 20;
        const uint64_t bg = __ballot(real && dg > d1), bc = __ballot(real && dg == d1);
        if (lane == 0) {
            const int wd = (base + 256 * e + 64 * w) >> 5;
            gt[wd] = (uint32_t)bg;
            gt[wd + 1] = (uint32_t)(bg >> 32);
        }
        if (bc) {
            uint32_t p0 = 0;
            if (lane == 0) p0 = atomicAdd(&lcnt, (uint32_t)__popcll(bc));
            p0 = readlane_u32(p0, 0);
            if (real && dg == d1) {
                const uint32_t p = p0 + __builtin_amdgcn_mbcnt_hi((uint32_t)(bc >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bc, 0u));
                cand[2 * p] = key;   // p < 1024: a workgroup has 1024 keys
                cand[2 * p + 1] = (uint32_t)j;
            }
        }
    }
    __syncthreads();
    if (tid == 0) cnts[blockIdx.x] = lcnt;
}

int launch_wide_select(const uint16_t* qi, const float* w, const uint16_t* ki, float* scores, int S, int n_ih,
                       int topk, int recent, uint32_t* sw, hipStream_t st) {
    const int n = S - recent;
    if (n > SEL_MAXN || n <= topk) return EMBLA_ERR_UNSUPPORTED;
    int rc = launch_index_scores(qi, w, ki, scores, n, n_ih, st, sw);
    if (rc) return rc;
    hipLaunchKernelGGL(wsel_classify_kernel, dim3((n + 1023) / 1024), dim3(256), 0, st, scores, n, topk, sw);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

// ------------------------------------------------------------------ index scorer
/// One set of n_ih (<= 4) fp16 index queries [n_ih][64] and weights; keys ki [n][64] fp16.
/// A wave takes 64 keys a round: load j (16 bytes a lane) covers keys 8j .. 8j + 7, lane l holding
/// key 8j + l / 8, dims 8 (l % 8) .. + 7, so every load of the wave reads 1 KB contiguous.
/// With the wide select's workspace `sw`, each workgroup also counts its scores' top 12 order bits
/// in LDS, then thread t adds the total of coarse bin t (the top 8 bits) to histogram copy
/// blockIdx % NCP of this call's buffer (sw's epoch word picks one of two) and stores its 16 fine
/// bins (12 bits) as uint16 into the workgroup's own fine-bin row. It also clears its slice of the
/// other coarse buffer for the next call.
template <int NIH>
__global__ __launch_bounds__(256) void index_scores_kernel(const uint16_t* __restrict__ qi, const float* __restrict__ wt,
                                                           const uint16_t* __restrict__ ki, float* __restrict__ scores,
                                                           int n, uint32_t* __restrict__ sw) {
    __shared__ uint32_t lh[DB];
    const int lane = threadIdx.x & 63, kq = lane & 7;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;
    // a block's keys, load j: keys 8j .. 8j + 7, lane l: key 8j + l / 8, dims 8 (l % 8) ..; keys
    // past n read key n - 1 (no branch; their scores are neither stored nor counted)
    u4_t raw[8];
    auto load_keys = [&](int base) {
#pragma unroll
        for (int j = 0; j < 8; j++) raw[j] = ld16(ki + (size_t)min(base + 8 * j + (lane >> 3), n - 1) * 64 + 8 * kq);
    };
    // the first block's keys are requested before anything else (a wave has one block at up to
    // 262144 keys): the histogram clear, its barrier and the queries' loads run under them
    load_keys(wave * 64);
    uint32_t epoch = 0;
    if (sw) {
        epoch = sw[2 * HWORDS + 3];
        for (int b = threadIdx.x; b < DB; b += 256) lh[b] = 0;
        __syncthreads();
    }
    float q[NIH][8], w[NIH];
#pragma unroll
    for (int h = 0; h < NIH; h++) {
        const u4_t r = ld16(qi + h * 64 + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[h][2 * i] = h2f((uint16_t)(r[i] & 0xFFFF));
            q[h][2 * i + 1] = h2f((uint16_t)(r[i] >> 16));
        }
        w[h] = wt[h];
    }
    for (int base = wave * 64; base < n; base += nwaves * 64) {
        if (base != wave * 64) load_keys(base);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float kf[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kf[2 * i] = h2f((uint16_t)(raw[j][i] & 0xFFFF));
                kf[2 * i + 1] = h2f((uint16_t)(raw[j][i] >> 16));
            }
            float s = 0.0f;
#pragma unroll
            for (int h = 0; h < NIH; h++) {
                float c = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) c = __builtin_fmaf(q[h][d], kf[d], c);
                // lane xor 1, xor 2 (quad_perm), then the other quad of the 8 (row_half_mirror: its 4
                // lanes agree by then): the spec's ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7))
                c = c + dpp_f32<0xB1>(c);
                c = c + dpp_f32<0x4E>(c);
                c = c + dpp_f32<0x141>(c);
                const float r = fmaxf(c, 0.0f);
                const float r2 = r * r;
                s = __builtin_fmaf(w[h], r2, s);
            }
            const int key = base + 8 * j + (lane >> 3);
            if (kq == 0 && key < n) {
                scores[key] = s;
                if (sw) atomicAdd(&lh[order_bits(s) >> 20], 1u);
            }
        }
    }
    if (sw) {
        __syncthreads();
        const int t = threadIdx.x;
        uint32_t* H = sw + (epoch & 1) * HWORDS + (blockIdx.x % NCP) * CB;
        uint32_t cs = 0;
        // the coarse bins by device atomics (few distinct a workgroup); the fine bins as this
        // workgroup's own uint16 row of the fine table, by plain stores (classify sums the rows
        // for the one coarse digit it picks: device atomics on ~100 fine bins a workgroup cost
        // ~2 us a call)
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t c0 = lh[16 * t + 2 * i], c1 = lh[16 * t + 2 * i + 1];   // <= 256 each
            cs += c0 + c1;
            pk[i] = c0 | (c1 << 16);
        }
        uint32_t* F = sw + kWideSelectFine + (size_t)blockIdx.x * 2048 + 8 * t;
        *(u4_t*)F = (u4_t){pk[0], pk[1], pk[2], pk[3]};
        *(u4_t*)(F + 4) = (u4_t){pk[4], pk[5], pk[6], pk[7]};
        if (cs) atomicAdd(&H[t], cs);
        uint32_t* Z = sw + ((epoch + 1) & 1) * HWORDS;
        for (int q = blockIdx.x * 256 + t; q < HWORDS; q += gridDim.x * 256) Z[q] = 0;
    }
}

int launch_index_scores(const uint16_t* qi, const float* w, const uint16_t* ki, float* scores, int n, int n_ih,
                        hipStream_t st, uint32_t* sw) {
    const int blocks = index_score_blocks(n);
    switch (n_ih) {
        case 1: hipLaunchKernelGGL(index_scores_kernel<1>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n, sw); break;
        case 2: hipLaunchKernelGGL(index_scores_kernel<2>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n, sw); break;
        case 4: hipLaunchKernelGGL(index_scores_kernel<4>, dim3(blocks), dim3(256), 0, st, qi, w, ki, scores, n, sw); break;
        default: return EMBLA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
