// The wide select (select_keys on many workgroups, select.hip) as seen by its last step: the
// workspace layout, the radix digit picks, and the ranking of the candidates in the k-th value's
// first digit, with the output in select_keys' order (attention.metal:680-744: keys above the
// topk-th value by index, then the first keys equal to it by index). That last step runs inside
// the sparse-layer decode's own workgroups, each producing the slice of the output ranks it
// attends, so the selection costs no launch of its own.
#pragma once
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

constexpr int SEL_MAXN = kWideSelectMaxN;   // candidates a set
constexpr int DB = 4096;                    // the wide select's 12-bit digits: bits 31..20, 19..8
constexpr int CB = 256;                     // its coarse first digit: bits 31..24
constexpr int NCP = WSEL_NCP;               // histogram copies (scorer workgroup % NCP)
constexpr int HWORDS = NCP * CB;            // words a histogram buffer (two, by call parity)
// The workspace sw, in words: two coarse histogram buffers [2][HWORDS] (NCP copies of the
// scores' top-8-bit counts); meta[64] (1: the first digit d1 of the topk-th largest, 2: keys in
// digits above d1, 3: the epoch picking the buffer, 4: calls that found their histogram buffer
// not clean and recounted, kWideSelectRecounts); the classify workgroups' candidate counts
// [SEL_MAXN / 1024]; the bitmap of keys above d1 [SEL_MAXN / 32]; each classify workgroup's
// candidate region (order bits, index) x 1024 (from kWideSelectFine on: the scorer workgroups'
// own rows of top-12-bit counts, uint16 [kWideSelectScorers][4096]).
__device__ __forceinline__ const uint32_t* wsel_meta(const uint32_t* sw) { return sw + 2 * HWORDS; }
static_assert(kWideSelectEpoch == 2 * HWORDS + 3, "the epoch word is meta[3]");

/// Digit (of 4096) holding the k-th largest of h: sel = {digit, keys in digits above}. Wave 0:
/// each lane sums 64 digits from the top; the lane whose digits hold the k-th is found by a scan
/// and a ballot, then its 64 digits go one a lane through a second scan.
__device__ __forceinline__ void pick4096(const uint32_t* h, uint32_t k, uint32_t* sel) {
    const int lane = threadIdx.x & 63;
    const int b0 = DB - 64 - 64 * lane;   // the lane's digits b0 .. b0 + 63
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const u4_t x = *(const u4_t*)(h + b0 + 4 * i);
        s += (x[0] + x[1]) + (x[2] + x[3]);
    }
    uint32_t above = s;
    above = wave_scan_incl(above);
    above -= s;
    const int L = max(__ffsll((long long)__ballot(above < k && above + s >= k)) - 1, 0);   // 0 if none
    const uint32_t base = readlane_u32(above, L);   // L is uniform
    const int d = DB - 1 - 64 * L - lane;
    const uint32_t c = h[d];
    uint32_t incl = c;
    incl = wave_scan_incl(incl);
    if (base + incl - c < k && base + incl >= k) { sel[0] = (uint32_t)d; sel[1] = base + incl - c; }
}

/// Digit (of 256) holding the k-th largest: wave 0, 4 digits a lane from the top. total (if set)
/// receives the sum of all 256 counts.
__device__ __forceinline__ void pick256(const uint32_t* h, uint32_t k, uint32_t* sel, uint32_t* total = nullptr) {
    const int lane = threadIdx.x & 63;
    uint32_t cc[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) { cc[i] = h[255 - 4 * lane - i]; s += cc[i]; }
    uint32_t above = s;
    above = wave_scan_incl(above);
    if (total && lane == 63) *total = above;
    above -= s;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (above < k && above + cc[i] >= k) { sel[0] = 255u - (4 * lane + i); sel[1] = above; }
        above += cc[i];
    }
}

/// Exclusive prefix sum over a BT-thread workgroup, and the total (wsum: BT / 64 words).
template <int BT>
__device__ __forceinline__ uint32_t wsel_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t incl = v;
    incl = wave_scan_incl(incl);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < BT / 64; i++) {
        const uint32_t x = wsum[i];
        before += i < w ? x : 0u;
        total += x;
    }
    __syncthreads();   // wsum is reused by the next scan
    return before + incl - v;
}

/// Emits the keys of ranks [r0, r0 + nr) of select_keys' order from the bitmaps of keys above the
/// topk-th value (g) and of keys equal to it (e): the thread holds words wd0 .. wd0 + NWD - 1 (keys
/// in index order), pg / pe are the keys of each kind before its words, ngt those above in all,
/// kt the ties to take (the first by index). rows[r - r0] and out[r] when not null.
template <int NWD>
__device__ __forceinline__ void wsel_emit(const uint32_t (&g)[NWD], const uint32_t (&e)[NWD], int wd0, uint32_t pg,
                                          uint32_t cg, uint32_t pe, uint32_t ce, uint32_t ngt, uint32_t kt, int topk,
                                          uint32_t r0, uint32_t nr, uint32_t* rows, uint32_t* __restrict__ out) {
    const uint32_t r1 = r0 + nr;
    if (pg < r1 && pg + cg > r0) {   // some of this thread's keys above the value fall in the slice
#pragma unroll 1
        for (int i = 0; i < NWD; i++)
            for (uint32_t b = g[i]; b && pg < (uint32_t)topk; b &= b - 1, pg++) {
                if (pg < r0 || pg >= r1) continue;
                const uint32_t j = 32u * (wd0 + i) + __ffs(b) - 1;
                if (rows) rows[pg - r0] = j;
                if (out) out[pg] = j;
            }
    }
    if (ngt + pe < r1 && ngt + pe + ce > r0) {   // ties
#pragma unroll 1
        for (int i = 0; i < NWD; i++)
            for (uint32_t b = e[i]; b && pe < kt && ngt + pe < (uint32_t)topk; b &= b - 1, pe++) {
                const uint32_t r = ngt + pe;
                if (r < r0 || r >= r1) continue;
                const uint32_t j = 32u * (wd0 + i) + __ffs(b) - 1;
                if (rows) rows[r - r0] = j;
                if (out) out[r] = j;
            }
    }
}

/// LDS words wsel_slice_block uses besides its copy of the candidate list: the second-level
/// histogram, the two bitmaps, the regions' offsets, scan and pick words.
constexpr int WSL_FIXED = DB + 2 * (SEL_MAXN / 32) + (SEL_MAXN / 1024 + 2) + 16 + 2;

/// The wide select's last step by a whole workgroup of BT threads (any number of candidates): the
/// second (bits 19..8) and third (7..0) radix levels over the candidate list (the keys in the
/// topk-th value's first digit) give the topk-th value E and the ties to take; candidates above E
/// join the bitmap of keys above the first digit, those equal to E form the tie bitmap, and block
/// scans of the bitmaps' popcounts give each key's rank (wsel_emit). L: LDS scratch of lwords
/// words (at least WSL_FIXED + 2, 8-byte aligned). Counts are clamped and every write is bounded,
/// so a workspace that was not zeroed gives a wrong selection, never a stray access.
template <int BT>
__device__ __forceinline__ void wsel_slice_block(int n, int topk, const uint32_t* __restrict__ sw, uint32_t* L,
                                                 int lwords, uint32_t r0, uint32_t nr, uint32_t* rows,
                                                 uint32_t* __restrict__ out) {
    constexpr int NW = SEL_MAXN / 32, WPT = NW / BT;   // bitmap words, words a thread
    constexpr int NR = SEL_MAXN / 1024;                // candidate regions
    static_assert(NW % BT == 0 && BT % 64 == 0 && BT <= 1024, "threads");
    uint32_t* h2 = L;
    uint32_t* gts = h2 + DB;
    uint32_t* eqs = gts + NW;
    uint32_t* coff = eqs + NW;          // NR + 1 offsets
    uint32_t* wsum = coff + NR + 2;     // 16
    uint32_t* sel = wsum + 16;
    uint32_t* cl = sel + 2;             // the candidate list, when it fits
    const uint32_t clcap = (uint32_t)(lwords - WSL_FIXED) / 2;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const uint32_t* meta = wsel_meta(sw);
    const uint32_t* cnts = meta + 64;
    const uint32_t* gt = cnts + NR;
    const uint32_t* creg = gt + NW;
    const int nw = (n + 31) / 32, nb = (n + 1023) / 1024;
    const uint32_t d1 = meta[1] & (DB - 1);
    uint32_t k = (uint32_t)topk - min(meta[2], (uint32_t)topk - 1);   // rank of the topk-th among the candidates
    for (int q = tid; q < DB; q += BT) h2[q] = 0;
#pragma unroll
    for (int i = 0; i < WPT; i++) {
        gts[WPT * tid + i] = WPT * tid + i < nw ? gt[WPT * tid + i] : 0u;
        eqs[WPT * tid + i] = 0;
    }
    if (w == 0) {   // offsets of the regions in the list (nb <= NR)
        const uint32_t c = lane < nb ? min(cnts[lane], 1024u) : 0u;
        uint32_t incl = c;
        incl = wave_scan_incl(incl);
        if (lane < nb) coff[lane] = incl - c;
        if (lane == nb - 1) coff[nb] = incl;
    }
    __syncthreads();
    const uint32_t cnt = coff[nb];
    const bool inl = cnt <= clcap;
    if (inl) {   // wave w copies regions w, w + BT / 64, ...
        for (int b = w; b < nb; b += BT / 64) {
            const uint32_t o = coff[b], nc = coff[b + 1] - o;
            for (uint32_t q = lane; q < nc; q += 64)
                *(u2_t*)(cl + 2 * (o + q)) = *(const u2_t*)(creg + 2 * (1024 * b + q));
        }
        __syncthreads();
    }
    // candidate q: from the list, else from region b at creg[2 (1024 b + q - coff[b])]
    auto cand = [&](uint32_t q, uint32_t& key, uint32_t& j) {
        if (inl) {
            key = cl[2 * q];
            j = cl[2 * q + 1];
            return;
        }
        int b = 0;
        while (b + 1 < nb && coff[b + 1] <= q) b++;
        const uint32_t* c2 = creg + 2 * (1024 * b + (q - coff[b]));
        key = c2[0];
        j = c2[1];
    };
    for (uint32_t q = tid; q < cnt; q += BT) {
        uint32_t key, j;
        cand(q, key, j);
        atomicAdd(&h2[(key >> 8) & 0xFFF], 1u);
    }
    if (tid == 0) { sel[0] = 0; sel[1] = 0; }
    __syncthreads();
    if (w == 0) pick4096(h2, k, sel);
    __syncthreads();
    const uint32_t p2 = (d1 << 12) | (sel[0] & (DB - 1));
    k -= sel[1];
    __syncthreads();
    for (int q = tid; q < 256; q += BT) h2[q] = 0;
    __syncthreads();
    for (uint32_t q = tid; q < cnt; q += BT) {
        uint32_t key, j;
        cand(q, key, j);
        if ((key >> 8) == p2) atomicAdd(&h2[key & 255], 1u);
    }
    if (tid == 0) { sel[0] = 0; sel[1] = 0; }
    __syncthreads();
    if (w == 0) pick256(h2, k, sel);
    __syncthreads();
    const uint32_t E = (p2 << 8) | (sel[0] & 255);
    k -= sel[1];   // keys equal to E to take (>= 1)
    for (uint32_t q = tid; q < cnt; q += BT) {
        uint32_t key, j;
        cand(q, key, j);
        j &= SEL_MAXN - 1;
        if (key > E) atomicOr(&gts[j >> 5], 1u << (j & 31));
        else if (key == E) atomicOr(&eqs[j >> 5], 1u << (j & 31));
    }
    __syncthreads();
    uint32_t g[WPT], e[WPT], cg = 0, ce = 0;
#pragma unroll
    for (int i = 0; i < WPT; i++) {
        g[i] = gts[WPT * tid + i];
        e[i] = eqs[WPT * tid + i];
        cg += __popc(g[i]);
        ce += __popc(e[i]);
    }
    uint32_t ngt, neq;
    const uint32_t pg = wsel_scan<BT>(cg, wsum, ngt);
    const uint32_t pe = wsel_scan<BT>(ce, wsum, neq);
    wsel_emit<WPT>(g, e, WPT * tid, pg, cg, pe, ce, ngt, k, topk, r0, nr, rows, out);
}

constexpr int WSL_WSPEC = 32;    // candidates a region the fast path reads (its limit a region)
constexpr int WSL_WMAX = 256;    // candidates the fast path ranks (one a thread)

/// Digit (of 1024) holding the k-th largest of h: sel = {digit, keys in digits above}. Wave 0:
/// each lane sums 16 digits from the top; the lane whose digits hold the k-th is found by a scan
/// and a ballot, then its 16 digits go one a lane through a second scan.
__device__ __forceinline__ void pick1024(const uint32_t* h, uint32_t k, uint32_t* sel) {
    const int lane = threadIdx.x & 63;
    const int b0 = 1024 - 16 - 16 * lane;   // the lane's digits b0 .. b0 + 15
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u4_t x = *(const u4_t*)(h + b0 + 4 * i);
        s += (x[0] + x[1]) + (x[2] + x[3]);
    }
    uint32_t above = s;
    above = wave_scan_incl(above);
    above -= s;
    const int L = max(__ffsll((long long)__ballot(above < k && above + s >= k)) - 1, 0);   // 0 if none
    const uint32_t base = readlane_u32(above, L);   // L is uniform
    const int d = 1023 - 16 * L - (lane & 15);
    const uint32_t c = lane < 16 ? h[d] : 0u;
    uint32_t incl = c;
    incl = row_scan_incl(incl);
    if (lane < 16 && base + incl - c < k && base + incl >= k) { sel[0] = (uint32_t)d; sel[1] = base + incl - c; }
}

/// The n-th (from 0) set bit of x (n < popcount(x)), by halving.
__device__ __forceinline__ uint32_t nth_set_bit(uint32_t x, uint32_t n) {
    uint32_t pos = 0;
#pragma unroll
    for (int h = 16; h >= 1; h >>= 1) {
        const uint32_t c = (uint32_t)__popc(x & ((1u << h) - 1u));
        if (n >= c) { n -= c; pos += h; x >>= h; }
    }
    return pos;
}

/// The wide select's last step for output ranks [r0, r0 + nr) of n candidates' top `topk` (nr
/// <= 64), in select_keys' order: rows[r - r0] (LDS) receives the key of rank r when rows is not
/// null, and out[r] when out is not null. BT threads (>= WSL_WMAX), every thread of the
/// workgroup; L: LDS scratch of lwords words (at least WSL_FIXED + 2, 8-byte aligned).
///
/// The common case keeps every dependent chain short (a lone wave issues about one instruction
/// in 8 cycles there, so the step is bound by its longest chain, not by its work):
///  - wave 0 requests, in one memory round, the bitmap of keys above the first digit (16 words a
///    lane), the candidate counts and the first WSL_WSPEC candidates of every region (16 a
///    lane), and compacts the candidates into LDS;
///  - the topk-th value E comes from two 10-bit digits of the candidates' low 20 bits (they share
///    the first 12): a candidate a thread adds itself to an LDS histogram, wave 0 picks the digit
///    holding the k-th; then every candidate marks itself in the bitmap (above E) or in the tie
///    bitmap (equal to E);
///  - wave 0 scans the bitmaps' popcounts into per-word prefixes, and lane i finds rank r0 + i by
///    a binary search over them and a halving search in the word.
/// A region with more than WSL_WSPEC candidates, more than WSL_WMAX in all, or a slice of more
/// than 64 ranks go to wsel_slice_block instead.
template <int BT>
__device__ __forceinline__ void wsel_slice(int n, int topk, const uint32_t* __restrict__ sw, uint32_t* L, int lwords,
                                           uint32_t r0, uint32_t nr, uint32_t* rows, uint32_t* __restrict__ out) {
    constexpr int NW = SEL_MAXN / 32, NR = SEL_MAXN / 1024;
    static_assert(NW == 16 * 64 && NR == 32 && 2 * WSL_WSPEC == 64 && BT >= WSL_WMAX, "the fast path's shape");
    static_assert(4 * NW + 2 * WSL_WMAX + 33 <= WSL_FIXED, "the fast path's words, its junk word included, within L");
    __shared__ uint32_t wsl_ok, wsl_tot, wsl_k, wsl_kt, wsl_sel[2];
    uint32_t* gts = L;                          // NW: keys above E
    uint32_t* eqs = L + NW;                     // NW: keys equal to E
    uint32_t* pg = L + 2 * NW;                  // NW: keys above E before word w (first: a histogram)
    uint32_t* pe = L + 3 * NW;                  // NW: keys equal to E before word w (first: a histogram)
    uint32_t* cj = L + 4 * NW;                  // WSL_WMAX candidate indices
    uint32_t* ck = cj + WSL_WMAX;               // WSL_WMAX + 16 candidate keys (16-byte aligned)
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t* meta = wsel_meta(sw);
    if (tid < 64) {
        const uint32_t* cnts = meta + 64;
        const uint32_t* gt = cnts + NR;
        const uint32_t* creg = gt + NW;
        const int nw = (n + 31) / 32, nb = (n + 1023) / 1024;
        const int rb = lane >> 1, rh = lane & 1;   // the lane's region and half of its first 32
        u4_t gw[4], cv[8];
#pragma unroll
        for (int i = 0; i < 4; i++) gw[i] = *(const u4_t*)(gt + 16 * lane + 4 * i);
#pragma unroll
        for (int i = 0; i < 8; i++) cv[i] = *(const u4_t*)(creg + 2 * (1024 * rb + 16 * rh) + 4 * i);
        const uint32_t cown = lane < nb ? min(cnts[lane], 1024u) : 0u;
        const uint32_t cb = __shfl(cown, rb, 64);   // the lane's region's count (0 past nb)
        const uint32_t tot = readlane_u32(wave_scan_incl(cown), 63);
        const bool ok = __ballot(cb > WSL_WSPEC) == 0 && tot <= WSL_WMAX && nr <= 64;
        if (ok) {
            const uint32_t nv = (uint32_t)min(max((int)cb - 16 * rh, 0), 16);   // the lane's candidates
            uint32_t incl = nv;
            incl = wave_scan_incl(incl);
            const uint32_t off = incl - nv;
            // a lane's items past its count go to a junk word past the keys' padding, never read
            // (unconditional stores: a store under a lane's own condition compiled to a branch each)
            uint32_t* const junk = ck + WSL_WMAX + 32;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const bool live = i < (int)nv;
                *(live ? ck + off + i : junk) = cv[i >> 1][2 * (i & 1)];
                *(live ? cj + off + i : junk) = cv[i >> 1][2 * (i & 1) + 1] & (SEL_MAXN - 1);
            }
            if (lane < 16) ck[tot + lane] = 0;   // zero keys up to a multiple of 4 (and beyond)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                u4_t v = gw[i];
#pragma unroll
                for (int x = 0; x < 4; x++) v[x] = 16 * lane + 4 * i + x < nw ? v[x] : 0u;
                *(u4_t*)(gts + 16 * lane + 4 * i) = v;
                *(u4_t*)(eqs + 16 * lane + 4 * i) = (u4_t){0, 0, 0, 0};
            }
        }
        if (lane == 0) {
            wsl_ok = ok;
            wsl_tot = tot;
            wsl_k = (uint32_t)topk - min(meta[2], (uint32_t)topk - 1);   // the topk-th's rank among the candidates
            wsl_kt = 0;
        }
    }
    else   // the other waves clear the two digit histograms meanwhile
        for (int q = tid - 64; q < 2 * NW / 4; q += BT - 64) *(u4_t*)(pg + 4 * q) = (u4_t){0, 0, 0, 0};
    __syncthreads();
    if (!wsl_ok) {   // uniform
        wsel_slice_block<BT>(n, topk, sw, L, lwords, r0, nr, rows, out);
        return;
    }
    const uint32_t tot = wsl_tot, k = wsl_k;
    // E by two 10-bit digits of the low 20 bits (the candidates share the first 12): histograms,
    // picks by wave 0; then each candidate marks itself above E or equal to it
    const uint32_t key = tid < (int)tot ? ck[tid] : 0u;
    if (tid < (int)tot) atomicAdd(&pg[(key >> 10) & 1023], 1u);
    __syncthreads();
    if (tid < 64) pick1024(pg, k, wsl_sel);
    __syncthreads();
    const uint32_t da = wsl_sel[0] & 1023, ka = k - wsl_sel[1];
    if (tid < (int)tot && ((key >> 10) & 1023) == da) atomicAdd(&pe[key & 1023], 1u);
    __syncthreads();
    if (tid < 64) pick1024(pe, ka, wsl_sel);
    __syncthreads();
    const uint32_t E = ((meta[1] & (DB - 1)) << 20) | (da << 10) | (wsl_sel[0] & 1023);
    if (tid < (int)tot) {
        const uint32_t j = cj[tid];
        if (key > E) atomicOr(&gts[j >> 5], 1u << (j & 31));
        else if (key == E) atomicOr(&eqs[j >> 5], 1u << (j & 31));
    }
    if (tid == 0) wsl_kt = ka - wsl_sel[1];   // the ties to take
    __syncthreads();
    if (tid < 64) {
        uint32_t g[16], e[16], cg = 0, ce = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u4_t a = *(const u4_t*)(gts + 16 * lane + 4 * i), z = *(const u4_t*)(eqs + 16 * lane + 4 * i);
#pragma unroll
            for (int x = 0; x < 4; x++) {
                g[4 * i + x] = (uint32_t)__popc(a[x]);
                e[4 * i + x] = (uint32_t)__popc(z[x]);
                cg += g[4 * i + x];
                ce += e[4 * i + x];
            }
        }
        uint32_t ig = cg, ie = ce;
        ig = wave_scan_incl(ig);
        ie = wave_scan_incl(ie);
        const uint32_t ngt = readlane_u32(ig, 63), kt = wsl_kt;
        uint32_t sg = ig - cg, se = ie - ce;
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            *(u4_t*)(pg + 16 * lane + i) = (u4_t){sg, sg + g[i], sg + g[i] + g[i + 1], sg + g[i] + g[i + 1] + g[i + 2]};
            *(u4_t*)(pe + 16 * lane + i) = (u4_t){se, se + e[i], se + e[i] + e[i + 1], se + e[i] + e[i + 1] + e[i + 2]};
            sg += (g[i] + g[i + 1]) + (g[i + 2] + g[i + 3]);
            se += (e[i] + e[i + 1]) + (e[i + 2] + e[i + 3]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lane i: rank r0 + i, above E (in index order) or the (r - ngt)-th tie
        const uint32_t r = r0 + (uint32_t)lane;
        if ((uint32_t)lane < nr && r < (uint32_t)topk && r < ngt + kt) {
            const bool isg = r < ngt;
            const uint32_t* pf = isg ? pg : pe;
            const uint32_t* bm = isg ? gts : eqs;
            const uint32_t t = isg ? r : r - ngt;
            uint32_t lo = 0;   // the last word whose prefix is <= t
#pragma unroll
            for (uint32_t h = NW / 2; h >= 1; h >>= 1)
                if (pf[lo + h] <= t) lo += h;
            const uint32_t j = 32u * lo + nth_set_bit(bm[lo], t - pf[lo]);
            if (rows) rows[lane] = j;
            if (out) out[r] = j;
        }
    }
    __syncthreads();
}

}  // namespace embla
