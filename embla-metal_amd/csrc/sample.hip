// The sampling tail after the lm-head: the greedy token, or a draw from softmax(softcap(l) / T)
// cut to its top-p nucleus, over V fp32 logits.
//
// Follows misc.metal:83-128 (argmax) and 164-298 (sample). Each logit is softcapped in bf16 as
// bf(bf(tanh(bf(bf(l) / 15))) * 15). The greedy token is the first index of the largest. The draw
// finds the nucleus' threshold on e = exp(x), x = c / T - max, by 20 bisection steps: over the
// tokens with e >= 1/16384 from [1/16384, 1) when there are at most 2048 of them and they hold
// top-p of the mass, else over all tokens from [0, 1). It then takes the argmax of x + Gumbel
// noise over the tokens with x >= log(threshold), the noise a hash of (seed, position, token).
// Outputs as the reference's: greedy[pos], token[pos + 1] past the prompt, and last the word
// greedy[-1] = (pos + 1) << 16 | token for a host that polls.
//
// MI355X design (the reference runs each as one 1024-thread threadgroup). A lone workgroup reads
// another kernel's fresh output at ~22 ns a 128-byte line, so the 256 KB row is read by 64
// workgroups of 1024 tokens:
//  - logit_scan_kernel: softcap, block max and its first index, and for the draw the capped row
//    as bf16 (128 KB) for the next kernels;
//  - greedy: argmax_final_kernel merges the 64 block maxima (one wave);
//  - draw: sample_weights_kernel (64 workgroups) takes the global max from the block maxima and
//    writes per block the sums of e and of e >= 1/16384, their count, the candidates (token and
//    capped value packed in a word, compacted in the block's own list) and the block's Gumbel
//    winner over all its tokens (the draw when the threshold stays 0); sample_final_kernel (one
//    workgroup) sums the block records and runs the bisection over the <= 2048 candidates in LDS;
//    when the reference would bisect over all tokens it holds the row's e in registers instead
//    (64 a thread), and draws again only the blocks whose winner over all tokens lies outside the
//    nucleus.
// Every value a later kernel needs is recomputed from the capped bf16 with the same rounded
// operations (__fmul_rn, __fsub_rn: no contraction), so x and e agree bit for bit between kernels.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

constexpr int SB = 1024;                   // tokens a block: 256 threads x 4
constexpr float CMIN = 1.0f / 16384.0f;    // the candidates' floor on e
constexpr int NCAND = 2048;                // candidates the bisection holds (misc.metal:231)

__device__ __forceinline__ float bfr(float x) { return bf2f(f2bf(x)); }

/// bf(bf(tanh(bf(bf(l) / 15))) * 15) with tanh correctly rounded to fp32: tanhf's result is exact
/// enough unless its low 16 bits sit near the bf16 rounding midpoint, and then tanh is taken in
/// fp64 and rounded once.
__device__ __forceinline__ uint16_t softcap_bits(float l) {
    const float y = bfr(__fdiv_rn(bfr(l), 15.0f));
    float t = tanhf(y);
    const uint32_t low = __float_as_uint(t) & 0xFFFFu;
    if (low >= 0x7FE0u && low <= 0x8020u) t = (float)tanh((double)y);
    return f2bf(__fmul_rn(bfr(t), 15.0f));
}

__host__ __device__ __forceinline__ uint32_t mix32(uint32_t x) {   // misc.metal:186-191
    x ^= x >> 16; x *= 0x7feb352du;
    x ^= x >> 15; x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

/// x + Gumbel noise of token i (misc.metal:278-281)
__device__ __forceinline__ float gumbel_score(float x, uint32_t key, uint32_t i) {
    const float u = __fmul_rn(__fadd_rn((float)(mix32(key ^ i) >> 8), 0.5f), 1.0f / 16777216.0f);
    return __fsub_rn(x, logf(-logf(u)));
}

/// (value, index) with the larger value winning and the lower index on ties
__device__ __forceinline__ void best_of(float& v, uint32_t& i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__device__ __forceinline__ void wave_best(float& v, uint32_t& i) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const uint32_t oi = __shfl_xor(i, o, 64);
        best_of(v, i, ov, oi);
    }
}

__device__ __forceinline__ float wave_sum(float v) {   // the xor butterfly's sum, bit for bit
    return wave_bfly(v, [](float a, float b) { return a + b; });
}

// ------------------------------------------------------------------ block scan
__global__ __launch_bounds__(256) void logit_scan_kernel(const float* __restrict__ logits, int V, float inv_t,
                                                         uint16_t* __restrict__ cb, float* __restrict__ bmax,
                                                         uint32_t* __restrict__ bidx) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const int t = threadIdx.x, i0 = blockIdx.x * SB + 4 * t;
    float l[4];
    if (i0 + 3 < V) {
        const float4 v = *(const float4*)(logits + i0);
        l[0] = v.x; l[1] = v.y; l[2] = v.z; l[3] = v.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) l[k] = i0 + k < V ? logits[i0 + k] : 0.0f;
    }
    float best = NEG_INF;
    uint32_t bi = 0xFFFFFFFFu;
    uint16_t c[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        c[k] = softcap_bits(l[k]);
        const float cs = __fmul_rn(bf2f(c[k]), inv_t);
        if (i0 + k < V && cs > best) { best = cs; bi = (uint32_t)(i0 + k); }
    }
    if (cb) {
        if (i0 + 3 < V) *(u2_t*)(cb + i0) = (u2_t){(uint32_t)c[0] | ((uint32_t)c[1] << 16), (uint32_t)c[2] | ((uint32_t)c[3] << 16)};
        else
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (i0 + k < V) cb[i0 + k] = c[k];
    }
    wave_best(best, bi);
    if ((t & 63) == 0) { sv[t >> 6] = best; si[t >> 6] = bi; }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 4; w++) best_of(best, bi, sv[w], si[w]);
        bmax[blockIdx.x] = best;
        bidx[blockIdx.x] = bi;
    }
}

/// The step's outputs as misc.metal:118-125 writes them, the polled word last.
__device__ __forceinline__ void write_token(uint32_t idx, uint32_t* token, uint32_t* greedy, int pos, int prompt) {
    greedy[pos] = idx;
    if (pos + 1 >= prompt) token[pos + 1] = idx;
    __threadfence_system();
    __hip_atomic_store(greedy - 1, ((uint32_t)(pos + 1) << 16) | idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ bmax, const uint32_t* __restrict__ bidx,
                                                          int G, uint32_t* token, uint32_t* greedy, int pos, int prompt) {
    const int t = threadIdx.x;
    float v = t < G ? bmax[t] : NEG_INF;
    uint32_t i = t < G ? bidx[t] : 0xFFFFFFFFu;
    wave_best(v, i);
    // every logit NaN leaves no maximum: token 0, as the reference's initial index
    if (t == 0) write_token(i == 0xFFFFFFFFu ? 0u : i, token, greedy, pos, prompt);
}

// ------------------------------------------------------------------ the draw
struct BlockRec { float z, cm; uint32_t nc; float s; uint32_t si; float x; uint32_t pad[2]; };   // x: the winner's

/// the global max of x's scale: the largest block maximum (every wave computes it)
__device__ __forceinline__ float global_max(const float* bmax, int G) {
    const int lane = threadIdx.x & 63;
    float m = lane < G ? bmax[lane] : NEG_INF;
    m = wave_bfly(m, [](float a, float b) { return fmaxf(a, b); });
    return m;
}

__global__ __launch_bounds__(256) void sample_weights_kernel(const uint16_t* __restrict__ cb, int V, float inv_t,
                                                             const float* __restrict__ bmax, int G, uint32_t key,
                                                             BlockRec* __restrict__ rec, uint32_t* __restrict__ cand) {
    __shared__ float sz[4], scm[4], ss[4];
    __shared__ uint32_t sn[4], ssi[4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, b = blockIdx.x, i0 = b * SB + 4 * t;
    const float M = global_max(bmax, G);
    uint16_t c[4];
    if (i0 + 3 < V) {
        const u2_t v = ld8(cb + i0);
        c[0] = v[0] & 0xFFFF; c[1] = v[0] >> 16; c[2] = v[1] & 0xFFFF; c[3] = v[1] >> 16;
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) c[k] = i0 + k < V ? cb[i0 + k] : 0;
    }
    float z = 0.0f, cm = 0.0f, best = NEG_INF;
    uint32_t n = 0, bi = 0xFFFFFFFFu, mine = 0;   // mine: bit k set for a candidate
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (i0 + k >= V) continue;
        const float x = __fsub_rn(__fmul_rn(bf2f(c[k]), inv_t), M);
        const float e = expf(x);
        z += e;
        if (e >= CMIN) { cm += e; n++; mine |= 1u << k; }
        best_of(best, bi, gumbel_score(x, key, (uint32_t)(i0 + k)), (uint32_t)(i0 + k));
    }
    // candidates compacted in the block's list, in token order: exclusive scan of n
    uint32_t incl = n;
    incl = wave_scan_incl(incl);
    z = wave_sum(z);
    cm = wave_sum(cm);
    wave_best(best, bi);
    if (lane == 63) sn[w] = incl;
    if (lane == 0) { sz[w] = z; scm[w] = cm; ss[w] = best; ssi[w] = bi; }
    __syncthreads();
    uint32_t at = incl - n;
    for (int ww = 0; ww < w; ww++) at += sn[ww];
    uint32_t* out = cand + (size_t)b * SB;
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (mine >> k & 1u) out[at++] = ((uint32_t)(i0 + k) << 16) | c[k];
    if (t == 0) {
        BlockRec r;
        r.z = sz[0]; r.cm = scm[0]; r.nc = sn[0]; r.s = ss[0]; r.si = ssi[0];
        for (int ww = 1; ww < 4; ww++) {
            r.z += sz[ww];
            r.cm += scm[ww];
            r.nc += sn[ww];
            best_of(r.s, r.si, ss[ww], ssi[ww]);
        }
        r.x = r.si < (uint32_t)V ? __fsub_rn(__fmul_rn(bf2f(cb[r.si]), inv_t), M) : NEG_INF;
        r.pad[0] = r.pad[1] = 0;
        rec[b] = r;
    }
}

constexpr int FT = 1024;              // threads of the final workgroup
constexpr int FW = FT / 64;
constexpr int FPT = 65536 / FT;       // tokens a thread holds on the all-token path

/// block-wide sum, every thread getting the same value; buf is FW floats, the caller alternates
/// two buffers between calls so one barrier a call suffices
__device__ __forceinline__ float block_sum(float v, float* buf) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < FW; w++) s += buf[w];
    return s;
}

__device__ __forceinline__ void block_best(float& v, uint32_t& i, float* bv, uint32_t* bi) {
    wave_best(v, i);
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = v; bi[threadIdx.x >> 6] = i; }
    __syncthreads();
    v = bv[0];
    i = bi[0];
#pragma unroll
    for (int w = 1; w < FW; w++) best_of(v, i, bv[w], bi[w]);
}

__global__ __launch_bounds__(FT) void sample_final_kernel(const uint16_t* __restrict__ cb, int V, float inv_t, float top_p,
                                                          const float* __restrict__ bmax, int G, uint32_t key,
                                                          const BlockRec* __restrict__ rec, const uint32_t* __restrict__ cand,
                                                          uint32_t* token, uint32_t* greedy, int pos, int prompt) {
    // the candidates' e and words
    __shared__ float lds[2 * NCAND];
    float* ce = lds;
    uint32_t* cw = (uint32_t*)(lds + NCAND);
    __shared__ uint32_t off[65];
    __shared__ float red[2][FW];
    __shared__ float bv[FW];
    __shared__ uint32_t bix[FW];
    __shared__ float tot[3];
    __shared__ float ws_[64], wx_[64];   // the blocks' all-token Gumbel winners: score, x
    __shared__ uint32_t wi_[64];
    const int t = threadIdx.x, lane = t & 63;
    const float M = global_max(bmax, G);
    // the block records: wave 0 sums them and scans the candidate counts
    if (t < 64) {
        BlockRec r = {};
        if (lane < G) r = rec[lane];
        uint32_t incl = lane < G ? r.nc : 0;
        incl = wave_scan_incl(incl);
        off[lane + 1] = incl;
        if (lane == 0) off[0] = 0;
        float s = lane < G ? r.s : NEG_INF;
        uint32_t si = lane < G ? r.si : 0xFFFFFFFFu;
        ws_[lane] = s;
        wi_[lane] = si;
        wx_[lane] = lane < G ? r.x : NEG_INF;
        wave_best(s, si);
        const float z = wave_sum(lane < G ? r.z : 0.0f), cm = wave_sum(lane < G ? r.cm : 0.0f);
        if (lane == 0) { tot[0] = z; tot[1] = cm; tot[2] = s; bix[0] = si; }
    }
    __syncthreads();
    const float z = tot[0], cm = tot[1];
    const uint32_t nc = off[G];
    float lo = 0.0f;
    if (top_p < 1.0f) {
        const float want = __fmul_rn(top_p, z);
        float hi = 1.0f;
        if (nc <= (uint32_t)NCAND && cm >= want) {
            // gather the candidates: slot j belongs to the block whose range of off holds it
            for (uint32_t j = t; j < nc; j += FT) {
                int b0 = 0, b1 = G - 1;   // last block with off[b] <= j
                while (b0 < b1) {
                    const int mid = (b0 + b1 + 1) >> 1;
                    if (off[mid] <= j) b0 = mid; else b1 = mid - 1;
                }
                const uint32_t wd = cand[(size_t)b0 * SB + (j - off[b0])];
                cw[j] = wd;
                ce[j] = expf(__fsub_rn(__fmul_rn(bf2f((uint16_t)(wd & 0xFFFF)), inv_t), M));
            }
            __syncthreads();
            // the 20 bisection steps as 5 rounds of 4: in a round, wave w = 1..15 sums the kept mass
            // at node w of the next 4 levels' decision tree (heap order; a passed step, kept >= want,
            // goes to child 2w + 1), its midpoint the one the steps on its path compute; then every
            // thread walks the 4 levels. The decisions are the sequential bisection's.
            {
                const int w = t >> 6;
                float ev[NCAND / 64];
#pragma unroll
                for (int k = 0; k < NCAND / 64; k++) ev[k] = (uint32_t)(64 * k + lane) < nc ? ce[64 * k + lane] : 0.0f;
                lo = CMIN;
                for (int r = 0; r < 5; r++) {
                    if (w >= 1 && w < 16) {
                        float l2 = lo, h2 = hi;
                        const int depth = 31 - __clz(w);
                        for (int d = depth - 1; d >= 0; d--) {   // the path's decisions: the bits of w below its top
                            const float m = __fmul_rn(0.5f, __fadd_rn(l2, h2));
                            if ((w >> d) & 1) l2 = m; else h2 = m;
                        }
                        const float mid = __fmul_rn(0.5f, __fadd_rn(l2, h2));
                        float kept = 0.0f;
#pragma unroll
                        for (int k = 0; k < NCAND / 64; k++) kept += ev[k] >= mid ? ev[k] : 0.0f;
                        kept = wave_sum(kept);
                        if (lane == 0) red[r & 1][w] = kept;
                    }
                    __syncthreads();
                    int node = 1;
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const float mid = __fmul_rn(0.5f, __fadd_rn(lo, hi));
                        const bool pass = red[r & 1][node] >= want;
                        if (pass) lo = mid; else hi = mid;
                        node = 2 * node + (pass ? 1 : 0);
                    }
                }
            }
            const float floor_x = logf(lo);
            float best = NEG_INF;
            uint32_t bi = 0xFFFFFFFFu;
            for (uint32_t j = t; j < nc; j += FT) {
                const uint32_t wd = cw[j], i = wd >> 16;
                const float x = __fsub_rn(__fmul_rn(bf2f((uint16_t)(wd & 0xFFFF)), inv_t), M);
                if (x >= floor_x) best_of(best, bi, gumbel_score(x, key, i), i);
            }
            block_best(best, bi, bv, bix);
            if (t == 0) write_token(bi, token, greedy, pos, prompt);
            return;
        }
        // every token: the row's e in registers (64 a thread), token 4 t + 4096 q + k
        auto quad = [&](int q) {
            const int i0 = 4 * t + 4 * FT * q;
            if (i0 + 3 < V) return ld8(cb + i0);
            uint32_t h[4];
#pragma unroll
            for (int k = 0; k < 4; k++) h[k] = i0 + k < V ? cb[i0 + k] : 0;
            return (u2_t){h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        };
        float e[FPT];
#pragma unroll
        for (int q = 0; q < FPT / 4; q++) {
            const u2_t c2 = quad(q);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = 4 * t + 4 * FT * q + k;
                const uint16_t c = (uint16_t)(c2[k >> 1] >> (16 * (k & 1)));
                const float v = i < V ? expf(__fsub_rn(__fmul_rn(bf2f(c), inv_t), M)) : 0.0f;
                e[4 * q + k] = v;
            }
        }
        for (int it = 0; it < 20; it++) {
            const float mid = __fmul_rn(0.5f, __fadd_rn(lo, hi));
            float kept = 0.0f;
#pragma unroll
            for (int k = 0; k < FPT; k++) kept += e[k] >= mid ? e[k] : 0.0f;
            if (block_sum(kept, red[it & 1]) >= want) lo = mid; else hi = mid;
        }
        if (lo > 0.0f) {
            // a block's winner over all its tokens is its winner over its nucleus tokens when it
            // is in the nucleus itself; the other blocks are drawn again, a wave a block
            const float floor_x = logf(lo);
            const int w = t >> 6;
            float best = NEG_INF;
            uint32_t bi = 0xFFFFFFFFu;
            for (int b = w; b < G; b += FW) {
                if (wx_[b] >= floor_x) {
                    best_of(best, bi, ws_[b], wi_[b]);
                    continue;
                }
#pragma unroll
                for (int q = 0; q < SB / 256; q++) {
                    const int i0 = b * SB + 256 * q + 4 * lane;
                    u2_t c2;
                    if (i0 + 3 < V) c2 = ld8(cb + i0);
                    else {
                        uint32_t h[4];
#pragma unroll
                        for (int k = 0; k < 4; k++) h[k] = i0 + k < V ? cb[i0 + k] : 0;
                        c2 = (u2_t){h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
                    }
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int i = i0 + k;
                        const float x = __fsub_rn(__fmul_rn(bf2f((uint16_t)(c2[k >> 1] >> (16 * (k & 1)))), inv_t), M);
                        if (i < V && x >= floor_x) best_of(best, bi, gumbel_score(x, key, (uint32_t)i), (uint32_t)i);
                    }
                }
            }
            block_best(best, bi, bv, bix);
            if (t == 0) write_token(bi, token, greedy, pos, prompt);
            return;
        }
    }
    // threshold 0: every token is in the nucleus, and the draw is the best block winner
    if (t == 0) write_token(bix[0], token, greedy, pos, prompt);
}

int launch_argmax(const float* logits, int V, uint32_t* token, uint32_t* greedy, int pos, int prompt, char* ws,
                  hipStream_t st) {
    const int G = (V + SB - 1) / SB;
    float* bmax = (float*)(ws + sample_ws_off_blk(V));
    uint32_t* bidx = (uint32_t*)(bmax + 64);
    hipLaunchKernelGGL(logit_scan_kernel, dim3(G), dim3(256), 0, st, logits, V, 1.0f, (uint16_t*)nullptr, bmax, bidx);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, st, bmax, bidx, G, token, greedy, pos, prompt);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

int launch_sample(const float* logits, int V, uint32_t* token, uint32_t* greedy, int pos, int prompt, float inv_t,
                  float top_p, uint32_t seed, char* ws, hipStream_t st) {
    const int G = (V + SB - 1) / SB;
    uint16_t* cb = (uint16_t*)ws;
    float* bmax = (float*)(ws + sample_ws_off_blk(V));
    uint32_t* bidx = (uint32_t*)(bmax + 64);
    BlockRec* rec = (BlockRec*)(bidx + 64);
    uint32_t* cand = (uint32_t*)(ws + sample_ws_off_cand(V));
    const uint32_t key = mix32(seed ^ mix32((uint32_t)pos * 0x9e3779b9u));   // misc.metal:276
    hipLaunchKernelGGL(logit_scan_kernel, dim3(G), dim3(256), 0, st, logits, V, inv_t, cb, bmax, bidx);
    hipLaunchKernelGGL(sample_weights_kernel, dim3(G), dim3(256), 0, st, cb, V, inv_t, bmax, G, key, rec, cand);
    hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(FT), 0, st, cb, V, inv_t, top_p, bmax, G, key, rec, cand,
                       token, greedy, pos, prompt);
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
