/* oracle.c — CPU restatement of the reference's attention math. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker the parity tests (tests/), __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg compare the HIP library against. Nothing in the product path links or calls
 * it. It restates, in plain fp32 C on logical row-major layouts, the math of:
 *   Sources/EmblaMetal/Kernels/common.metal:13-26 (head_norm), 28-37 (rope), 72-84 (write_row8)
 *   Sources/EmblaMetal/Kernels/attention.metal:26-102 (attn_sliding), 113-140 (kv_append),
 *     148-220 / 235-363 (attn_full, attn_full8: ReLU² + sink, SCORES),
 *     370-441 / 448-584 (attn_sparse, attn_sparse8: softmax, SEL), 655-744 (select_keys)
 *   Sources/EmblaMetal/Kernels/prefill.metal:127-180, 428-548 (sliding prefill),
 *     214-282 (attn_full_b); attn_nax.metal:61-364 (causal ReLU² prefill)
 *   Sources/EmblaMetal/Kernels/gemv.metal:1-92, gemm.metal:1-134, common.metal:104-152 (the
 *     4-bit projections either side of attention: y = W x with MLX's affine 4-bit layout)
 *   Sources/EmblaMetal/Kernels/misc.metal:83-128 (argmax), 164-298 (sample: the top-p nucleus by
 *     bisection and the Gumbel-max draw)
 * and the BASELINE configs' variants of them (softmax full layers, fp16 scales, 4 kv heads,
 * window 1024, the ReLU² index scorer  score_j = Σ_h w_h relu(q_h·k_j)²).
 *
 * Pinning (tests/test_oracle.py): the reference ships no golden vectors for attention and cannot
 * be built here (Swift + Metal), so every function is checked against an independent numpy fp64
 * brute force, closed forms and invariants; the integer outputs (int8 bytes, top-k index sets)
 * against their definitions. Compile: see oracle/Makefile (-O2 -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HD 128
#define EPS32 1.1920929e-07f

/* ------------------------------------------------------------------ element types */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* RNE, as BFloat16.swift:4-9 */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}
static float bf(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

float orc_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else { /* subnormal: m * 2^-24 */
            float f = ldexpf((float)m, -24);
            memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) u = s | 0x7F800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* IEEE binary16, round to nearest even */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000);
    const float a = fabsf(f);
    if (a != a) return s | 0x7E00;
    if (a >= 65520.0f) return s | 0x7C00;
    if (a < 6.103515625e-05f) { /* subnormal range: quantum 2^-24 */
        const float q = nearbyintf(a * 16777216.0f); /* exact scaling, RNE */
        return s | (uint16_t)q;
    }
    uint32_t au;
    memcpy(&au, &a, 4);
    const uint32_t e = (au >> 23) - 112, m = au & 0x7FFFFF;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return s | (uint16_t)h;
}

/* ------------------------------------------------------------------ row helpers */
/* Σx² of a 128-dim row in the fixed order the GPU kernels use: lane l (0..63) holds dims 2l,
 * 2l+1 and sums their squares, then lanes combine pairwise (xor 32, 16, .., 1). */
static float sumsq_bfly(const float* x) {
    float v[64], t[64];
    for (int l = 0; l < 64; l++) {
        const float a = x[2 * l] * x[2 * l], b = x[2 * l + 1] * x[2 * l + 1];
        v[l] = a + b;
    }
    for (int m = 32; m >= 1; m >>= 1) {
        for (int l = 0; l < 64; l++) t[l] = v[l] + v[l ^ m];
        memcpy(v, t, sizeof v);
    }
    return v[0];
}

/* head_norm (common.metal:13-26): x * r * (1 + g1) * (1 + g2) for the first ng gains,
 * r = 1 / sqrt(Σx² / 128 + 2^-23); then rounded to bf16 when round_bf is set. */
void orc_head_norm(const float* x, const float* g1, const float* g2, int ng, int round_bf, float* out) {
    const float r = 1.0f / sqrtf(sumsq_bfly(x) / 128.0f + EPS32);
    for (int d = 0; d < HD; d++) {
        float g = r;
        if (ng >= 1) g = g * (1.0f + g1[d]);
        if (ng >= 2) g = g * (1.0f + g2[d]);
        const float y = x[d] * g;
        out[d] = round_bf ? bf(y) : y;
    }
}

/* RoPE as common.metal:39-47: dims d and d + 32 (d < 32) rotate by theta = -pos * f_d with
 * f_d = 10000^(-d/32). The spec fixes the rounding: f_d is the fp32 nearest to the exact value (a
 * table), theta is the fp32 product -(float)pos * f_d, and cos/sin are taken of that fp32 theta. */
float orc_rope_freq(int d) { return (float)exp2(-(double)d / 32.0 * 13.287712379549449); }
void orc_rope(float* x, int pos) {
    for (int d = 0; d < 32; d++) {
        const float th = -(float)pos * orc_rope_freq(d);
        const float c = (float)cos((double)th), s = (float)sin((double)th);
        const float x1 = x[d], x2 = x[d + 32];
        x[d] = x1 * c - x2 * s;
        x[d + 32] = x1 * s + x2 * c;
    }
}

/* write_row8 (common.metal:72-84) on one row: v = x (bf16-rounded when round_bf), a = max|v|,
 * q = rint(v * (127 / a)) (0 when a = 0), scale = a / 127. With norm, x is first RMS-normed
 * without gains (kv_append, attention.metal:128). */
void orc_quant_row(const float* x_in, int norm, int round_bf, int8_t* q, float* scale) {
    float x[HD];
    if (norm) {
        const float r = 1.0f / sqrtf(sumsq_bfly(x_in) / 128.0f + EPS32);
        for (int d = 0; d < HD; d++) x[d] = x_in[d] * r;
    } else {
        memcpy(x, x_in, sizeof x);
    }
    float a = 0.0f;
    for (int d = 0; d < HD; d++) {
        if (round_bf) x[d] = bf(x[d]);
        a = fmaxf(a, fabsf(x[d]));
    }
    const float inv = a > 0.0f ? 127.0f / a : 0.0f;
    for (int d = 0; d < HD; d++) q[d] = (int8_t)(int)rintf(x[d] * inv);
    *scale = a / 127.0f;
}

/* ------------------------------------------------------------------ decode over an int8 cache
 * q [n_q][128] fp32 (prepared); K, V int8 [n_kv][S][128] logical rows with scales ks, vs
 * [n_kv][S] (already converted to fp32 from their stored dtype); query head h uses kv head
 * h / (n_q / n_kv). weights 0: softmax(q·k·ks / √128) over V·vs (attn_sparse KV8,
 * attention.metal:401-441). weights 1: w = relu(q·k·ks / √128)², o = Σ w·vs·v / (√128 + Σ w)
 * (attn_full8, attention.metal:280-363). scores (optional, [n_kv][S]): max over the kv head's
 * query heads of q·k·ks (attention.metal:295-305). rows (optional, [n_kv][S_sel]): attend only
 * those rows (SEL), S then counts selected rows. */
void orc_decode_int8(const float* q, const int8_t* K, const float* ks, const int8_t* V, const float* vs,
                     int S, int S_cache, int n_q, int n_kv, int weights, const uint32_t* rows,
                     float* out, float* scores) {
    const int gq = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)HD);
    if (scores)
        for (int i = 0; i < n_kv * S_cache; i++) scores[i] = -INFINITY;
    /* heads are independent (the OpenMP build splits them over threads; with scores, whose
     * maxima several heads update, it stays serial) */
#pragma omp parallel for schedule(static) if (!scores)
    for (int h = 0; h < n_q; h++) {
        const int kvh = h / gq;
        const float* qh = q + (size_t)h * HD;
        float m = -INFINITY, l = 0.0f, acc[HD];
        memset(acc, 0, sizeof acc);
        for (int j = 0; j < S; j++) {
            const size_t r = rows ? rows[(size_t)kvh * S + j] : (size_t)j;
            const int8_t* kr = K + ((size_t)kvh * S_cache + r) * HD;
            const int8_t* vr = V + ((size_t)kvh * S_cache + r) * HD;
            float dot = 0.0f;
            for (int d = 0; d < HD; d++) dot += qh[d] * (float)kr[d];
            const float s = dot * ks[(size_t)kvh * S_cache + r];
            const float vsc = vs[(size_t)kvh * S_cache + r];
            if (scores) {
                float* sp = scores + (size_t)kvh * S_cache + r;
                if (s > *sp) *sp = s;
            }
            if (weights == 1) {
                const float a = fmaxf(s * scale, 0.0f), w = a * a;
                if (w != 0.0f) {
                    l += w;
                    for (int d = 0; d < HD; d++) acc[d] += w * vsc * (float)vr[d];
                }
            } else {
                const float x = s * scale, mn = fmaxf(m, x);
                const float cf = expf(m - mn), p = expf(x - mn);
                l = l * cf + p;
                for (int d = 0; d < HD; d++) acc[d] = acc[d] * cf + p * vsc * (float)vr[d];
                m = mn;
            }
        }
        const float den = weights == 1 ? sqrtf((float)HD) + l : l;
        for (int d = 0; d < HD; d++) out[(size_t)h * HD + d] = acc[d] / den;
    }
}

/* ------------------------------------------------------------------ decode over a bf16 cache
 * The full layers' caches without KV8 (bf16 rows, no scales; the rows passed here as their fp32
 * values [n_kv][S_cache][128]): attn_full (attention.metal:148-220) with weights 1, ReLU² over
 * s = q·k: w = relu(s / √128)², o = Σ w·v / (√128 + Σ w), scores (optional, [n_kv][S_cache]) the
 * max over the kv head's query heads of the raw s (attention.metal:183, 193-202); attn_sparse
 * (attention.metal:370-441) with weights 0, softmax of s / √128. rows (optional, [n_kv][S]):
 * attend only those rows (SEL). The same arithmetic as orc_decode_int8 with unit scales. */
void orc_decode_f32(const float* q, const float* K, const float* V, int S, int S_cache, int n_q, int n_kv,
                    int weights, const uint32_t* rows, float* out, float* scores) {
    const int gq = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)HD);
    if (scores)
        for (int i = 0; i < n_kv * S_cache; i++) scores[i] = -INFINITY;
#pragma omp parallel for schedule(static) if (!scores)
    for (int h = 0; h < n_q; h++) {
        const int kvh = h / gq;
        const float* qh = q + (size_t)h * HD;
        float m = -INFINITY, l = 0.0f, acc[HD];
        memset(acc, 0, sizeof acc);
        for (int j = 0; j < S; j++) {
            const size_t r = rows ? rows[(size_t)kvh * S + j] : (size_t)j;
            const float* kr = K + ((size_t)kvh * S_cache + r) * HD;
            const float* vr = V + ((size_t)kvh * S_cache + r) * HD;
            float dot = 0.0f;
            for (int d = 0; d < HD; d++) dot += qh[d] * kr[d];
            if (scores) {
                float* sp = scores + (size_t)kvh * S_cache + r;
                if (dot > *sp) *sp = dot;
            }
            if (weights == 1) {
                const float a = fmaxf(dot * scale, 0.0f), w = a * a;
                if (w != 0.0f) {
                    l += w;
                    for (int d = 0; d < HD; d++) acc[d] += w * vr[d];
                }
            } else {
                const float x = dot * scale, mn = fmaxf(m, x);
                const float cf = expf(m - mn), p = expf(x - mn);
                l = l * cf + p;
                for (int d = 0; d < HD; d++) acc[d] = acc[d] * cf + p * vr[d];
                m = mn;
            }
        }
        const float den = weights == 1 ? sqrtf((float)HD) + l : l;
        for (int d = 0; d < HD; d++) out[(size_t)h * HD + d] = acc[d] / den;
    }
}

/* ------------------------------------------------------------------ decode over 16-bit K/V
 * Softmax over explicit float K/V rows [n_kv][S_cache][128] at positions pos[j] (j < n): the
 * sliding window (attn_sliding, attention.metal:63-101: keys pos-n+1 .. pos) and the sparse
 * layers' gathered keys (C4) are both this with different position lists. pos_list is
 * [n_kv][n] or shared ([n], per_head = 0). */
void orc_decode_rows(const float* q, const float* K, const float* V, int S_cache, int n_q, int n_kv,
                     const int32_t* pos_list, int n, int per_head, float* out) {
    const int gq = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)HD);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_q; h++) {
        const int kvh = h / gq;
        const int32_t* pl = pos_list + (per_head ? (size_t)kvh * n : 0);
        float m = -INFINITY, l = 0.0f, acc[HD];
        memset(acc, 0, sizeof acc);
        for (int j = 0; j < n; j++) {
            const float* kr = K + ((size_t)kvh * S_cache + pl[j]) * HD;
            const float* vr = V + ((size_t)kvh * S_cache + pl[j]) * HD;
            float dot = 0.0f;
            for (int d = 0; d < HD; d++) dot += q[(size_t)h * HD + d] * kr[d];
            const float x = dot * scale, mn = fmaxf(m, x);
            const float cf = expf(m - mn), p = expf(x - mn);
            l = l * cf + p;
            for (int d = 0; d < HD; d++) acc[d] = acc[d] * cf + p * vr[d];
            m = mn;
        }
        for (int d = 0; d < HD; d++) out[(size_t)h * HD + d] = acc[d] / l;
    }
}

/* ------------------------------------------------------------------ key selection */
/* order_bits (attention.metal:657-660): float -> uint with the same order. */
uint32_t orc_order_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static int cmp_desc_u32(const void* a, const void* b) {
    const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? 1 : x > y ? -1 : 0;
}

/* select_keys (attention.metal:680-744) for one set: among keys [0, n = S - recent) the topk with
 * the highest order_bits(score); out[0 .. ngt) = keys above the topk-th largest value in index
 * order, then the first (topk - ngt) keys equal to it in index order, then n .. S-1. S must be
 * > topk + recent. */
void orc_select_keys(const float* sc, int S, int topk, int recent, uint32_t* out) {
    const int n = S - recent;
    uint32_t* b = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    for (int j = 0; j < n; j++) b[j] = orc_order_bits(sc[j]);
    qsort(b, (size_t)n, sizeof(uint32_t), cmp_desc_u32);
    const uint32_t kth = b[topk - 1];
    free(b);
    int g = 0, ngt = 0;
    for (int j = 0; j < n; j++) ngt += orc_order_bits(sc[j]) > kth;
    int e = ngt;
    for (int j = 0; j < n; j++) {
        const uint32_t v = orc_order_bits(sc[j]);
        if (v > kth) out[g++] = (uint32_t)j;
        else if (v == kth && e < topk) out[e++] = (uint32_t)j;
    }
    for (int j = 0; j < recent; j++) out[topk + j] = (uint32_t)(n + j);
}

/* ------------------------------------------------------------------ index scorer (C4/C5)
 * score_j = Σ_h w_h relu(q_h·k_j)², fp16 q [n_ih][64], k [n][64], w [n_ih] fp32, in the fixed fp32
 * order the spec gives (and the GPU kernel, select.hip, implements): 8 partial dots c_k, each an
 * fma chain over dims 8k .. 8k+7 from 0 (fp16 products are exact in fp32, so each step is one
 * rounding); dot = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)); r = max(dot, 0); then
 * s = fma(w_h, r * r, s) over h = 0 .. from s = 0. */
void orc_index_scores(const uint16_t* qi, const float* w, const uint16_t* ki, int n, int n_ih,
                      float* out) {
    float qf[16 * 64];
    for (int i = 0; i < n_ih * 64; i++) qf[i] = orc_f16_to_f32(qi[i]);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < n; j++) {
        float kf[64];
        for (int d = 0; d < 64; d++) kf[d] = orc_f16_to_f32(ki[(size_t)j * 64 + d]);
        float s = 0.0f;
        for (int h = 0; h < n_ih; h++) {
            float c[8];
            for (int k = 0; k < 8; k++) {
                float acc = 0.0f;
                for (int d = 8 * k; d < 8 * k + 8; d++) acc = fmaf(qf[h * 64 + d], kf[d], acc);
                c[k] = acc;
            }
            const float s01 = c[0] + c[1], s23 = c[2] + c[3], s45 = c[4] + c[5], s67 = c[6] + c[7];
            const float s03 = s01 + s23, s47 = s45 + s67;
            const float dot = s03 + s47;
            const float r = fmaxf(dot, 0.0f);
            const float r2 = r * r;
            s = fmaf(w[h], r2, s);
        }
        out[j] = s;
    }
}

/* ------------------------------------------------------------------ prefill over an int8 cache
 * Rows i = 0 .. T-1 at positions p0 + i attend keys [lo_i, p0 + i] with lo_i = 0 (causal) or
 * p0 + i - window + 1 (window > 0); q [T][n_q][128] fp32; K/V int8 logical rows [n_kv][S_cache][128]
 * with scales. weights as orc_decode_int8 (attn_nax.metal:231-357 for ReLU²: p = relu(s·scale)²,
 * out = Σp·vs·v / (√128 + Σp)). rows_sel (optional, [T][nsel]): the keys of row i are exactly
 * rows_sel[i] (the sparse layer). */
void orc_prefill_int8(const float* q, const int8_t* K, const float* ks, const int8_t* V, const float* vs,
                      int T, int p0, int S_cache, int n_q, int n_kv, int weights, int window,
                      const uint32_t* rows_sel, int nsel, float* out) {
    const int gq = n_q / n_kv;
    const float scale = 1.0f / sqrtf((float)HD);
#pragma omp parallel for schedule(dynamic)
    for (int i = 0; i < T; i++) {
        const int pos = p0 + i;
        const int lo = window > 0 ? (pos - window + 1 > 0 ? pos - window + 1 : 0) : 0;
        const int n = rows_sel ? nsel : pos - lo + 1;
        for (int h = 0; h < n_q; h++) {
            const int kvh = h / gq;
            const float* qh = q + ((size_t)i * n_q + h) * HD;
            float m = -INFINITY, l = 0.0f, acc[HD];
            memset(acc, 0, sizeof acc);
            for (int jj = 0; jj < n; jj++) {
                const size_t j = rows_sel ? rows_sel[(size_t)i * nsel + jj] : (size_t)(lo + jj);
                const int8_t* kr = K + ((size_t)kvh * S_cache + j) * HD;
                const int8_t* vr = V + ((size_t)kvh * S_cache + j) * HD;
                float dot = 0.0f;
                for (int d = 0; d < HD; d++) dot += qh[d] * (float)kr[d];
                const float s = dot * ks[(size_t)kvh * S_cache + j] * scale;
                const float vsc = vs[(size_t)kvh * S_cache + j];
                if (weights == 1) {
                    const float a = fmaxf(s, 0.0f), w = a * a;
                    l += w;
                    for (int d = 0; d < HD; d++) acc[d] += w * vsc * (float)vr[d];
                } else {
                    const float mn = fmaxf(m, s), cf = expf(m - mn), p = expf(s - mn);
                    l = l * cf + p;
                    for (int d = 0; d < HD; d++) acc[d] = acc[d] * cf + p * vsc * (float)vr[d];
                    m = mn;
                }
            }
            const float den = weights == 1 ? sqrtf((float)HD) + l : l;
            for (int d = 0; d < HD; d++) out[((size_t)i * n_q + h) * HD + d] = acc[d] / den;
        }
    }
}

/* ------------------------------------------------------------------ 4-bit projections */
/* y = W x of one token (gemv.metal:36-92 with MIX = 0; gemm.metal:1-134 row by row for T tokens),
 * W in MLX's affine 4-bit layout (gemm.metal:1-3; common.metal:105-152): words [O][K/8], nibble q
 * of word c (bits 4q .. 4q+3) the weight of column 8c + q; scales and biases bf16 [O][K/64]
 * (group g = columns 64g .. 64g+63); w = s * nibble + b. The dot product accumulates in double
 * (the GPU's fp32 sums in its own order are compared within tolerance), then the epilogue
 * (gemv.metal:77-88): 0 y = bf16(acc), 1 y = bf16(relu(bf16(acc))^2), 2 y += bf16(acc) (y fp32),
 * 3 y = bf16(acc) (fp32), 4 y = acc. Outputs are written as floats (bf16 values exactly). */
void orc_q4_matvec(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x, int O, int K,
                   int epi, float* y) {
    for (int r = 0; r < O; r++) {
        double acc = 0.0;
        for (int c = 0; c < K; c++) {
            const uint32_t q = (w[(size_t)r * (K / 8) + c / 8] >> (4 * (c % 8))) & 0xFu;
            const double wt = (double)orc_bf16_to_f32(s[(size_t)r * (K / 64) + c / 64]) * q +
                              (double)orc_bf16_to_f32(b[(size_t)r * (K / 64) + c / 64]);
            acc += wt * (double)orc_bf16_to_f32(x[c]);
        }
        const float a = (float)acc;
        switch (epi) {
            case 0: y[r] = bf(a); break;
            case 1: { const float v = fmaxf(bf(a), 0.0f); y[r] = bf(v * v); break; }
            case 2: y[r] += bf(a); break;
            case 3: y[r] = bf(a); break;
            default: y[r] = a; break;
        }
    }
}

/* ------------------------------------------------------------------ sampling tail
 * misc.metal:83-128 (argmax) and 164-298 (sample). */

/* The softcap of one logit as the reference computes it: bf(bf(tanh(bf(bf(l) / 15))) * 15)
 * (misc.metal:101, 216). tanh in fp64 rounded once to fp32: the correctly rounded fp32 tanh that
 * precise::tanh approximates. */
float orc_softcap(float l) {
    const float y = bf(bf(l) / 15.0f);
    const float t = (float)tanh((double)y);
    return bf(bf(t) * 15.0f);
}

/* The first index of the largest softcapped logit (misc.metal:99-121). */
uint32_t orc_argmax(const float* logits, int V) {
    float best = -INFINITY;
    uint32_t idx = 0;
    for (int i = 0; i < V; i++) {
        const float c = orc_softcap(logits[i]);
        if (c > best) { best = c; idx = (uint32_t)i; }
    }
    return idx;
}

/* The 32-bit integer mix of misc.metal:186-191 (the "lowbias32" finaliser: xorshift-multiply
 * rounds with the constants 0x7feb352d and 0x846ca68b). */
uint32_t orc_mix32(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352du;
    x ^= x >> 15; x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

/* Gumbel noise of token i for a step key: -log(-log(u)), u in (0, 1) from the hash's top 24 bits
 * (misc.metal:278-281). */
static float gumbel_g(uint32_t key, uint32_t i) {
    const float u = ((float)(orc_mix32(key ^ i) >> 8) + 0.5f) * (1.0f / 16777216.0f);
    return logf(-logf(u));
}

static double rel(double a, double b) { return fabs(a - b) / (fabs(b) > 1e-30 ? fabs(b) : 1e-30); }
/* a within 2 fp32 ulps of b: an exp or log that differs by an ulp may order them otherwise */
static int near2(float a, float b) { return fabs((double)a - b) <= 2.0 * ((double)nextafterf(fabsf(b), INFINITY) - fabsf(b)); }

/* The token misc.metal:196-298 draws at position pos: softmax(softcap(l) / T) cut to its top-p
 * nucleus by bisection on exp(x) (over the tokens with exp(x) >= 1/16384 when they are at most 2048
 * and hold top-p of the mass, else over all), then the argmax of x + Gumbel noise over the nucleus.
 * Sums are in fp64 (the reference's are fp32 in an unspecified order). *fragile is set when a
 * decision of the draw lies within floating-point error of its boundary (a sum within 2e-5 of
 * top-p's mass, relative: above the error of an fp32 sum of 65536 terms by blocks and trees; an
 * exp(x) within 2 ulps of a threshold it is compared with; an x within 2 ulps of the nucleus
 * floor; the two best Gumbel scores unequal and within 1e-5): an implementation
 * that sums in another order or whose exp/log differ by an ulp may then draw another token. Equal
 * best scores are no hazard: they come from one x and one hash value, equal everywhere, and the
 * lower index wins. */
static float sample_threshold(const float* logits, int V, float inv_t, float top_p, float* x, int* fragile) {
    const float CMIN = 1.0f / 16384.0f;
    float* e = (float*)malloc(sizeof(float) * (size_t)V);
    float mx = -INFINITY;
    for (int i = 0; i < V; i++) {
        x[i] = orc_softcap(logits[i]) * inv_t;
        mx = fmaxf(mx, x[i]);
    }
    double z = 0.0;
    for (int i = 0; i < V; i++) {
        x[i] = x[i] - mx;
        e[i] = expf(x[i]);
        z += e[i];
    }
    int frag = 0;
    float lo = 0.0f;
    if (top_p < 1.0f) {
        const float want = top_p * (float)z;
        int nc = 0;
        double cm = 0.0;
        for (int i = 0; i < V; i++) {
            if (near2(e[i], CMIN)) frag = 1;
            if (e[i] >= CMIN) { nc++; cm += e[i]; }
        }
        float hi = 1.0f;
        const int cand = nc <= 2048 && cm >= want;
        if (nc <= 2048 && rel(cm, want) < 2e-5) frag = 1;
        lo = cand ? CMIN : 0.0f;
        for (int it = 0; it < 20; it++) {
            const float mid = 0.5f * (lo + hi);
            double kept = 0.0;
            for (int i = 0; i < V; i++) {
                if (cand && e[i] < CMIN) continue;
                if (near2(e[i], mid)) frag = 1;
                kept += e[i] >= mid ? e[i] : 0.0f;
            }
            if (rel(kept, want) < 2e-5) frag = 1;
            if (kept >= want) lo = mid; else hi = mid;
        }
    }
    free(e);
    *fragile = frag;
    return lo;
}

/* The draw at pos given x and the threshold lo (misc.metal:274-298). */
static uint32_t sample_draw(const float* x, int V, float lo, int pos, uint32_t seed, int* fragile) {
    int frag = 0;
    const float floor_x = lo > 0.0f ? logf(lo) : -INFINITY;
    const uint32_t key = orc_mix32(seed ^ orc_mix32((uint32_t)pos * 0x9e3779b9u));
    float best = -INFINITY, second = -INFINITY;
    uint32_t idx = 0;
    for (int i = 0; i < V; i++) {
        if (lo > 0.0f && near2(x[i], floor_x)) frag = 1;
        if (x[i] < floor_x) continue;
        const float sc = x[i] - gumbel_g(key, (uint32_t)i);
        if (sc > best) { second = best; best = sc; idx = (uint32_t)i; }
        else if (sc > second) second = sc;
    }
    if (best > second && best - second < 1e-5 * fmax(1.0, fabs(best))) frag = 1;
    *fragile = frag;
    return idx;
}

uint32_t orc_sample(const float* logits, int V, int pos, float inv_t, float top_p, uint32_t seed, int* fragile) {
    float* x = (float*)malloc(sizeof(float) * (size_t)V);
    int f1 = 0, f2 = 0;
    const float lo = sample_threshold(logits, V, inv_t, top_p, x, &f1);
    const uint32_t tok = sample_draw(x, V, lo, pos, seed, &f2);
    free(x);
    if (fragile) *fragile = f1 | f2;
    return tok;
}

/* Draws at positions pos0 .. pos0 + n - 1 of one row of logits (the threshold does not depend on
 * the position). */
void orc_sample_many(const float* logits, int V, int pos0, int n, float inv_t, float top_p, uint32_t seed,
                     uint32_t* tokens, int32_t* fragile) {
    float* x = (float*)malloc(sizeof(float) * (size_t)V);
    int f1 = 0;
    const float lo = sample_threshold(logits, V, inv_t, top_p, x, &f1);
    for (int k = 0; k < n; k++) {
        int f2 = 0;
        tokens[k] = sample_draw(x, V, lo, pos0 + k, seed, &f2);
        fragile[k] = f1 | f2;
    }
    free(x);
}
