// The C++ attention engine (Engine.encodeAttention's mirror) over a three-layer stack on the GPU,
// every stage checked against the C oracle on the GPU's own inputs to that stage.
//
// Layers as the reference arranges a block (Engine.swift:441-485): 0 sliding (4 kv heads, bf16
// ring of 4096, window 128), 1 full (2 kv heads, int8 cache with fp32 scales, ReLU² with sink; it
// scores and selects for the sparse layers), 2 sparse (softmax over its block's full-layer cache;
// the selected 1024 + 128 rows once keys pass 1152). One token a step from position 0; at the
// checked positions each layer's q/k/v projection, k/v append (bytes and scales, bit for bit),
// attention output, scores and selection (bit for bit), ring row and residual are compared with
// oracle/oracle.c; then the engine's prefix-block save/restore and token step. Then the prefill
// mirror (PrefillEncoder, Prefill.encode) against the decode path (prefill row i equals decode at
// p0 + i, as the reference designs it, Prefill.swift:10-13):
// a sliding and a full layer prefilled in two chunks (the second over the first's prefix) and
// decoded token by token into separate caches give the same residuals and caches. Exit status 0
// when every check passes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "attention_engine.hpp"
#include "common.hpp"   // the cache tile offsets (host-callable)

extern "C" {
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float f);
void orc_head_norm(const float* x, const float* g1, const float* g2, int ng, int round_bf, float* out);
void orc_rope(float* x, int pos);
void orc_quant_row(const float* x_in, int norm, int round_bf, int8_t* q, float* scale);
void orc_decode_int8(const float* q, const int8_t* K, const float* ks, const int8_t* V, const float* vs, int S,
                     int S_cache, int n_q, int n_kv, int weights, const uint32_t* rows, float* out, float* scores);
void orc_decode_f32(const float* q, const float* K, const float* V, int S, int S_cache, int n_q, int n_kv, int weights,
                    const uint32_t* rows, float* out, float* scores);
void orc_decode_rows(const float* q, const float* K, const float* V, int S_cache, int n_q, int n_kv,
                     const int32_t* pos_list, int n, int per_head, float* out);
void orc_select_keys(const float* sc, int S, int topk, int recent, uint32_t* out);
void orc_q4_matvec(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x, int O, int K,
                   int epi, float* y);
uint32_t orc_argmax(const float* logits, int V);
uint32_t orc_sample(const float* logits, int V, int pos, float inv_t, float top_p, uint32_t seed, int* fragile);
}

using embla_host::AttentionEngine;
using embla_host::Layer;
using embla_host::LayerKind;
using embla_host::PrefillEncoder;

namespace {

constexpr int D = 2048, HDIM = 128, MAXS = 2048, RING = 4096, WINDOW = 128, NSEL = 1152;

#define HIPCHECK(x)                                                                  \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                            \
        }                                                                            \
    } while (0)

struct SplitMix64 {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
    double normal() {   // Box-Muller
        const double u1 = uniform() + 1e-300, u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

float bf(uint16_t b) { return orc_bf16_to_f32(b); }
uint16_t tobf(float f) { return orc_f32_to_bf16(f); }

int failures = 0, checks = 0;
void expect(bool ok, const char* what, int pos, int layer) {
    ++checks;
    if (!ok) {
        ++failures;
        std::printf("FAIL pos %d layer %d: %s\n", pos, layer, what);
    }
}

/// |got - ref| <= atol + rtol |ref| everywhere; reports the worst element
bool close(const float* got, const float* ref, int n, float atol, float rtol, float* worst) {
    bool ok = true;
    *worst = 0.0f;
    for (int i = 0; i < n; i++) {
        const float e = std::fabs(got[i] - ref[i]);
        if (!(e <= atol + rtol * std::fabs(ref[i]))) ok = false;
        if (e > *worst || std::isnan(e)) *worst = e;
    }
    return ok;
}

/// A 4-bit matrix of O rows x D inputs in MLX's layout, kept on the host for the oracle.
struct Mat {
    int O;
    size_t w, s, b;   // byte offsets in the weight blob
};

struct Blob {
    std::vector<uint8_t> bytes;
    size_t add(size_t n) {
        const size_t at = (bytes.size() + 255) / 256 * 256;
        bytes.resize(at + n);
        return at;
    }
};

Mat add_mat(Blob& W, SplitMix64& g, int O) {
    Mat m{O, 0, 0, 0};
    m.w = W.add((size_t)O * D / 2);
    m.s = W.add((size_t)O * (D / 64) * 2);
    m.b = W.add((size_t)O * (D / 64) * 2);
    for (size_t i = 0; i < (size_t)O * D / 2; i++) W.bytes[m.w + i] = (uint8_t)(g.next() & 0xFF);
    for (size_t i = 0; i < (size_t)O * (D / 64); i++) {
        const float s = 0.004f + 0.004f * (float)g.uniform();
        const uint16_t sb = tobf(s), bb = tobf(-7.5f * bf(sb));
        std::memcpy(&W.bytes[m.s + 2 * i], &sb, 2);
        std::memcpy(&W.bytes[m.b + 2 * i], &bb, 2);
    }
    return m;
}

size_t add_gain(Blob& W, SplitMix64& g) {
    const size_t at = W.add(HDIM * 2);
    for (int i = 0; i < HDIM; i++) {
        const uint16_t v = tobf((float)(0.1 * g.normal()));
        std::memcpy(&W.bytes[at + 2 * i], &v, 2);
    }
    return at;
}

EmblaSeg seg(const Mat& m, unsigned end, unsigned x, unsigned y) {
    EmblaSeg s{};
    s.w = m.w;
    s.s = m.s;
    s.b = m.b;
    s.end = end;
    s.x = x;
    s.y = y;
    return s;
}

/// The oracle's y = W x for one matrix (epi as the library's), x bf16 [D].
void matvec(const Blob& W, const Mat& m, const uint16_t* x, int epi, float* y) {
    orc_q4_matvec((const uint32_t*)&W.bytes[m.w], (const uint16_t*)&W.bytes[m.s], (const uint16_t*)&W.bytes[m.b], x, m.O,
                  D, epi, y);
}

void gain_f32(const Blob& W, size_t at, float* out) {
    for (int i = 0; i < HDIM; i++) {
        uint16_t v;
        std::memcpy(&v, &W.bytes[at + 2 * i], 2);
        out[i] = bf(v);
    }
}

/// An int8 region (tile layout, fp32 scales) read back as row-major rows and scales.
void read_int8_region(const std::vector<uint8_t>& cache, size_t off, bool is_v, int n_kv, std::vector<int8_t>& rows,
                      std::vector<float>& sc) {
    rows.assign((size_t)n_kv * MAXS * HDIM, 0);
    sc.assign((size_t)n_kv * MAXS, 0.0f);
    for (int h = 0; h < n_kv; h++)
        for (int j = 0; j < MAXS; j++) {
            for (int d = 0; d < HDIM; d++) {
                const size_t o = is_v ? embla::vt_off(h, MAXS, j, d, 1) : embla::kt_off(h, MAXS, j, d, 1);
                rows[((size_t)h * MAXS + j) * HDIM + d] = (int8_t)cache[off + o];
            }
            std::memcpy(&sc[(size_t)h * MAXS + j], &cache[off + (size_t)n_kv * MAXS * HDIM + ((size_t)h * MAXS + j) * 4], 4);
        }
}

/// A 16-bit region (tile layout, ES 2) of n_kv heads x S slots read back as fp32 rows
/// [n_kv][S][128] and raw bits: a bf16 ring, or a bf16 full-layer cache.
void read16(const std::vector<uint8_t>& cache, size_t off, bool is_v, int n_kv, int S, std::vector<float>& rows,
            std::vector<uint16_t>& bits) {
    rows.assign((size_t)n_kv * S * HDIM, 0.0f);
    bits.assign((size_t)n_kv * S * HDIM, 0);
    for (int h = 0; h < n_kv; h++)
        for (int j = 0; j < S; j++)
            for (int d = 0; d < HDIM; d++) {
                const size_t o = is_v ? embla::vt_off(h, S, j, d, 2) : embla::kt_off(h, S, j, d, 2);
                uint16_t v;
                std::memcpy(&v, &cache[off + o], 2);
                bits[((size_t)h * S + j) * HDIM + d] = v;
                rows[((size_t)h * S + j) * HDIM + d] = bf(v);
            }
}

/// A bf16 ring (4 kv heads x RING slots) read back as fp32 rows and raw bits.
void read_ring(const std::vector<uint8_t>& cache, size_t off, bool is_v, std::vector<float>& rows,
               std::vector<uint16_t>& bits) {
    read16(cache, off, is_v, 4, RING, rows, bits);
}

}  // namespace

/// The full (li 1: append bytes, ReLU² output, scores, selection) or sparse (li 2: softmax over
/// every key or the selected rows) layer over bf16 caches at position pos.
void check_bf16_layer(const std::vector<uint8_t>& cache, size_t fk, size_t fv, const std::vector<uint16_t>& qkv,
                      const std::vector<float>& q_raw, const std::vector<float>& got_o, const float* ga, const float* gb,
                      int pos, int li, const embla_host::Buffers& B) {
    std::vector<float> K, V;
    std::vector<uint16_t> Kb, Vb;
    read16(cache, fk, false, 2, MAXS, K, Kb);
    read16(cache, fv, true, 2, MAXS, V, Vb);
    char msg[200];
    float worst;
    if (li == 1) {   // the k/v append of this position: K normed (no gains) and rounded, V copied
        bool ok = true;
        for (int h = 0; h < 2; h++) {
            float kx[HDIM], kn[HDIM];
            for (int d = 0; d < HDIM; d++) kx[d] = bf(qkv[2048 + h * HDIM + d]);
            orc_head_norm(kx, nullptr, nullptr, 0, 1, kn);
            for (int d = 0; d < HDIM; d++) {
                const size_t at = ((size_t)h * MAXS + pos) * HDIM + d;
                ok = ok && Kb[at] == tobf(kn[d]) && Vb[at] == qkv[2560 + h * HDIM + d];
            }
        }
        expect(ok, "bf16 k/v append, bit for bit", pos, li);
    }
    std::vector<float> q(16 * HDIM), out(16 * HDIM);
    for (int h = 0; h < 16; h++) orc_head_norm(&q_raw[h * HDIM], ga, gb, 2, 1, &q[h * HDIM]);
    const int keys = pos + 1;
    const bool selecting = keys > 1024 + 128;
    if (li == 1) {
        std::vector<float> sc((size_t)2 * MAXS);
        orc_decode_f32(q.data(), K.data(), V.data(), keys, MAXS, 16, 2, 1, nullptr, out.data(), sc.data());
        const bool ok = close(got_o.data(), out.data(), 16 * HDIM, 2e-3f, 1e-2f, &worst);
        std::snprintf(msg, sizeof msg, "bf16 full attention, worst |err| %.3g", worst);
        expect(ok, msg, pos, li);
        if (selecting) {
            std::vector<float> gsc((size_t)2 * MAXS);
            std::vector<uint32_t> gsel((size_t)2 * NSEL), want(NSEL);
            HIPCHECK(hipMemcpy(gsc.data(), B.scores, 2 * MAXS * 4, hipMemcpyDeviceToHost));
            HIPCHECK(hipMemcpy(gsel.data(), B.sel, 2 * NSEL * 4, hipMemcpyDeviceToHost));
            float amax = 0.0f;
            for (int h = 0; h < 2; h++)
                for (int j = 0; j < keys; j++) amax = std::fmax(amax, std::fabs(sc[(size_t)h * MAXS + j]));
            bool sok = true, selok = true;
            for (int h = 0; h < 2; h++) {
                float w;
                sok = sok && close(&gsc[(size_t)h * MAXS], &sc[(size_t)h * MAXS], keys, 1e-3f * amax, 0.0f, &w);
                orc_select_keys(&gsc[(size_t)h * MAXS], keys, 1024, 128, want.data());
                selok = selok && std::memcmp(want.data(), &gsel[(size_t)h * NSEL], NSEL * 4) == 0;
            }
            expect(sok, "bf16 scores", pos, li);
            expect(selok, "bf16 selection (select_keys over the GPU's scores), bit for bit", pos, li);
        }
    } else {
        std::vector<uint32_t> gsel((size_t)2 * NSEL);
        if (selecting) HIPCHECK(hipMemcpy(gsel.data(), B.sel, 2 * NSEL * 4, hipMemcpyDeviceToHost));
        orc_decode_f32(q.data(), K.data(), V.data(), selecting ? NSEL : keys, MAXS, 16, 2, 0,
                       selecting ? gsel.data() : nullptr, out.data(), nullptr);
        const bool ok = close(got_o.data(), out.data(), 16 * HDIM, 2e-3f, 1e-2f, &worst);
        std::snprintf(msg, sizeof msg, "bf16 sparse attention (%s), worst |err| %.3g",
                      selecting ? "selected rows" : "every key", worst);
        expect(ok, msg, pos, li);
    }
}

/// kv8: the full layers' caches in int8 (the reference's default), else bf16 (EMBLA_KV8=0).
int run_decode_stack(bool kv8) {
    std::printf("decode stack, %s full-layer caches\n", kv8 ? "int8" : "bf16");
    SplitMix64 g{20261201};

    // ---- weights: gains and 4-bit projections of three layers (Engine.swift:441-485)
    Blob W;
    const size_t qg0 = add_gain(W, g), kg0 = add_gain(W, g), qg1 = add_gain(W, g), kg1 = add_gain(W, g),
                 qg2 = add_gain(W, g), kg2 = add_gain(W, g);
    const Mat q0 = add_mat(W, g, 2048), k0 = add_mat(W, g, 512), v0 = add_mat(W, g, 512), o0 = add_mat(W, g, 2048);
    const Mat q1 = add_mat(W, g, 2048), k1 = add_mat(W, g, 256), v1 = add_mat(W, g, 256), o1 = add_mat(W, g, 2048);
    const Mat q2 = add_mat(W, g, 2048), o2 = add_mat(W, g, 2048);

    // ---- the cache: layer 0's K and V rings, layer 1's int8 (or bf16) K and V regions
    const size_t ring_bytes = (size_t)4 * RING * HDIM * 2;
    const size_t region_bytes = kv8 ? (size_t)2 * MAXS * (HDIM + 4) : (size_t)2 * MAXS * HDIM * 2;
    const size_t rk = 0, rv = ring_bytes, fk = 2 * ring_bytes, fv = fk + (region_bytes + 255) / 256 * 256;
    const size_t cache_bytes = fv + region_bytes;

    Layer L0, L1, L2;
    L0.index = 0; L0.kind = LayerKind::sliding; L0.qGain = qg0; L0.kGain = kg0; L0.kOffset = rk; L0.vOffset = rv;
    L0.nGains = 1; L0.oFirst = true;
    L0.qkv = {seg(q0, 2048, 0, 0), seg(k0, 2560, 0, 2048), seg(v0, 3072, 0, 2560)};
    L0.oproj = {seg(o0, 2048, 0, 0)};
    L1.index = 1; L1.kind = LayerKind::full; L1.qGain = qg1; L1.kGain = kg1; L1.kOffset = fk; L1.vOffset = fv;
    // KV jobs: byte offsets with KV8, element offsets without (Engine.swift:457)
    L1.kvJobs = {kv8 ? EmblaKVJob{2048, 2560, (uint32_t)fk, (uint32_t)fv}
                     : EmblaKVJob{2048, 2560, (uint32_t)(fk / 2), (uint32_t)(fv / 2)}};
    L1.qkv = {seg(q1, 2048, 0, 0), seg(k1, 2304, 0, 2048), seg(v1, 2560, 0, 2560)};
    L1.oproj = {seg(o1, 2048, 0, 0)};
    L2.index = 2; L2.kind = LayerKind::sparse; L2.qGain = qg2; L2.kGain = kg2; L2.kOffset = fk; L2.vOffset = fv;
    L2.qkv = {seg(q2, 2048, 0, 0)};
    L2.oproj = {seg(o2, 2048, 0, 0)};

    // ---- device buffers (Engine.swift:252-267)
    embla_host::Buffers B;
    const size_t ws_bytes = embla_workspace_bytes(MAXS, 16);
    HIPCHECK(hipMalloc(&B.W, W.bytes.size()));
    HIPCHECK(hipMemcpy(B.W, W.bytes.data(), W.bytes.size(), hipMemcpyHostToDevice));
    HIPCHECK(hipMalloc(&B.cache, cache_bytes));
    HIPCHECK(hipMemset(B.cache, 0, cache_bytes));
    HIPCHECK(hipMalloc(&B.hs, D * 2));
    HIPCHECK(hipMalloc(&B.qkv, 4096 * 2));
    HIPCHECK(hipMemset(B.qkv, 0, 4096 * 2));
    HIPCHECK(hipMalloc(&B.o, D * 2));
    HIPCHECK(hipMalloc((void**)&B.x, D * 4));
    HIPCHECK(hipMemset(B.x, 0, D * 4));
    HIPCHECK(hipMalloc((void**)&B.apart, ws_bytes));
    HIPCHECK(hipMemset(B.apart, 0, ws_bytes));
    HIPCHECK(hipMalloc((void**)&B.scores, 2 * MAXS * 4));
    HIPCHECK(hipMalloc((void**)&B.sel, 2 * NSEL * 4));
    HIPCHECK(hipMalloc((void**)&B.counter, 64));
    HIPCHECK(hipMemset(B.counter, 0, 64));
    hipStream_t st;
    HIPCHECK(hipStreamCreate(&st));
    const AttentionEngine E(MAXS, B, {1}, kv8);

    float g0q[HDIM], g0k[HDIM], g1q[HDIM], g1k[HDIM], g2q[HDIM], g2k[HDIM];
    gain_f32(W, qg0, g0q); gain_f32(W, kg0, g0k); gain_f32(W, qg1, g1q); gain_f32(W, kg1, g1k);
    gain_f32(W, qg2, g2q); gain_f32(W, kg2, g2k);

    const int check_at[] = {5, 700, 1400};
    const int last = 1400;
    std::vector<uint16_t> hs(D);
    for (int pos = 0; pos <= last; pos++) {
        for (int i = 0; i < D; i++) hs[i] = tobf((float)g.normal());
        HIPCHECK(hipMemcpy(B.hs, hs.data(), D * 2, hipMemcpyHostToDevice));
        const bool check = pos == check_at[0] || pos == check_at[1] || pos == check_at[2];
        const Layer* layers[3] = {&L0, &L1, &L2};
        for (int li = 0; li < 3; li++) {
            const Layer& L = *layers[li];
            std::vector<float> x_before(D);
            if (check) HIPCHECK(hipMemcpy(x_before.data(), B.x, D * 4, hipMemcpyDeviceToHost));
            const int rc = E.encodeAttention(L, pos, st);
            if (rc != EMBLA_OK) {
                std::printf("FAIL pos %d layer %d: encodeAttention returned %d\n", pos, li, rc);
                return 1;
            }
            if (!check) continue;
            HIPCHECK(hipStreamSynchronize(st));
            std::printf("check pos %d layer %d (%s)\n", pos, li, li == 0 ? "sliding" : li == 1 ? "full" : "sparse");
            std::vector<uint16_t> qkv(4096), o(D);
            std::vector<float> x_after(D);
            std::vector<uint8_t> cache(cache_bytes);
            HIPCHECK(hipMemcpy(qkv.data(), B.qkv, 4096 * 2, hipMemcpyDeviceToHost));
            HIPCHECK(hipMemcpy(o.data(), B.o, D * 2, hipMemcpyDeviceToHost));
            HIPCHECK(hipMemcpy(x_after.data(), B.x, D * 4, hipMemcpyDeviceToHost));
            HIPCHECK(hipMemcpy(cache.data(), B.cache, cache_bytes, hipMemcpyDeviceToHost));
            float worst;
            char msg[200];

            // the q/k/v projection: within the bf16 output's rounding
            {
                const Mat* ms[3] = {li == 0 ? &q0 : li == 1 ? &q1 : &q2, li == 0 ? &k0 : &k1, li == 0 ? &v0 : &v1};
                const unsigned ys[3] = {0, 2048, 2560};
                const int nm = li == 2 ? 1 : 3;
                for (int m = 0; m < nm; m++) {
                    std::vector<float> ref(ms[m]->O), got(ms[m]->O);
                    matvec(W, *ms[m], hs.data(), EMBLA_EPI_BF16, ref.data());
                    for (int r = 0; r < ms[m]->O; r++) got[r] = bf(qkv[ys[m] + r]);
                    const bool ok = close(got.data(), ref.data(), ms[m]->O, 1e-3f, 1.0f / 128, &worst);
                    std::snprintf(msg, sizeof msg, "q/k/v segment %d, worst |err| %.3g", m, worst);
                    expect(ok, msg, pos, li);
                }
            }
            std::vector<float> q_raw(16 * HDIM);
            for (int i = 0; i < 16 * HDIM; i++) q_raw[i] = bf(qkv[i]);
            std::vector<float> out(16 * HDIM), got_o(16 * HDIM);
            for (int i = 0; i < 16 * HDIM; i++) got_o[i] = bf(o[i]);

            if (li == 0) {
                // sliding: q and k normed with their gains, rotated, rounded to bf16; the window
                // pos - 127 .. pos of the ring (the kernel wrote the new k, v into slot pos % RING)
                std::vector<float> Kf, Vf;
                std::vector<uint16_t> Kb, Vb;
                read_ring(cache, rk, false, Kf, Kb);
                read_ring(cache, rv, true, Vf, Vb);
                std::vector<float> q(16 * HDIM);
                for (int h = 0; h < 16; h++) {
                    float t[HDIM];
                    orc_head_norm(&q_raw[h * HDIM], g0q, nullptr, 1, 0, t);
                    orc_rope(t, pos);
                    for (int d = 0; d < HDIM; d++) q[h * HDIM + d] = bf(tobf(t[d]));
                }
                bool ring_ok = true;
                for (int h = 0; h < 4; h++) {
                    float t[HDIM], kr[HDIM];
                    for (int d = 0; d < HDIM; d++) kr[d] = bf(qkv[2048 + h * HDIM + d]);
                    orc_head_norm(kr, g0k, nullptr, 1, 0, t);
                    orc_rope(t, pos);
                    for (int d = 0; d < HDIM; d++) {
                        const size_t at = ((size_t)h * RING + pos % RING) * HDIM + d;
                        if (Kb[at] != tobf(t[d])) ring_ok = false;
                        if (Vb[at] != qkv[2560 + h * HDIM + d]) ring_ok = false;
                    }
                }
                expect(ring_ok, "new ring row (k and v bit for bit)", pos, li);
                const int lo = pos - WINDOW + 1 > 0 ? pos - WINDOW + 1 : 0;
                std::vector<int32_t> slots;
                for (int p = lo; p <= pos; p++) slots.push_back(p % RING);
                orc_decode_rows(q.data(), Kf.data(), Vf.data(), RING, 16, 4, slots.data(), (int)slots.size(), 0, out.data());
                const bool ok = close(got_o.data(), out.data(), 16 * HDIM, 2e-3f, 1e-2f, &worst);
                std::snprintf(msg, sizeof msg, "sliding attention, worst |err| %.3g", worst);
                expect(ok, msg, pos, li);
            } else if (!kv8) {
                check_bf16_layer(cache, fk, fv, qkv, q_raw, got_o, li == 1 ? g1q : g2q, li == 1 ? g1k : g2k, pos, li, B);
            } else {
                std::vector<int8_t> K, V;
                std::vector<float> ks, vs;
                read_int8_region(cache, fk, false, 2, K, ks);
                read_int8_region(cache, fv, true, 2, V, vs);
                if (li == 1) {   // the k/v append of this position, bit for bit
                    bool ok = true;
                    for (int h = 0; h < 2; h++) {
                        float kx[HDIM], vx[HDIM], s;
                        int8_t qk[HDIM];
                        for (int d = 0; d < HDIM; d++) {
                            kx[d] = bf(qkv[2048 + h * HDIM + d]);
                            vx[d] = bf(qkv[2560 + h * HDIM + d]);
                        }
                        orc_quant_row(kx, 1, 1, qk, &s);
                        ok = ok && std::memcmp(qk, &K[((size_t)h * MAXS + pos) * HDIM], HDIM) == 0 && s == ks[(size_t)h * MAXS + pos];
                        orc_quant_row(vx, 0, 1, qk, &s);
                        ok = ok && std::memcmp(qk, &V[((size_t)h * MAXS + pos) * HDIM], HDIM) == 0 && s == vs[(size_t)h * MAXS + pos];
                    }
                    expect(ok, "k/v append bytes and scales", pos, li);
                }
                const float* ga = li == 1 ? g1q : g2q;
                const float* gb = li == 1 ? g1k : g2k;
                std::vector<float> q(16 * HDIM);
                for (int h = 0; h < 16; h++) orc_head_norm(&q_raw[h * HDIM], ga, gb, 2, 1, &q[h * HDIM]);
                const int keys = pos + 1;
                const bool selecting = keys > 1024 + 128;
                if (li == 1) {
                    std::vector<float> sc((size_t)2 * MAXS);   // the oracle's scores: [n_kv][S_cache]
                    orc_decode_int8(q.data(), K.data(), ks.data(), V.data(), vs.data(), keys, MAXS, 16, 2, 1, nullptr,
                                    out.data(), sc.data());
                    const bool ok = close(got_o.data(), out.data(), 16 * HDIM, 2e-3f, 1e-2f, &worst);
                    std::snprintf(msg, sizeof msg, "full attention, worst |err| %.3g", worst);
                    expect(ok, msg, pos, li);
                    if (selecting) {
                        std::vector<float> gsc((size_t)2 * MAXS);
                        std::vector<uint32_t> gsel((size_t)2 * NSEL), want(NSEL);
                        HIPCHECK(hipMemcpy(gsc.data(), B.scores, 2 * MAXS * 4, hipMemcpyDeviceToHost));
                        HIPCHECK(hipMemcpy(gsel.data(), B.sel, 2 * NSEL * 4, hipMemcpyDeviceToHost));
                        float amax = 0.0f;
                        for (int h = 0; h < 2; h++)
                            for (int j = 0; j < keys; j++) amax = std::fmax(amax, std::fabs(sc[(size_t)h * MAXS + j]));
                        bool sok = true, selok = true;
                        for (int h = 0; h < 2; h++) {
                            float w;
                            sok = sok && close(&gsc[(size_t)h * MAXS], &sc[(size_t)h * MAXS], keys, 1e-3f * amax, 0.0f, &w);
                            orc_select_keys(&gsc[(size_t)h * MAXS], keys, 1024, 128, want.data());
                            selok = selok && std::memcmp(want.data(), &gsel[(size_t)h * NSEL], NSEL * 4) == 0;
                        }
                        expect(sok, "scores", pos, li);
                        expect(selok, "selection (select_keys over the GPU's scores), bit for bit", pos, li);
                    }
                } else {
                    std::vector<uint32_t> gsel((size_t)2 * NSEL);
                    if (selecting) HIPCHECK(hipMemcpy(gsel.data(), B.sel, 2 * NSEL * 4, hipMemcpyDeviceToHost));
                    orc_decode_int8(q.data(), K.data(), ks.data(), V.data(), vs.data(), selecting ? NSEL : keys, MAXS,
                                    16, 2, 0, selecting ? gsel.data() : nullptr, out.data(), nullptr);
                    const bool ok = close(got_o.data(), out.data(), 16 * HDIM, 2e-3f, 1e-2f, &worst);
                    std::snprintf(msg, sizeof msg, "sparse attention (%s), worst |err| %.3g",
                                  selecting ? "selected rows" : "every key", worst);
                    expect(ok, msg, pos, li);
                }
            }
            // the o-projection into the residual: x = bf16(W o) for a block's first layer, else
            // x += bf16(W o)
            {
                const Mat& om = li == 0 ? o0 : li == 1 ? o1 : o2;
                std::vector<float> ref = x_before;
                matvec(W, om, o.data(), L.oFirst ? EMBLA_EPI_F32_BF : EMBLA_EPI_ADD, ref.data());
                float amax = 0.0f;
                for (float v : ref) amax = std::fmax(amax, std::fabs(v));
                const bool ok = close(x_after.data(), ref.data(), D, 1e-3f * amax + 1e-3f, 1.0f / 128, &worst);
                std::snprintf(msg, sizeof msg, "residual after the o-projection, worst |err| %.3g", worst);
                expect(ok, msg, pos, li);
            }
        }
    }
    HIPCHECK(hipStreamSynchronize(st));
    if (!kv8) {   // the block store holds int8 rows and scales: not for bf16 caches
        const std::vector<const Layer*> fl{&L1};
        expect(E.copyFullBlock(fl, 1280, B.apart, true, st) == EMBLA_ERR_UNSUPPORTED,
               "full-layer block copy refused without KV8", 1280, -1);
        return 0;
    }

    // ---- prefix-cache blocks through the engine (fullSpans / windowSpans + copy): positions
    // 1280 ..< 1408 saved from this cache and restored into a zeroed one come back exactly there
    {
        const int p0 = 1280;
        void *sf, *sr, *cache2;
        const size_t fb = embla_kv_block_bytes(1, 2, EMBLA_F32), rb = embla_ring_block_bytes(1, 4);
        HIPCHECK(hipMalloc(&sf, fb));
        HIPCHECK(hipMalloc(&sr, rb));
        HIPCHECK(hipMalloc(&cache2, cache_bytes));
        HIPCHECK(hipMemset(cache2, 0, cache_bytes));
        int rc = E.copyFullBlock({&L1}, p0, sf, true, st);
        if (!rc) rc = E.copyWindowBlock({&L0}, p0, sr, true, st);
        embla_host::Buffers B2 = B;
        B2.cache = cache2;
        const AttentionEngine E2(MAXS, B2, {1});
        if (!rc) rc = E2.copyFullBlock({&L1}, p0, sf, false, st);
        if (!rc) rc = E2.copyWindowBlock({&L0}, p0, sr, false, st);
        HIPCHECK(hipStreamSynchronize(st));
        expect(rc == EMBLA_OK, "block copies returned OK", p0, -1);
        std::vector<uint8_t> c1(cache_bytes), c2(cache_bytes);
        HIPCHECK(hipMemcpy(c1.data(), B.cache, cache_bytes, hipMemcpyDeviceToHost));
        HIPCHECK(hipMemcpy(c2.data(), cache2, cache_bytes, hipMemcpyDeviceToHost));
        bool ok = true;
        for (int kind = 0; kind < 2; kind++) {
            std::vector<int8_t> r1, r2;
            std::vector<float> s1, s2;
            read_int8_region(c1, kind ? fv : fk, kind == 1, 2, r1, s1);
            read_int8_region(c2, kind ? fv : fk, kind == 1, 2, r2, s2);
            for (int h = 0; h < 2; h++)
                for (int j = 0; j < MAXS; j++) {
                    const size_t r = (size_t)h * MAXS + j;
                    const bool in = j >= p0 && j < p0 + 128;
                    for (int d = 0; d < HDIM; d++) ok = ok && r2[r * HDIM + d] == (in ? r1[r * HDIM + d] : 0);
                    ok = ok && s2[r] == (in ? s1[r] : 0.0f);
                }
            std::vector<float> f1, f2;
            std::vector<uint16_t> b1, b2;
            read_ring(c1, kind ? rv : rk, kind == 1, f1, b1);
            read_ring(c2, kind ? rv : rk, kind == 1, f2, b2);
            for (int h = 0; h < 4; h++)
                for (int j = 0; j < RING; j++) {
                    const bool in = j >= p0 % RING && j < p0 % RING + 128;
                    for (int d = 0; d < HDIM; d++) {
                        const size_t i = ((size_t)h * RING + j) * HDIM + d;
                        ok = ok && b2[i] == (in ? b1[i] : 0);
                    }
                }
        }
        expect(ok, "prefix block save + restore: the block's rows, scales and ring slots, nothing else", p0, -1);
        std::printf("prefix block save/restore checked\n");
    }

    // ---- the step's token (Engine.swift:972-987): greedy, then a top-p draw
    {
        const int V = 65536, pos = 10, prompt = 5;
        std::vector<float> lg(V);
        for (auto& v : lg) v = (float)(3.0 * g.normal());
        float* dl;
        uint32_t *tokens, *greedy;
        void* scratch;
        const size_t sb = embla_sample_workspace_bytes(V);
        HIPCHECK(hipMalloc((void**)&dl, V * 4));
        HIPCHECK(hipMemcpy(dl, lg.data(), V * 4, hipMemcpyHostToDevice));
        HIPCHECK(hipMalloc((void**)&tokens, 64 * 4));
        HIPCHECK(hipMalloc((void**)&greedy, 64 * 4));
        HIPCHECK(hipMemset(tokens, 0xFF, 64 * 4));
        HIPCHECK(hipMemset(greedy, 0, 64 * 4));
        HIPCHECK(hipMalloc(&scratch, sb));
        AttentionEngine::Sampling greedy_s;
        int rc = E.encodeToken(dl, V, tokens, greedy + 1, pos, prompt, greedy_s, scratch, sb, st);
        AttentionEngine::Sampling draw_s;
        draw_s.temperature = 0.8f;
        draw_s.topP = 0.9f;
        draw_s.seed = 1234;
        if (!rc) rc = E.encodeToken(dl, V, tokens, greedy + 1, pos + 1, prompt, draw_s, scratch, sb, st);
        HIPCHECK(hipStreamSynchronize(st));
        std::vector<uint32_t> gw(64), tw(64);
        HIPCHECK(hipMemcpy(gw.data(), greedy, 64 * 4, hipMemcpyDeviceToHost));
        HIPCHECK(hipMemcpy(tw.data(), tokens, 64 * 4, hipMemcpyDeviceToHost));
        const uint32_t want_g = orc_argmax(lg.data(), V);
        int fragile = 0;
        const uint32_t want_d = orc_sample(lg.data(), V, pos + 1, 1.0f / 0.8f, 0.9f, 1234, &fragile);
        expect(rc == EMBLA_OK, "encodeToken returned OK", pos, -1);
        expect(gw[1 + pos] == want_g && tw[pos + 1] == want_g, "greedy token (greedy[pos], tokens[pos + 1])", pos, -1);
        expect(fragile || (gw[1 + pos + 1] == want_d && tw[pos + 2] == want_d), "top-p draw against the oracle", pos + 1, -1);
        expect(gw[0] == ((uint32_t)(pos + 2) << 16 | gw[1 + pos + 1]), "the polled word: (pos + 1) << 16 | token", pos + 1, -1);
        std::printf("token step checked (greedy %u, draw %u%s)\n", want_g, want_d, fragile ? ", draw fragile" : "");
    }
    return 0;
}

/// Prefill in two chunks against decode token by token: a sliding and a full layer, separate
/// caches, the same weights and inputs; kv8 as run_decode_stack.
int run_prefill_vs_decode(bool kv8) {
    std::printf("prefill vs decode, %s full-layer caches\n", kv8 ? "int8" : "bf16");
    SplitMix64 g{777};
    constexpr int T1 = 160, T2 = 96, N = T1 + T2;
    Blob W;
    const size_t qg0 = add_gain(W, g), kg0 = add_gain(W, g), qg1 = add_gain(W, g), kg1 = add_gain(W, g);
    const Mat q0 = add_mat(W, g, 2048), k0 = add_mat(W, g, 512), v0 = add_mat(W, g, 512), o0 = add_mat(W, g, 2048);
    const Mat q1 = add_mat(W, g, 2048), k1 = add_mat(W, g, 256), v1 = add_mat(W, g, 256), o1 = add_mat(W, g, 2048);
    const size_t ring_bytes = (size_t)4 * RING * HDIM * 2;
    const size_t region_bytes = kv8 ? (size_t)2 * MAXS * (HDIM + 4) : (size_t)2 * MAXS * HDIM * 2;
    const size_t rk = 0, rv = ring_bytes, fk = 2 * ring_bytes, fv = fk + (region_bytes + 255) / 256 * 256;
    const size_t cache_bytes = fv + region_bytes;
    Layer L0, L1;
    L0.index = 0; L0.kind = LayerKind::sliding; L0.qGain = qg0; L0.kGain = kg0; L0.kOffset = rk; L0.vOffset = rv;
    L0.nGains = 1; L0.oFirst = true;
    L0.qkv = {seg(q0, 2048, 0, 0), seg(k0, 2560, 0, 2048), seg(v0, 3072, 0, 2560)};
    L0.oproj = {seg(o0, 2048, 0, 0)};
    L1.index = 1; L1.kind = LayerKind::full; L1.qGain = qg1; L1.kGain = kg1; L1.kOffset = fk; L1.vOffset = fv;
    L1.kvJobs = {kv8 ? EmblaKVJob{2048, 2560, (uint32_t)fk, (uint32_t)fv}
                     : EmblaKVJob{2048, 2560, (uint32_t)(fk / 2), (uint32_t)(fv / 2)}};
    L1.qkv = {seg(q1, 2048, 0, 0), seg(k1, 2304, 0, 2048), seg(v1, 2560, 0, 2560)};
    L1.oproj = {seg(o1, 2048, 0, 0)};

    std::vector<uint16_t> hs((size_t)N * D);
    for (auto& v : hs) v = tobf((float)g.normal());
    void *dW, *cacheA, *cacheB;
    HIPCHECK(hipMalloc(&dW, W.bytes.size()));
    HIPCHECK(hipMemcpy(dW, W.bytes.data(), W.bytes.size(), hipMemcpyHostToDevice));
    HIPCHECK(hipMalloc(&cacheA, cache_bytes));
    HIPCHECK(hipMalloc(&cacheB, cache_bytes));
    HIPCHECK(hipMemset(cacheA, 0, cache_bytes));
    HIPCHECK(hipMemset(cacheB, 0, cache_bytes));
    hipStream_t st;
    HIPCHECK(hipStreamCreate(&st));

    // decode, token by token, into cache A
    embla_host::Buffers B;
    const size_t ws_bytes = embla_workspace_bytes(MAXS, 16);
    B.W = dW; B.cache = cacheA;
    HIPCHECK(hipMalloc(&B.hs, D * 2));
    HIPCHECK(hipMalloc(&B.qkv, 4096 * 2));
    HIPCHECK(hipMalloc(&B.o, D * 2));
    HIPCHECK(hipMalloc((void**)&B.x, D * 4));
    HIPCHECK(hipMalloc((void**)&B.apart, ws_bytes));
    HIPCHECK(hipMemset(B.apart, 0, ws_bytes));
    HIPCHECK(hipMalloc((void**)&B.scores, 2 * MAXS * 4));
    HIPCHECK(hipMalloc((void**)&B.sel, 2 * NSEL * 4));
    HIPCHECK(hipMalloc((void**)&B.counter, 64));
    const AttentionEngine E(MAXS, B, {}, kv8);
    std::vector<float> xd((size_t)N * D);
    for (int pos = 0; pos < N; pos++) {
        HIPCHECK(hipMemcpy(B.hs, &hs[(size_t)pos * D], D * 2, hipMemcpyHostToDevice));
        int rc = E.encodeAttention(L0, pos, st);
        if (!rc) rc = E.encodeAttention(L1, pos, st);
        if (rc) { std::printf("FAIL decode pos %d: %d\n", pos, rc); return 1; }
        HIPCHECK(hipMemcpyAsync(&xd[(size_t)pos * D], B.x, D * 4, hipMemcpyDeviceToHost, st));
    }
    HIPCHECK(hipStreamSynchronize(st));

    // prefill, two chunks, into cache B
    embla_host::PrefillBuffers P;
    P.W = dW; P.cache = cacheB;
    HIPCHECK(hipMalloc(&P.hs, (size_t)T1 * D * 2));
    HIPCHECK(hipMalloc(&P.qkv, (size_t)T1 * 4096 * 2));
    HIPCHECK(hipMalloc(&P.qn, (size_t)16 * T1 * HDIM * 2));
    HIPCHECK(hipMalloc(&P.o, (size_t)T1 * D * 2));
    HIPCHECK(hipMalloc((void**)&P.x, (size_t)T1 * D * 4));
    HIPCHECK(hipMalloc((void**)&P.counter, 64));
    const PrefillEncoder PE(MAXS, P, kv8);
    std::vector<float> xp((size_t)N * D);
    const int chunks[2][2] = {{0, T1}, {T1, T2}};
    for (const auto& c : chunks) {
        const int p0 = c[0], T = c[1];
        std::printf("prefill chunk p0 %d T %d\n", p0, T);
        HIPCHECK(hipMemcpy(P.hs, &hs[(size_t)p0 * D], (size_t)T * D * 2, hipMemcpyHostToDevice));
        int rc = PE.encode(L0, p0, T, st);
        if (!rc) rc = PE.encode(L1, p0, T, st);
        if (rc) { std::printf("FAIL prefill p0 %d: %d\n", p0, rc); return 1; }
        HIPCHECK(hipMemcpyAsync(&xp[(size_t)p0 * D], P.x, (size_t)T * D * 4, hipMemcpyDeviceToHost, st));
        HIPCHECK(hipStreamSynchronize(st));
    }
    // the residuals, token by token (q/k/v by GEMM or GEMV round to bf16 apart by a step at most,
    // and an int8 key or value can move by one: a few parts in a hundred, against O(1) for a
    // wrong position, window or row)
    float xmax = 0.0f;
    for (float v : xd) xmax = std::fmax(xmax, std::fabs(v));
    int bad_tok = -1;
    float worst = 0.0f;
    for (int t = 0; t < N; t++) {
        float w;
        if (!close(&xp[(size_t)t * D], &xd[(size_t)t * D], D, 0.03f * xmax, 0.03f, &w) && bad_tok < 0) bad_tok = t;
        worst = std::fmax(worst, w);
    }
    char msg[160];
    std::snprintf(msg, sizeof msg, "prefill residuals = decode residuals (worst |err| %.3g of max %.3g, first bad token %d)",
                  worst, xmax, bad_tok);
    std::printf("%s\n", msg);
    expect(bad_tok < 0, msg, N - 1, -1);
    // the caches: the full layer's int8 rows dequantised, the sliding ring's rows
    std::vector<uint8_t> ca(cache_bytes), cb(cache_bytes);
    HIPCHECK(hipMemcpy(ca.data(), cacheA, cache_bytes, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(cb.data(), cacheB, cache_bytes, hipMemcpyDeviceToHost));
    bool cache_ok = true;
    for (int kind = 0; kind < 2 && !kv8; kind++) {   // bf16 rows
        std::vector<float> fa, fb;
        std::vector<uint16_t> ba, bb;
        read16(ca, kind ? fv : fk, kind == 1, 2, MAXS, fa, ba);
        read16(cb, kind ? fv : fk, kind == 1, 2, MAXS, fb, bb);
        for (int h = 0; h < 2; h++)
            for (int j = 0; j < N; j++)
                for (int d = 0; d < HDIM; d++) {
                    const size_t i = ((size_t)h * MAXS + j) * HDIM + d;
                    if (std::fabs(fa[i] - fb[i]) > 0.03f * (std::fabs(fa[i]) + 1.0f)) cache_ok = false;
                }
    }
    for (int kind = 0; kind < 2 && kv8; kind++) {
        std::vector<int8_t> ra, rb;
        std::vector<float> sa, sb;
        read_int8_region(ca, kind ? fv : fk, kind == 1, 2, ra, sa);
        read_int8_region(cb, kind ? fv : fk, kind == 1, 2, rb, sb);
        for (int h = 0; h < 2; h++)
            for (int j = 0; j < N; j++) {
                const size_t r = (size_t)h * MAXS + j;
                float amax = 0.0f;
                for (int d = 0; d < HDIM; d++) amax = std::fmax(amax, std::fabs(ra[r * HDIM + d] * sa[r]));
                for (int d = 0; d < HDIM; d++)
                    if (std::fabs(ra[r * HDIM + d] * sa[r] - rb[r * HDIM + d] * sb[r]) > 0.03f * amax) cache_ok = false;
            }
    }
    expect(cache_ok, "full layer's cache rows: prefill = decode (within 3%)", N - 1, 1);
    std::vector<float> ka, kb2;
    std::vector<uint16_t> kab, kbb;
    bool ring_ok = true;
    for (int kind = 0; kind < 2; kind++) {
        read_ring(ca, kind ? rv : rk, kind == 1, ka, kab);
        read_ring(cb, kind ? rv : rk, kind == 1, kb2, kbb);
        for (int h = 0; h < 4; h++)
            for (int j = 0; j < N; j++)
                for (int d = 0; d < HDIM; d++) {
                    const size_t i = ((size_t)h * RING + j) * HDIM + d;
                    if (std::fabs(ka[i] - kb2[i]) > 0.03f * (std::fabs(ka[i]) + 1.0f)) ring_ok = false;
                }
    }
    expect(ring_ok, "sliding ring rows: prefill = decode", N - 1, 0);
    return 0;
}

int main() {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);   // line-buffered: a failing run still shows its last step
    HIPCHECK(hipSetDevice(0));
    for (const bool kv8 : {true, false}) {
        if (run_decode_stack(kv8)) return 1;
        if (run_prefill_vs_decode(kv8)) return 1;
    }
    std::printf("%d checks, %d failed\n", checks, failures);
    return failures ? 1 : 0;
}
