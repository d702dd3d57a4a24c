// The C ABI: host-side validation, chunking and launch order, mirroring the attention parts of
// Engine.encodeAttention (Sources/EmblaMetal/Engine.swift:743-832) and Prefill.encode
// (Sources/EmblaMetal/Prefill.swift:290-341, 378-407).
#include <stdlib.h>
#include <string.h>
#include "embla_internal.hpp"

using namespace embla;

namespace {

constexpr size_t kCounterBytes = 1024;  // reserved (zeroed by embla_workspace_init)
constexpr int kMaxChunks = 256;         // chunks the merge kernel takes (decode_full.hip)
constexpr int kMaxKV = 16;
constexpr int kPartStride = 132;
constexpr int kRefWindow = 128;         // the reference's sliding window (Engine.swift:9)
constexpr int kRefRing = 4096;          // the reference's ring (attention.metal:6)
constexpr int kTopK = 1024, kRecent = 128;   // Engine.swift:9 (topk, recent)
constexpr int kSparseRefCH = 128;        // keys a chunk of the gathered reference sparse decode
#ifndef IDX_CHUNK
#define IDX_CHUNK 512   // C5 sparse layer: 0.428 ms at 2048 keys, 0.417-0.424 at 512, 0.426 at 256, 0.469 at 4096
#endif
constexpr int kIndexChunk = IDX_CHUNK;    // keys a workgroup of the MFMA indexer
constexpr int kPrefillSplits = 4;       // most key-range splits of a prefill chunk (workspace sizing)

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

/// Key-range splits of a prefill launch: as many as keep every split >= 4 key tiles while the grid
/// is under 256 workgroups (one a CU: 8 waves, 2 a SIMD), at most kPrefillSplits, and only with a
/// workspace for the partial rows. EMBLA_PREFILL_SPLITS caps it (tuning).
int prefill_splits(const void* ws, size_t ws_bytes, int T, int n_q, int blocks, int tiles) {
    if (!ws || ws_bytes < (size_t)kPrefillSplits * T * n_q * kPartStride * 4) return 1;
    static const int cap = [] {
        const char* e = getenv("EMBLA_PREFILL_SPLITS");
        return e ? atoi(e) : 2;
    }();
    int ns = 1;
    while (ns * 2 <= cap && ns * 2 <= kPrefillSplits && blocks * ns < 256 && tiles / (ns * 2) >= 4) ns *= 2;
    return ns;
}

struct Workspace {
    uint32_t* counter;
    uint16_t* qprep;
    float* part;
};

size_t qprep_bytes(int n_q) { return round_up((size_t)n_q * 128 * 2, 256); }
size_t part_bytes(int max_s, int n_q) { return (size_t)((max_s + 31) / 32) * n_q * kPartStride * 4; }

Workspace carve(void* ws, int max_s, int n_q) {
    char* p = (char*)ws;
    Workspace w;
    w.counter = (uint32_t*)p;
    w.qprep = (uint16_t*)(p + kCounterBytes);
    w.part = (float*)(p + kCounterBytes + qprep_bytes(n_q));
    return w;
}

/// A tuning override from the environment, or dflt. Call sites keep the value in a static, so the
/// environment is read once a process, not on every launch.
int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    if (!s || !*s) return dflt;
    return atoi(s);
}

/// Keys a workgroup for the split decode: about EMBLA_DECODE_WG workgroups over all kv heads
/// (default 256, one a CU on MI355X), at most kMaxChunks a kv head, at least 128 keys (a 32-key
/// tile for 4 of the 8 waves: short contexts gain from more workgroups), a multiple of 32. The reference's chunks8 makes the same choice for its GPU
/// (Engine.swift:736-739).
int decode_chunk(int S, int n_kv, int extra = 0) {
    static const int env_target = env_int("EMBLA_DECODE_WG", 256);
    // extra: workgroups the launch adds (the decode step's appends); the chunks then leave them
    // CUs with a sixteenth to spare, so that no workgroup waits for a CU (C3 step: 11.83 us a
    // layer with 64 chunks a kv head + 4 appends, 11.15-11.17 with 57)
    const int target = extra ? env_target * 15 / 16 - extra : env_target;
    int per_head = target / n_kv > 0 ? target / n_kv : 1;
    if (per_head > kMaxChunks) per_head = kMaxChunks;
    int ch = (S + per_head - 1) / per_head;
    ch = (ch + 31) / 32 * 32;
    return ch < 128 ? 128 : ch;   // 16-layer graph at 4096 keys: 128 keys 9.5 us a layer, 256 10.2
}

bool valid_act(int dt) { return dt == EMBLA_F16 || dt == EMBLA_BF16; }
bool valid_scale(int dt) { return dt == EMBLA_F16 || dt == EMBLA_F32; }

}  // namespace

extern "C" {

int embla_version(void) { return 1; }

size_t embla_workspace_bytes(int max_s, int n_q) {
    if (max_s <= 0 || n_q <= 0) return 0;
    return kCounterBytes + qprep_bytes(n_q) + part_bytes(max_s, n_q);
}

int embla_workspace_init(void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!ws || ws_bytes < kCounterBytes) return EMBLA_ERR_WORKSPACE;
    return hipMemsetAsync(ws, 0, kCounterBytes, stream) == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // extern "C"

namespace {

/// The split-K decode's arguments from embla_decode_int8's (validated); rc != 0 on a bad argument.
int full_decode_args(const void* q, const void* kc, const void* vc, void* o, float* scores, int S, int max_s, int n_q,
                     int n_kv, int weights, int scale_dtype, int out_dtype, int chunk, void* ws, size_t ws_bytes,
                     FullDecodeArgs& a) {
    const int rc = embla::full_decode_plan(q, kc, vc, o, scores, S, max_s, n_q, n_kv, weights, scale_dtype, out_dtype,
                                           chunk, a);
    if (rc) return rc;
    if (a.C > 1) {
        if (!ws || ws_bytes < embla_workspace_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
        if ((size_t)a.C * n_q * kPartStride * 4 > part_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
    }
    a.part = ws ? carve(ws, max_s, n_q).part : nullptr;
    return EMBLA_OK;
}

/// The bf16-cache decode of the reference's full (ReLU², optional scores) and sparse (softmax,
/// optional SEL rows) layers: 16 query heads over 2 kv heads, part as the workspace.
int attn16(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc, float* part,
           float* scores, const uint32_t* idx, uint32_t* counter, void* o, const EmblaAttnParams* p, bool relu2,
           hipStream_t stream) {
    if (!p || !part || !counter || !kc || !vc || !o) return EMBLA_ERR_INVALID;
    if (p->S <= 0 || p->maxS <= 0 || p->maxS % 32 || p->S > p->maxS) return EMBLA_ERR_INVALID;
    if (!qraw || p->ng < 0 || p->ng > 2 || (p->ng >= 1 && !g1) || (p->ng >= 2 && !g2)) return EMBLA_ERR_INVALID;
    (void)counter;   // no counters: the partials are merged by a second kernel
    int ch = p->CH;
    if (ch <= 0) {   // about 256 workgroups over the 2 kv heads, a 32-key tile a wave at least
        ch = (p->S + 127) / 128;
        ch = (ch + 31) / 32 * 32;
        if (ch < 128) ch = 128;
    }
    if (ch % 32 || (p->S + ch - 1) / ch > kMaxChunks) return EMBLA_ERR_INVALID;
    Full16Args a;
    a.q = (const uint16_t*)qraw; a.g1 = (const uint16_t*)g1; a.g2 = (const uint16_t*)g2; a.ng = p->ng;
    a.kc = (const uint16_t*)kc; a.vc = (const uint16_t*)vc;
    a.idx = idx;
    a.part = carve(part, p->maxS, 16).part;
    a.scores = scores;
    a.o = (uint16_t*)o;
    a.S = p->S; a.CH = ch; a.C = (p->S + ch - 1) / ch; a.max_s = p->maxS; a.n_q = 16; a.n_kv = 2;
    a.relu2 = relu2;
    return launch_full16_decode(a, stream);
}

}  // namespace

namespace embla {

int full_decode_plan(const void* q, const void* kc, const void* vc, void* o, float* scores, int S, int max_s, int n_q,
                     int n_kv, int weights, int scale_dtype, int out_dtype, int chunk, FullDecodeArgs& a) {
    if (S <= 0 || max_s <= 0 || max_s % 32 || S > max_s) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV) return EMBLA_ERR_INVALID;
    if (weights != EMBLA_SOFTMAX && weights != EMBLA_RELU2_SINK) return EMBLA_ERR_INVALID;
    if (!valid_scale(scale_dtype) || !valid_act(out_dtype)) return EMBLA_ERR_INVALID;
    if (scores && weights != EMBLA_RELU2_SINK) return EMBLA_ERR_UNSUPPORTED;
    if (chunk < 0 || chunk % 32) return EMBLA_ERR_INVALID;
    const int ch = chunk ? chunk : decode_chunk(S, n_kv);
    const int C = (S + ch - 1) / ch;
    if (C > kMaxChunks) return EMBLA_ERR_INVALID;
    a.q = (const uint16_t*)q;
    a.kc = (const int8_t*)kc;
    a.vc = (const int8_t*)vc;
    a.part = nullptr;
    a.scores = scores;
    a.o = (uint16_t*)o;
    a.S = S; a.CH = ch; a.C = C; a.max_s = max_s; a.n_q = n_q; a.n_kv = n_kv;
    a.relu2 = weights == EMBLA_RELU2_SINK;
    a.scale32 = scale_dtype == EMBLA_F32;
    a.out_bf16 = out_dtype == EMBLA_BF16;
    return EMBLA_OK;
}

}  // namespace embla

extern "C" {

int embla_decode_int8(const void* q, const void* kc, const void* vc, void* o, float* scores, int S,
                      int max_s, int n_q, int n_kv, int weights, int scale_dtype, int out_dtype,
                      int chunk, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!q || !kc || !vc || !o) return EMBLA_ERR_INVALID;
    FullDecodeArgs a;
    const int rc = full_decode_args(q, kc, vc, o, scores, S, max_s, n_q, n_kv, weights, scale_dtype, out_dtype, chunk,
                                    ws, ws_bytes, a);
    return rc ? rc : launch_full_decode(a, stream);
}

int embla_decode_int8_partials(const void* q, const void* kc, const void* vc, float* scores, int S, int max_s,
                               int n_q, int n_kv, int weights, int scale_dtype, int out_dtype, int chunk, void* ws,
                               size_t ws_bytes, hipStream_t stream) {
    if (!q || !kc || !vc || !ws) return EMBLA_ERR_INVALID;
    FullDecodeArgs a;
    const int rc = full_decode_args(q, kc, vc, nullptr, scores, S, max_s, n_q, n_kv, weights, scale_dtype, out_dtype,
                                    chunk, ws, ws_bytes, a);
    if (rc) return rc;
    if (a.C < 2) return EMBLA_ERR_INVALID;   // one chunk writes o itself: nothing to merge
    a.merge = false;
    return launch_full_decode(a, stream);
}

int embla_decode_int8_merge(void* o, int S, int max_s, int n_q, int n_kv, int weights, int out_dtype, int chunk,
                            void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!o || !ws) return EMBLA_ERR_INVALID;
    FullDecodeArgs a;
    const int rc = full_decode_args(o, o, o, o, nullptr, S, max_s, n_q, n_kv, weights, EMBLA_F16, out_dtype, chunk, ws,
                                    ws_bytes, a);
    if (rc) return rc;
    if (a.C < 2) return EMBLA_ERR_INVALID;
    return launch_full_decode_merge(a, stream);
}

int embla_decode_int8_qraw(const void* qraw, const void* g1, const void* g2, int ng, const void* kc, const void* vc,
                           void* o, int S, int max_s, int n_q, int n_kv, int scale_dtype, int out_dtype, int chunk,
                           void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!qraw || !kc || !vc || !o || ng < 0 || ng > 2 || (ng >= 1 && !g1) || (ng >= 2 && !g2)) return EMBLA_ERR_INVALID;
    if (S <= 0 || max_s <= 0 || max_s % 32 || S > max_s) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV) return EMBLA_ERR_INVALID;
    if (!valid_scale(scale_dtype) || !valid_act(out_dtype)) return EMBLA_ERR_INVALID;
    if (chunk < 0 || chunk % 32) return EMBLA_ERR_INVALID;
    const int ch = chunk ? chunk : decode_chunk(S, n_kv);
    const int C = (S + ch - 1) / ch;
    if (C > kMaxChunks) return EMBLA_ERR_INVALID;
    if (C > 1) {
        if (!ws || ws_bytes < embla_workspace_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
        if ((size_t)C * n_q * kPartStride * 4 > part_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
    }
    Workspace w = ws ? carve(ws, max_s, n_q) : Workspace{nullptr, nullptr, nullptr};
    FullDecodeArgs a;
    a.q = (const uint16_t*)qraw;
    a.g1 = (const uint16_t*)g1;
    a.g2 = (const uint16_t*)g2;
    a.ng = ng;
    a.kc = (const int8_t*)kc;
    a.vc = (const int8_t*)vc;
    a.part = w.part;
    a.scores = nullptr;
    a.o = (uint16_t*)o;
    a.S = S; a.CH = ch; a.C = C; a.max_s = max_s; a.n_q = n_q; a.n_kv = n_kv;
    a.relu2 = false;
    a.scale32 = scale_dtype == EMBLA_F32;
    a.out_bf16 = out_dtype == EMBLA_BF16;
    return launch_full_decode(a, stream);
}

int embla_decode_step_int8(const void* qkv, int q_off, int k_off, int v_off, const void* g1, const void* g2, int ng,
                           void* kc, void* vc, void* o, int pos, int max_s, int n_q, int n_kv, int scale_dtype,
                           int norm_k, int out_dtype, int chunk, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!qkv || !kc || !vc || !o || ng < 0 || ng > 2 || (ng >= 1 && !g1) || (ng >= 2 && !g2)) return EMBLA_ERR_INVALID;
    // q is read 16 bytes at a time: 8-element offsets from a 16-byte aligned buffer
    if (q_off < 0 || k_off < 0 || v_off < 0 || (q_off | k_off | v_off) & 7 || (uintptr_t)qkv & 15)
        return EMBLA_ERR_INVALID;
    if (pos < 0 || max_s <= 0 || max_s % 32 || pos >= max_s) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV) return EMBLA_ERR_INVALID;
    if (!valid_scale(scale_dtype) || !valid_act(out_dtype) || chunk < 0 || chunk % 32) return EMBLA_ERR_INVALID;
    const int ch = pos == 0 ? 32 : chunk ? chunk : decode_chunk(pos, n_kv, n_kv);
    const int C = (pos + ch - 1) / ch;   // chunks over the cached keys 0 .. pos - 1
    if (C + 1 > kMaxChunks) return EMBLA_ERR_INVALID;
    if (!ws || ws_bytes < embla_workspace_bytes(max_s, n_q) || (size_t)(C + 1) * n_q * kPartStride * 4 > part_bytes(max_s, n_q))
        return EMBLA_ERR_WORKSPACE;
    Workspace w = carve(ws, max_s, n_q);
    const uint16_t* base = (const uint16_t*)qkv;
    FullDecodeArgs a;
    a.q = base + q_off;
    a.g1 = (const uint16_t*)g1;
    a.g2 = (const uint16_t*)g2;
    a.ng = ng;
    a.kc = (const int8_t*)kc;
    a.vc = (const int8_t*)vc;
    a.part = w.part;
    a.scores = nullptr;
    a.o = (uint16_t*)o;
    a.S = pos; a.CH = ch; a.C = C; a.max_s = max_s; a.n_q = n_q; a.n_kv = n_kv;
    a.relu2 = false;
    a.scale32 = scale_dtype == EMBLA_F32;
    a.out_bf16 = out_dtype == EMBLA_BF16;
    a.append = true;
    a.knew = base + k_off;
    a.vnew = base + v_off;
    a.kcw = (int8_t*)kc;
    a.vcw = (int8_t*)vc;
    a.pos = pos;
    a.norm_k = norm_k ? 1 : 0;
    return launch_full_decode(a, stream);
}

int embla_q_prep(const void* qraw, const void* g1, const void* g2, int ng, int stride, int T,
                 int n_q, void* out, int out_dtype, hipStream_t stream) {
    if (!qraw || !out || T <= 0 || n_q <= 0 || ng < 0 || ng > 2 || stride < n_q * 128) return EMBLA_ERR_INVALID;
    if ((ng >= 1 && !g1) || (ng >= 2 && !g2) || !valid_act(out_dtype)) return EMBLA_ERR_INVALID;
    QPrepArgs a{(const uint16_t*)qraw, (const uint16_t*)g1, (const uint16_t*)g2, ng, stride, T, n_q,
                (uint16_t*)out, out_dtype == EMBLA_BF16};
    return launch_q_prep(a, stream);
}

int embla_q_prep_b(const void* qkv, const void* g1, const void* g2, void* qn, int T, hipStream_t stream) {
    if (!qkv || !g1 || !g2 || !qn || T <= 0) return EMBLA_ERR_INVALID;
    QPrepArgs a{(const uint16_t*)qkv, (const uint16_t*)g1, (const uint16_t*)g2, 2, 4096, T, 16, (uint16_t*)qn, true};
    a.head_major = true;
    return launch_q_prep(a, stream);
}

int embla_attn_full8(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                     float* part, float* scores, uint32_t* counter, void* o, const EmblaAttnParams* p,
                     hipStream_t stream) {
    if (!p || !part || !counter) return EMBLA_ERR_INVALID;
    if (p->S <= 0 || p->maxS <= 0 || p->maxS % 32 || p->S > p->maxS) return EMBLA_ERR_INVALID;
    if (!qraw || p->ng < 0 || p->ng > 2 || (p->ng >= 1 && !g1) || (p->ng >= 2 && !g2)) return EMBLA_ERR_INVALID;
    // the reference's part buffer doubles as this call's workspace (the partials); the head norm
    // of q runs inside the decode kernel, as in the reference's kernel
    Workspace w = carve(part, p->maxS, 16);
    const int ch = p->CH > 0 ? p->CH : decode_chunk(p->S, 2);
    if (ch % 32 || (p->S + ch - 1) / ch > kMaxChunks) return EMBLA_ERR_INVALID;
    FullDecodeArgs a;
    a.q = (const uint16_t*)qraw;
    a.g1 = (const uint16_t*)g1;
    a.g2 = (const uint16_t*)g2;
    a.ng = p->ng;
    a.kc = (const int8_t*)kc;
    a.vc = (const int8_t*)vc;
    a.part = w.part;
    (void)counter;   // no counters: the partials are merged by a second kernel
    a.scores = scores;
    a.o = (uint16_t*)o;
    a.S = p->S; a.CH = ch; a.C = (p->S + ch - 1) / ch; a.max_s = p->maxS; a.n_q = 16; a.n_kv = 2;
    a.relu2 = true; a.scale32 = true; a.out_bf16 = true;
    return launch_full_decode(a, stream);
}

int embla_attn_full(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc, float* part,
                    float* scores, uint32_t* counter, void* o, const EmblaAttnParams* p, hipStream_t stream) {
    return attn16(qraw, g1, g2, kc, vc, part, scores, nullptr, counter, o, p, true, stream);
}

int embla_attn_sparse(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                      float* part, const uint32_t* idx, uint32_t* counter, void* o, const EmblaAttnParams* p,
                      hipStream_t stream) {
    return attn16(qraw, g1, g2, kc, vc, part, nullptr, idx, counter, o, p, false, stream);
}

int embla_kv_append_bf16(const void* qkv, void* cache, const EmblaKVJob* jobs, int njobs, int pm_pos, int maxS, int T,
                         hipStream_t stream) {
    if (!qkv || !cache || !jobs || njobs <= 0 || T <= 0 || pm_pos < 0 || maxS <= 0 || maxS % 32) return EMBLA_ERR_INVALID;
    if (pm_pos + T > maxS) return EMBLA_ERR_INVALID;
    for (int i = 0; i < njobs; i++) {
        const EmblaKVJob& j = jobs[i];
        const uint16_t* base = (const uint16_t*)qkv;
        uint16_t* c = (uint16_t*)cache;
        RingAppendArgs a{base + j.k, base + j.v, 4096, T, pm_pos, 2, maxS, c + j.kc, c + j.vc, nullptr};
        a.norm_k = true;
        const int rc = launch_ring_append(a, stream);
        if (rc) return rc;
    }
    return EMBLA_OK;
}

int embla_attn_full_b(const void* qkv, const void* g1, const void* g2, const void* kc, const void* vc, float* part,
                      uint32_t* counter, void* o, const EmblaAttnB* p, int T, hipStream_t stream) {
    if (!qkv || !g1 || !g2 || !kc || !vc || !part || !counter || !o || !p || T <= 0) return EMBLA_ERR_INVALID;
    if (p->p0 < 0 || p->maxS <= 0 || p->maxS % 32 || p->p0 + T > p->maxS) return EMBLA_ERR_INVALID;
    (void)counter;   // no counters: one pass over every key of a row, no chunk partials
    // q_prep_b's queries (both gains, bf16) in the part buffer, token-major [T][16][128]; the
    // ReLU² prefill over the bf16 cache (keys 0 .. p0 + t for row t) on the 16-bit tile path
    uint16_t* qn = (uint16_t*)part;
    QPrepArgs qa{(const uint16_t*)qkv, (const uint16_t*)g1, (const uint16_t*)g2, 2, 4096, T, 16, qn, true};
    int rc = launch_q_prep(qa, stream);
    if (rc) return rc;
    PrefillArgs a;
    a.q = qn; a.q_tok_stride = 16 * 128; a.q_head_stride = 128;
    a.kc = nullptr; a.vc = nullptr;
    a.o = (uint16_t*)o; a.o_tok_stride = 2048; a.o_head_stride = 128;
    a.T = T; a.p0 = p->p0; a.max_s = p->maxS; a.n_q = 16; a.n_kv = 2; a.window = 0;
    a.nsplit = 1; a.part = nullptr;
    a.relu2 = true; a.scale32 = false; a.q_bf16 = true; a.out_bf16 = true;
    a.kring = (const uint16_t*)kc; a.vring = (const uint16_t*)vc; a.R = p->maxS; a.qg = nullptr;
    return launch_prefill_ring(a, stream);
}

int embla_attn_sparse8(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                       float* part, const uint32_t* idx, uint32_t* counter, void* o, const EmblaAttnParams* p,
                       hipStream_t stream) {
    if (!p || !part || !counter) return EMBLA_ERR_INVALID;
    if (p->S <= 0 || p->maxS <= 0 || p->maxS % 32 || p->S > p->maxS) return EMBLA_ERR_INVALID;
    Workspace w = carve(part, p->maxS, 16);
    (void)counter;   // no counters: the partials are merged by a second kernel
    if (!idx) {      // SEL = 0: every key 0 .. S-1, softmax (attention.metal:448-584); the head
                     // norm of q inside the decode kernel
        if (!qraw || p->ng < 0 || p->ng > 2 || (p->ng >= 1 && !g1) || (p->ng >= 2 && !g2)) return EMBLA_ERR_INVALID;
        const int ch = p->CH > 0 ? p->CH : decode_chunk(p->S, 2);
        if (ch % 32 || (p->S + ch - 1) / ch > kMaxChunks) return EMBLA_ERR_INVALID;
        FullDecodeArgs a;
        a.q = (const uint16_t*)qraw;
        a.g1 = (const uint16_t*)g1;
        a.g2 = (const uint16_t*)g2;
        a.ng = p->ng;
        a.kc = (const int8_t*)kc;
        a.vc = (const int8_t*)vc;
        a.part = w.part;
        a.scores = nullptr;
        a.o = (uint16_t*)o;
        a.S = p->S; a.CH = ch; a.C = (p->S + ch - 1) / ch; a.max_s = p->maxS; a.n_q = 16; a.n_kv = 2;
        a.relu2 = false; a.scale32 = true; a.out_bf16 = true;
        return launch_full_decode(a, stream);
    }
    // SEL: the rows idx[kv head][0 .. S) of the tile cache, gathered
    int rc = embla_q_prep(qraw, g1, g2, p->ng, 16 * 128, 1, 16, w.qprep, EMBLA_F16, stream);
    if (rc) return rc;
    const int ch = p->CH > 0 ? p->CH : kSparseRefCH;
    if (ch % 32 || ch > kTopK + kRecent) return EMBLA_ERR_INVALID;
    const int C = (p->S + ch - 1) / ch;
    if (C > kMaxChunks) return EMBLA_ERR_INVALID;
    SparseRows8Args a{w.qprep, 0, (const int8_t*)kc, (const int8_t*)vc, idx, 0, p->S, p->S, p->S, 1,
                      (uint16_t*)o, 0, w.part, ch, C, p->maxS, 16, 2, false, true, true, true};
    return launch_sparse_rows8(a, stream);
}

int embla_kv_quant_append(const void* k, const void* v, int in_dtype, int stride, int T, int p0,
                          int n_kv, void* kc, void* vc, int max_s, int scale_dtype, int norm_k,
                          hipStream_t stream) {
    if (!k || !v || !kc || !vc || T <= 0 || p0 < 0 || n_kv <= 0 || stride < n_kv * 128) return EMBLA_ERR_INVALID;
    if (max_s <= 0 || max_s % 32 || p0 + T > max_s) return EMBLA_ERR_INVALID;
    if (!valid_act(in_dtype) || !valid_scale(scale_dtype)) return EMBLA_ERR_INVALID;
    KVQuantArgs a{(const uint16_t*)k, (const uint16_t*)v, stride, T, p0, n_kv, max_s,
                  (int8_t*)kc, (int8_t*)vc, in_dtype == EMBLA_BF16, scale_dtype == EMBLA_F32, norm_k != 0};
    return launch_kv_quant(a, stream);
}

int embla_kv_append(const void* qkv, void* cache, const EmblaKVJob* jobs, int njobs, int pm_pos,
                    int maxS, int T, hipStream_t stream) {
    if (!qkv || !cache || !jobs || njobs <= 0 || T <= 0) return EMBLA_ERR_INVALID;
    for (int i = 0; i < njobs; i++) {
        const EmblaKVJob& j = jobs[i];
        const uint16_t* base = (const uint16_t*)qkv;
        char* c = (char*)cache;
        const int rc = embla_kv_quant_append(base + j.k, base + j.v, EMBLA_BF16, 4096, T, pm_pos, 2,
                                             c + j.kc, c + j.vc, maxS, EMBLA_F32, 1, stream);
        if (rc) return rc;
    }
    return EMBLA_OK;
}

int embla_sliding_decode(const void* q, const void* k_new, const void* v_new, void* kring, void* vring,
                         void* o, int pos, int window, int ring, int n_q, int n_kv, int dtype, int chunk,
                         void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!q || !k_new || !v_new || !kring || !vring || !o) return EMBLA_ERR_INVALID;
    if (pos < 0 || window <= 0 || ring <= 0 || ring % 32 || window > ring || !valid_act(dtype)) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV) return EMBLA_ERR_INVALID;
    if (n_q / n_kv != 4) return EMBLA_ERR_UNSUPPORTED;
    if (chunk < 0 || chunk % 32) return EMBLA_ERR_INVALID;
    const int lo = pos - window + 1 > 0 ? pos - window + 1 : 0;
    const int span = pos - (lo & ~31);   // ring keys from the first tile on (the current key is extra)
    static const int ch_env = env_int("EMBLA_SLIDING_CH", 192);
    const int ch = chunk ? chunk : ch_env;   // C2 step: 8.61 us at 192, 8.74 at 256, 8.67-8.82 at 160, 9.48 at 224, 8.77 at 96
    if (ch <= 0 || ch % 32) return EMBLA_ERR_INVALID;   // (a bad EMBLA_SLIDING_CH)
    int C = (span + ch - 1) / ch;
    if (C < 1) C = 1;
    if (C > kMaxChunks) return EMBLA_ERR_INVALID;
    if (C > 1 && (!ws || ws_bytes < embla_workspace_bytes(ring, n_q))) return EMBLA_ERR_WORKSPACE;
    RingArgs a;
    a.q = (const uint16_t*)q; a.q_stride = 128;
    a.k_new = (const uint16_t*)k_new; a.v_new = (const uint16_t*)v_new;
    a.qg = nullptr; a.kg = nullptr;
    a.kring = (uint16_t*)kring; a.vring = (uint16_t*)vring;
    a.part = ws ? carve(ws, ring, n_q).part : nullptr;
    a.o = (uint16_t*)o;
    a.pos = pos; a.W = window; a.R = ring; a.CH = ch; a.C = C; a.n_q = n_q; a.n_kv = n_kv;
    a.bf16 = dtype == EMBLA_BF16; a.preops = false;
    return launch_ring_decode(a, stream);
}

int embla_attn_sliding(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o,
                       int pos, hipStream_t stream) {
    if (!qkv || !qg || !kg || !kc || !vc || !o || pos < 0) return EMBLA_ERR_INVALID;
    const uint16_t* row = (const uint16_t*)qkv;
    RingArgs a;
    a.q = row; a.q_stride = 128;
    a.k_new = row + 16 * 128; a.v_new = row + 20 * 128;
    a.qg = (const uint16_t*)qg; a.kg = (const uint16_t*)kg;
    a.kring = (uint16_t*)kc; a.vring = (uint16_t*)vc;
    a.part = nullptr;
    a.o = (uint16_t*)o;
    a.pos = pos; a.W = kRefWindow; a.R = kRefRing; a.CH = kRefWindow + 32; a.C = 1; a.n_q = 16; a.n_kv = 4;
    // one chunk: at most 127 ring keys counted from a 32-aligned tile fit in kRefWindow + 32
    a.bf16 = true; a.preops = true;
    return launch_ring_decode(a, stream);
}

int embla_index_scores(const void* qi, const float* w, const void* ki, float* scores, int n, int n_ih,
                       hipStream_t stream) {
    if (!qi || !w || !ki || !scores || n <= 0) return EMBLA_ERR_INVALID;
    if (n_ih != 1 && n_ih != 2 && n_ih != 4) return EMBLA_ERR_UNSUPPORTED;
    return launch_index_scores((const uint16_t*)qi, w, (const uint16_t*)ki, scores, n, n_ih, stream);
}

int embla_select_topk(const float* scores, int score_stride, uint32_t* idx, int idx_stride, int S, int n_sets,
                      int topk, int recent, hipStream_t stream) {
    if (!scores || !idx || n_sets <= 0 || topk <= 0 || recent < 0) return EMBLA_ERR_INVALID;
    if (S <= topk + recent) return EMBLA_ERR_INVALID;   // the reference selects only past topk + recent keys
    if (n_sets > 1 && (score_stride < S || idx_stride < topk + recent)) return EMBLA_ERR_INVALID;
    return launch_select_topk(scores, score_stride, idx, idx_stride, S, n_sets, topk, recent, stream);
}

int embla_select_keys(const float* scores, uint32_t* idx, int S, int maxS, hipStream_t stream) {
    return embla_select_topk(scores, maxS, idx, kTopK + kRecent, S, 2, kTopK, kRecent, stream);
}

namespace {
/// Checks embla_sparse_decode's arguments and fills its launch (fs: the wide select's fields of
/// SparseArgs, sel_* set, for the select's last step fused into the attention). Launches nothing,
/// so a caller can check every argument before it starts any kernel of a multi-kernel step.
int sparse_decode_prepare(const void* q, const void* kc, const void* vc, const uint32_t* idx, int idx_stride,
                          int nsel, void* o, int max_s, int n_q, int n_kv, int dtype, int chunk, void* ws,
                          size_t ws_bytes, const SparseArgs* fs, SparseArgs& a) {
    if (!q || !kc || !vc || !o || nsel <= 0 || max_s <= 0 || idx_stride < 0) return EMBLA_ERR_INVALID;
    if (!idx && nsel > max_s) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV || !valid_act(dtype)) return EMBLA_ERR_INVALID;
    if (n_q / n_kv != 4 && n_q / n_kv != 8) return EMBLA_ERR_UNSUPPORTED;
    if (chunk < 0 || chunk % 32) return EMBLA_ERR_INVALID;
    static const int ch_env = env_int("EMBLA_SPARSE_CH", 64);
    int ch = chunk ? chunk : ch_env;   // C4 step: 32.0 us at 64, 32.4 at 128, 36.4 at 256
    if (ch <= 0 || ch % 32) return EMBLA_ERR_INVALID;
    if (fs) {   // the fused select ranks a chunk's rows in LDS: at most kSparseFusedMaxCh of them
        if (ch > kSparseFusedMaxCh) ch = kSparseFusedMaxCh;
        if (!fs->sel_ws || !fs->sel_epoch || fs->sel_topk <= 0 || fs->sel_n <= fs->sel_topk ||
            fs->sel_n > kWideSelectMaxN || nsel < fs->sel_topk)
            return EMBLA_ERR_INVALID;
    }
    const int C = (nsel + ch - 1) / ch;
    if (C > kMaxChunks) return EMBLA_ERR_INVALID;
    if (C > 1 && (!ws || ws_bytes < embla_workspace_bytes(32 * C, n_q))) return EMBLA_ERR_WORKSPACE;
    a = SparseArgs{};
    a.q = (const uint16_t*)q; a.kc = (const uint16_t*)kc; a.vc = (const uint16_t*)vc;
    a.idx = idx; a.idx_stride = idx_stride; a.nsel = nsel;
    a.part = ws ? carve(ws, 32 * C, n_q).part : nullptr;
    a.o = (uint16_t*)o;
    a.CH = ch; a.C = C; a.max_s = max_s; a.n_q = n_q; a.n_kv = n_kv; a.bf16 = dtype == EMBLA_BF16;
    if (fs) {
        a.sel_ws = fs->sel_ws; a.sel_n = fs->sel_n; a.sel_topk = fs->sel_topk;
        a.sel_out = fs->sel_out; a.sel_epoch = fs->sel_epoch;
    }
    return EMBLA_OK;
}
}  // namespace

int embla_sparse_decode(const void* q, const void* kc, const void* vc, const uint32_t* idx, int idx_stride,
                        int nsel, void* o, int max_s, int n_q, int n_kv, int dtype, int chunk, void* ws,
                        size_t ws_bytes, hipStream_t stream) {
    SparseArgs a;
    const int rc = sparse_decode_prepare(q, kc, vc, idx, idx_stride, nsel, o, max_s, n_q, n_kv, dtype, chunk, ws,
                                         ws_bytes, nullptr, a);
    return rc ? rc : launch_sparse_decode(a, stream);
}

size_t embla_sparse_workspace_bytes(int max_s, int n_q) {
    if (max_s <= 0 || n_q <= 0) return 0;
    return round_up((size_t)max_s * 4, 256) + round_up((size_t)(kTopK + kRecent) * 4, 256) +
           round_up(embla_workspace_bytes(kTopK + kRecent, n_q), 256) + kWideSelectWords * 4;
}

size_t embla_sparse_workspace_recount_offset(int max_s, int n_q) {
    if (max_s <= 0 || n_q <= 0) return 0;
    return round_up((size_t)max_s * 4, 256) + round_up((size_t)(kTopK + kRecent) * 4, 256) +
           round_up(embla_workspace_bytes(kTopK + kRecent, n_q), 256) + kWideSelectRecounts * 4;
}

int embla_sparse_workspace_audit(void* ws, size_t ws_bytes, int max_s, int n_q, hipStream_t stream) {
    if (!ws || max_s <= 0 || n_q <= 0) return EMBLA_ERR_INVALID;
    if (ws_bytes < embla_sparse_workspace_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
    uint32_t* word = (uint32_t*)((char*)ws + embla_sparse_workspace_recount_offset(max_s, n_q));
    uint32_t n = 0;
    if (hipMemcpyAsync(&n, word, 4, hipMemcpyDeviceToHost, stream) != hipSuccess) return EMBLA_ERR_HIP;
    if (hipStreamSynchronize(stream) != hipSuccess) return EMBLA_ERR_HIP;
    if (n == 0) return EMBLA_OK;
    if (hipMemsetAsync(word, 0, 4, stream) != hipSuccess || hipStreamSynchronize(stream) != hipSuccess)
        return EMBLA_ERR_HIP;
    return EMBLA_ERR_WORKSPACE;
}

int embla_sparse_layer_decode(const void* q, const void* qi, const float* w, const void* ki, const void* kc,
                              const void* vc, void* o, int S, int max_s, int n_q, int n_kv, int n_ih, int dtype,
                              void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!q || !qi || !w || !ki || !kc || !vc || !o || S <= 0 || S > max_s) return EMBLA_ERR_INVALID;
    if (!ws || ws_bytes < embla_sparse_workspace_bytes(max_s, n_q)) return EMBLA_ERR_WORKSPACE;
    char* p = (char*)ws;
    float* scores = (float*)p;
    uint32_t* idx = (uint32_t*)(p + round_up((size_t)max_s * 4, 256));
    void* aws = p + round_up((size_t)max_s * 4, 256) + round_up((size_t)(kTopK + kRecent) * 4, 256);
    const size_t abytes = embla_workspace_bytes(kTopK + kRecent, n_q);
    if (S <= kTopK + kRecent)   // every key (Engine.swift:796-799: no selection yet)
        return embla_sparse_decode(q, kc, vc, nullptr, 0, S, o, max_s, n_q, n_kv, dtype, 0, aws, abytes, stream);
    if (n_ih != 1 && n_ih != 2 && n_ih != 4) return EMBLA_ERR_UNSUPPORTED;
    // index scores, then the exact top-k on many workgroups (the select's workspace follows the
    // decode's). Its last step runs inside the attention's workgroups, each ranking the rows it
    // attends; the selection still lands in idx. Every argument of both launches is checked
    // before the first: a call rejected after the scorer had counted into the histogram buffer
    // would leave that buffer stale for the next call.
    uint32_t* sel_ws = (uint32_t*)((char*)aws + round_up(abytes, 256));
    SparseArgs fs;
    fs.sel_ws = sel_ws; fs.sel_n = S - kRecent; fs.sel_topk = kTopK; fs.sel_out = idx;
    fs.sel_epoch = sel_ws + kWideSelectEpoch;
    SparseArgs a;
    int rc = sparse_decode_prepare(q, kc, vc, nullptr, 0, kTopK + kRecent, o, max_s, n_q, n_kv, dtype, 0, aws, abytes,
                                   &fs, a);
    if (rc) return rc;
    rc = launch_wide_select((const uint16_t*)qi, w, (const uint16_t*)ki, scores, S, n_ih, kTopK, kRecent, sel_ws,
                            stream);
    if (rc) return rc;
    return launch_sparse_decode(a, stream);
}

size_t embla_prefill_workspace_bytes(int T, int n_q) {
    if (T <= 0 || n_q <= 0) return 0;
    return (size_t)kPrefillSplits * T * n_q * kPartStride * 4;
}

int embla_prefill_int8(const void* q, int q_dtype, long q_tok_stride, long q_head_stride, const void* kc,
                       const void* vc, void* o, int o_dtype, long o_tok_stride, long o_head_stride, int T, int p0,
                       int max_s, int n_q, int n_kv, int weights, int scale_dtype, int window, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
    if (!q || !kc || !vc || !o || T <= 0 || p0 < 0 || max_s <= 0 || max_s % 32 || p0 + T > max_s) return EMBLA_ERR_INVALID;
    if (!valid_act(q_dtype) || !valid_act(o_dtype) || !valid_scale(scale_dtype) || window < 0) return EMBLA_ERR_INVALID;
    if (weights != EMBLA_SOFTMAX && weights != EMBLA_RELU2_SINK) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv) return EMBLA_ERR_INVALID;
    PrefillArgs a;
    a.q = (const uint16_t*)q; a.q_tok_stride = q_tok_stride; a.q_head_stride = q_head_stride;
    a.kc = (const int8_t*)kc; a.vc = (const int8_t*)vc;
    a.o = (uint16_t*)o; a.o_tok_stride = o_tok_stride; a.o_head_stride = o_head_stride;
    a.T = T; a.p0 = p0; a.max_s = max_s; a.n_q = n_q; a.n_kv = n_kv; a.window = window;
    // two key-range splits when a workspace is given and the blocks are too few to fill the GPU
    // with two waves a SIMD (the split partials cost one merge pass)
    const int gqw = n_q / n_kv, rows_wg = gqw >= 1 && gqw <= 8 ? 32 * (8 / gqw) : 32;   // query rows a workgroup
    const int blocks = (T + rows_wg - 1) / rows_wg * n_kv;
    a.nsplit = prefill_splits(ws, ws_bytes, T, n_q, blocks,
                              window > 0 ? min((p0 + T) / 64, (window + 63) / 64 + 1) : (p0 + T) / 64);
    a.part = (float*)ws;
    a.kring = nullptr; a.vring = nullptr; a.R = 0; a.qg = nullptr;
    a.relu2 = weights == EMBLA_RELU2_SINK; a.scale32 = scale_dtype == EMBLA_F32;
    a.q_bf16 = q_dtype == EMBLA_BF16; a.out_bf16 = o_dtype == EMBLA_BF16;
    // a workspace large enough for the staged copy: the region's keys are converted to fp16 once
    // (prestage_kernel) instead of once a workgroup, for the instances that have a staged form
    const size_t staged = embla_prefill_staged_workspace_bytes(T, p0, n_q, n_kv);
    if (ws && staged && ws_bytes >= staged && window == 0 && !a.relu2 && !a.scale32 && a.q_bf16 && a.out_bf16 &&
        n_q == 4 * n_kv) {
        const int R = (p0 + T + 127) / 128 * 128;
        uint16_t* k16 = (uint16_t*)((char*)ws + round_up(embla_prefill_workspace_bytes(T, n_q), 256));
        return launch_prefill_prestaged(a, k16, k16 + (size_t)n_kv * R * 128, R, stream);
    }
    return launch_prefill_int8(a, stream);
}

size_t embla_prefill_staged_workspace_bytes(int T, int p0, int n_q, int n_kv) {
    if (T <= 0 || p0 < 0 || n_q <= 0 || n_kv <= 0) return 0;
    const size_t R = (size_t)(p0 + T + 127) / 128 * 128;
    return round_up(embla_prefill_workspace_bytes(T, n_q), 256) + 2 * (size_t)n_kv * R * 128 * 2;
}

int embla_prefill_full(const void* q, const void* k, const void* v, void* kc, void* vc, void* o, int T, int p0,
                       int max_s, int n_q, int n_kv, void* ws, size_t ws_bytes, hipStream_t stream) {
    int rc = embla_kv_quant_append(k, v, EMBLA_BF16, n_kv * 128, T, p0, n_kv, kc, vc, max_s, EMBLA_F16, 0, stream);
    if (rc) return rc;
    return embla_prefill_int8(q, EMBLA_BF16, (long)n_q * 128, 128, kc, vc, o, EMBLA_BF16, (long)n_q * 128, 128, T,
                              p0, max_s, n_q, n_kv, EMBLA_SOFTMAX, EMBLA_F16, 0, ws, ws_bytes, stream);
}

int embla_relu2_prefill(const void* qn, const void* kc, const void* vc, void* o, int Tq, int Tk, int maxS,
                        hipStream_t stream) {
    if (Tk < Tq) return EMBLA_ERR_INVALID;
    // q [16][Tq][128] head-major (q_prep_b), out token-major [Tq][2048] (attn_nax.metal:358)
    return embla_prefill_int8(qn, EMBLA_BF16, 128, (long)Tq * 128, kc, vc, o, EMBLA_BF16, 2048, 128, Tq, Tk - Tq,
                              maxS, 16, 2, EMBLA_RELU2_SINK, EMBLA_F32, 0, nullptr, 0, stream);
}

int embla_ring_append(const void* k, const void* v, int dtype, int stride, int T, int p0, int n_kv, void* kring,
                      void* vring, int ring, const void* kg, hipStream_t stream) {
    if (!k || !v || !kring || !vring || T <= 0 || p0 < 0 || n_kv <= 0 || stride < n_kv * 128) return EMBLA_ERR_INVALID;
    if (ring <= 0 || ring % 32 || T > ring || !valid_act(dtype)) return EMBLA_ERR_INVALID;
    if (kg && dtype != EMBLA_BF16) return EMBLA_ERR_UNSUPPORTED;
    RingAppendArgs a{(const uint16_t*)k, (const uint16_t*)v, stride, T, p0, n_kv, ring, (uint16_t*)kring,
                     (uint16_t*)vring, (const uint16_t*)kg};
    return launch_ring_append(a, stream);
}

int embla_prefill_ring(const void* q, int dtype, long q_tok_stride, long q_head_stride, const void* kring,
                       const void* vring, int ring, void* o, long o_tok_stride, long o_head_stride, int T, int p0,
                       int n_q, int n_kv, int window, const void* qg, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!q || !kring || !vring || !o || T <= 0 || p0 < 0 || window <= 0 || !valid_act(dtype)) return EMBLA_ERR_INVALID;
    if (ring <= 0 || ring % 32 || window - 1 + T > ring) return EMBLA_ERR_INVALID;   // the window and chunk fit the ring
    if (n_kv <= 0 || n_q % n_kv) return EMBLA_ERR_INVALID;
    if (qg && dtype != EMBLA_BF16) return EMBLA_ERR_UNSUPPORTED;
    PrefillArgs a;
    a.q = (const uint16_t*)q; a.q_tok_stride = q_tok_stride; a.q_head_stride = q_head_stride;
    a.kc = nullptr; a.vc = nullptr;
    a.o = (uint16_t*)o; a.o_tok_stride = o_tok_stride; a.o_head_stride = o_head_stride;
    a.T = T; a.p0 = p0; a.max_s = ring; a.n_q = n_q; a.n_kv = n_kv; a.window = window;
    const int gqw = n_q / n_kv, rows_wg = gqw >= 1 && gqw <= 8 ? 32 * (8 / gqw) : 32;   // query rows a workgroup
    const int blocks = (T + rows_wg - 1) / rows_wg * n_kv;
    a.nsplit = prefill_splits(ws, ws_bytes, T, n_q, blocks, (window + 63) / 64 + 1);
    a.part = (float*)ws;
    a.relu2 = false; a.scale32 = false; a.q_bf16 = dtype == EMBLA_BF16; a.out_bf16 = dtype == EMBLA_BF16;
    a.kring = (const uint16_t*)kring; a.vring = (const uint16_t*)vring; a.R = ring; a.qg = (const uint16_t*)qg;
    return launch_prefill_ring(a, stream);
}

int embla_prefill_sliding(const void* q, const void* k, const void* v, void* kring, void* vring, void* o, int T,
                          int p0, int ring, int window, int n_q, int n_kv, void* ws, size_t ws_bytes,
                          hipStream_t stream) {
    int rc = embla_ring_append(k, v, EMBLA_BF16, n_kv * 128, T, p0, n_kv, kring, vring, ring, nullptr, stream);
    if (rc) return rc;
    return embla_prefill_ring(q, EMBLA_BF16, (long)n_q * 128, 128, kring, vring, ring, o, (long)n_q * 128, 128, T, p0,
                              n_q, n_kv, window, nullptr, ws, ws_bytes, stream);
}

int embla_attn_sliding8_b(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o, int p0, int T,
                          hipStream_t stream) {
    if (!qkv || !qg || !kg) return EMBLA_ERR_INVALID;
    const uint16_t* row = (const uint16_t*)qkv;
    int rc = embla_ring_append(row + 16 * 128, row + 20 * 128, EMBLA_BF16, 4096, T, p0, 4, kc, vc, kRefRing, kg, stream);
    if (rc) return rc;
    return embla_prefill_ring(row, EMBLA_BF16, 4096, 128, kc, vc, kRefRing, o, 2048, 128, T, p0, 16, 4, kRefWindow, qg,
                              nullptr, 0, stream);
}

int embla_attn_sliding_b(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o, int p0, int T,
                         hipStream_t stream) {
    // the scalar prefill's math is attn_sliding8_b's (prefill.metal:129-180 against 428-548)
    return embla_attn_sliding8_b(qkv, qg, kg, kc, vc, o, p0, T, stream);
}

size_t embla_sparse_prefill_workspace_bytes(int T, int p0) {
    if (T <= 0 || p0 < 0) return 0;
    const size_t ld = round_up((size_t)(p0 + T > kRecent ? p0 + T - kRecent : 1), kIndexChunk);
    const size_t nch = ld / kIndexChunk;
    return round_up((size_t)T * ld * 2, 256) + round_up(nch * 4, 256) + round_up((size_t)T * 8, 256) +
           (size_t)T * (kTopK + kRecent) * 4;
}

int embla_prefill_sparse(const void* q, const void* k, const void* v, const void* qi, const float* w, const void* ki,
                         void* kc, void* vc, void* o, uint32_t* idx, int T, int p0, int max_s, int n_q, int n_kv,
                         void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!q || !k || !v || !qi || !w || !ki || !kc || !vc || !o || T <= 0 || p0 < 0) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_q % n_kv || n_kv > kMaxKV || max_s <= 0 || p0 + T > max_s) return EMBLA_ERR_INVALID;
    if (!ws || ws_bytes < embla_sparse_prefill_workspace_bytes(T, p0)) return EMBLA_ERR_WORKSPACE;
    if (p0 + T - kRecent > 32768) return EMBLA_ERR_UNSUPPORTED;
    const int ld = (int)round_up((size_t)(p0 + T > kRecent ? p0 + T - kRecent : 1), kIndexChunk);
    const int nch = ld / kIndexChunk;
    char* wp = (char*)ws;
    uint16_t* keys = (uint16_t*)wp;
    wp += round_up((size_t)T * ld * 2, 256);
    float* kmax = (float*)wp;
    wp += round_up((size_t)nch * 4, 256);
    uint32_t* ovf = (uint32_t*)wp;   // the band select's overflow records
    wp += round_up((size_t)T * 8, 256);
    uint32_t* sel = idx ? idx : (uint32_t*)wp;
    // the chunk's K, V quantised into the row-major int8 cache
    KVQuantArgs qa{(const uint16_t*)k, (const uint16_t*)v, n_kv * 128, T, p0, n_kv, max_s,
                   (int8_t*)kc, (int8_t*)vc, true, false, false, true};
    int rc = launch_kv_quant(qa, stream);
    if (rc) return rc;
    IndexMfmaArgs ia{(const uint16_t*)qi, w, (const uint16_t*)ki, keys, kmax, T, p0 + T, ld, kIndexChunk,
                     p0 + 1 - kRecent};
    if ((rc = launch_index_mfma(ia, stream))) return rc;
    BandSelectArgs ba{keys, ld, (const uint16_t*)qi, w, (const uint16_t*)ki, kmax, nch, sel, kTopK + kRecent,
                      T, p0, kTopK, kRecent, ovf};
    if ((rc = launch_select_band(ba, stream))) return rc;
    SparseRows8Args sa{(const uint16_t*)q, (long)n_q * 128, (const int8_t*)kc, (const int8_t*)vc, sel,
                       kTopK + kRecent, 0, kTopK + kRecent, p0, T, (uint16_t*)o, (long)n_q * 128, nullptr,
                       p0 + T > kTopK + kRecent ? kTopK + kRecent : p0 + T, 1, max_s, n_q, n_kv,
                       true, true, false, false};
    return launch_sparse_rows8(sa, stream);
}

// ---------------------------------------------------------------- prefix-cache blocks
size_t embla_kv_block_bytes(int n_layers, int n_kv, int scale_dtype) {
    if (n_layers <= 0 || n_kv <= 0 || !valid_scale(scale_dtype)) return 0;
    return (size_t)n_layers * 2 * n_kv * 128 * (128 + (scale_dtype == EMBLA_F32 ? 4 : 2));
}

int embla_kv_block_copy(void* cache, const unsigned long long* regions, int n_layers, int p0, int max_s, int n_kv,
                        int scale_dtype, void* stored, int save, hipStream_t stream) {
    if (!cache || !regions || !stored || n_layers <= 0 || n_layers > kMaxBlockLayers) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_kv > kMaxKV || max_s <= 0 || max_s % 32 || p0 < 0 || p0 % 128 || p0 + 128 > max_s)
        return EMBLA_ERR_INVALID;
    if (!valid_scale(scale_dtype)) return EMBLA_ERR_INVALID;
    BlockCopyArgs a{};
    a.cache = (char*)cache;
    a.stored = (char*)stored;
    for (int l = 0; l < 2 * n_layers; l++) {
        if (regions[l] % 16) return EMBLA_ERR_INVALID;
        a.off[l] = regions[l];
    }
    a.n_layers = n_layers; a.n_kv = n_kv; a.max_s = max_s; a.p0 = p0;
    a.elem = 1;
    a.row_units = 128 * 128 / 16;
    a.scale_bytes = scale_dtype == EMBLA_F32 ? 4 : 2;
    a.scale_units = 128 * a.scale_bytes / 16;
    a.save = save ? 1 : 0;
    return launch_block_copy(a, stream);
}

size_t embla_ring_block_bytes(int n_layers, int n_kv) {
    if (n_layers <= 0 || n_kv <= 0) return 0;
    return (size_t)n_layers * 2 * n_kv * 128 * 128 * 2;
}

int embla_ring_block_copy(void* cache, const unsigned long long* regions, int n_layers, int p0, int ring, int n_kv,
                          void* stored, int save, hipStream_t stream) {
    if (!cache || !regions || !stored || n_layers <= 0 || n_layers > kMaxBlockLayers) return EMBLA_ERR_INVALID;
    if (n_kv <= 0 || n_kv > kMaxKV || ring <= 0 || ring % 128 || p0 < 0 || p0 % 128) return EMBLA_ERR_INVALID;
    BlockCopyArgs a{};
    a.cache = (char*)cache;
    a.stored = (char*)stored;
    for (int l = 0; l < 2 * n_layers; l++) {
        if (regions[l] % 16) return EMBLA_ERR_INVALID;
        a.off[l] = regions[l];
    }
    a.n_layers = n_layers; a.n_kv = n_kv; a.max_s = ring; a.p0 = p0 % ring;   // the block's slots
    a.elem = 2;
    a.row_units = 128 * 128 * 2 / 16;
    a.scale_bytes = 0;
    a.scale_units = 0;
    a.save = save ? 1 : 0;
    return launch_block_copy(a, stream);
}

// ---------------------------------------------------------------- 4-bit projections
int embla_gemv_q4(const void* W, const void* X, void* Y, const EmblaSeg* segs, int nseg, int K, int epi,
                  hipStream_t stream) {
    if (!W || !X || !Y || !segs || nseg <= 0 || nseg > kMaxGemvSegs) return EMBLA_ERR_INVALID;
    if ((K != 2048 && K != 4096) || epi < EMBLA_EPI_BF16 || epi > EMBLA_EPI_F32) return EMBLA_ERR_INVALID;
    GemvArgs a{};
    a.W = W; a.X = X; a.Y = Y; a.nseg = nseg; a.K = K;
    unsigned int prev = 0;
    for (int i = 0; i < nseg; i++) {
        const EmblaSeg& g = segs[i];
        if (g.end <= prev || g.end % 4 || g.w % 16 || g.s % 2 || g.b % 2 || g.x % 8) return EMBLA_ERR_INVALID;
        a.seg[i] = GemvSeg{g.w, g.s, g.b, g.end, g.x, g.y, 0};
        prev = g.end;
    }
    return launch_gemv_q4(a, epi, stream);
}

int embla_gemm_q4(const void* W, const unsigned long long* wo, const void* X, void* Y, int T, int O, int K,
                  int ldx, int ldy, int epi, hipStream_t stream) {
    if (!W || !wo || !X || !Y || T <= 0 || O <= 0 || K <= 0 || K % 64) return EMBLA_ERR_INVALID;
    if (ldx < K || ldx % 8 || ldy < O || epi < EMBLA_EPI_BF16 || epi > EMBLA_EPI_F32) return EMBLA_ERR_INVALID;
    if (wo[0] % 16 || wo[1] % 2 || wo[2] % 2) return EMBLA_ERR_INVALID;
    GemmArgs a{W, wo[0], wo[1], wo[2], (const uint16_t*)X, Y, T, O, K, ldx, ldy};
    return launch_gemm_q4(a, epi, stream);
}

size_t embla_sample_workspace_bytes(int V) { return V > 0 && V <= 65536 ? sample_ws_bytes(V) : 0; }

int embla_argmax(const float* logits, uint32_t* token, int V, uint32_t* greedy, int pos, int prompt_len, void* ws,
                 size_t ws_bytes, hipStream_t stream) {
    if (!logits || !token || !greedy || V <= 0 || V > 65536 || pos < 0 || (uintptr_t)logits % 16) return EMBLA_ERR_INVALID;
    if (!ws || ws_bytes < sample_ws_bytes(V)) return EMBLA_ERR_WORKSPACE;
    return launch_argmax(logits, V, token, greedy, pos, prompt_len, (char*)ws, stream);
}

int embla_sample(const float* logits, uint32_t* token, int V, uint32_t* greedy, int pos, int prompt_len, float inv_t,
                 float top_p, uint32_t seed, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!logits || !token || !greedy || V <= 0 || V > 65536 || pos < 0 || (uintptr_t)logits % 16) return EMBLA_ERR_INVALID;
    if (!(inv_t > 0.0f) || !(inv_t < __builtin_huge_valf()) || !(top_p > 0.0f) || !(top_p <= 1.0f)) return EMBLA_ERR_INVALID;
    if (!ws || ws_bytes < sample_ws_bytes(V)) return EMBLA_ERR_WORKSPACE;
    return launch_sample(logits, V, token, greedy, pos, prompt_len, inv_t, top_p, seed, (char*)ws, stream);
}

}  // extern "C"
