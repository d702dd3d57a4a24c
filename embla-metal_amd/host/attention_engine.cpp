// Engine.encodeAttention (Sources/EmblaMetal/Engine.swift:743-832) over the C ABI; see the header.
#include "attention_engine.hpp"

namespace embla_host {

namespace {
const char* at(const void* base, size_t off) { return static_cast<const char*>(base) + off; }
char* at(void* base, size_t off) { return static_cast<char*>(base) + off; }
}  // namespace

int AttentionEngine::encodeAttention(const Layer& L, int pos, hipStream_t st, bool kvOnly) const {
    if (pos < 0 || pos >= maxContext_ || L.qkv.empty() || L.oproj.empty()) return EMBLA_ERR_INVALID;
    // the q/k/v projection (Engine.swift:745-749)
    int rc = embla_gemv_q4(b_.W, b_.hs, b_.qkv, L.qkv.data(), (int)L.qkv.size(), d, EMBLA_EPI_BF16, st);
    if (rc) return rc;
    // the k/v appends of the full layers (Engine.swift:754-764, 782-793)
    const bool appends = L.kind != LayerKind::sliding && !L.kvJobs.empty();
    if (appends) {
        rc = kv8_ ? embla_kv_append(b_.qkv, b_.cache, L.kvJobs.data(), (int)L.kvJobs.size(), pos, maxContext_, 1, st)
                  : embla_kv_append_bf16(b_.qkv, b_.cache, L.kvJobs.data(), (int)L.kvJobs.size(), pos, maxContext_, 1,
                                         st);
        if (rc) return rc;
    }
    if (kvOnly) return EMBLA_OK;
    const void* qg = at(b_.W, L.qGain);
    const void* kg = at(b_.W, L.kGain);
    if (L.kind == LayerKind::sliding) {   // Engine.swift:771-780 (writes the new k, v into its ring)
        rc = embla_attn_sliding(b_.qkv, qg, kg, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset), b_.o, pos, st);
    } else {
        // past topk + recent keys the selecting full layers score every key and select, and the
        // sparse layers attend the selected rows only (Engine.swift:794-799)
        const int keys = pos + 1;
        const bool sel = selecting(pos), score = scoring(L, pos);
        const int rows = sel && L.kind == LayerKind::sparse ? topk + recent : keys;
        EmblaAttnParams ap{rows, 0, 0, maxContext_, pos, L.nGains, 0, 0};
        // the pipelines (Engine.swift:223-226): attn_full8 / attn_sparse8, or without KV8 the bf16 ones
        const auto full = kv8_ ? embla_attn_full8 : embla_attn_full;
        const auto sparse = kv8_ ? embla_attn_sparse8 : embla_attn_sparse;
        if (L.kind == LayerKind::full) {
            rc = full(b_.qkv, qg, kg, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset), b_.apart,
                      score ? b_.scores : nullptr, b_.counter, b_.o, &ap, st);
            if (!rc && score) rc = embla_select_keys(b_.scores, b_.sel, keys, maxContext_, st);   // 819-827
        } else {
            rc = sparse(b_.qkv, qg, kg, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset), b_.apart,
                        sel ? b_.sel : nullptr, b_.counter, b_.o, &ap, st);
        }
    }
    if (rc) return rc;
    // the o-projection into the residual (Engine.swift:830)
    return embla_gemv_q4(b_.W, b_.o, b_.x, L.oproj.data(), (int)L.oproj.size(), d,
                         L.oFirst ? EMBLA_EPI_F32_BF : EMBLA_EPI_ADD, st);
}

int AttentionEngine::copyFullBlock(const std::vector<const Layer*>& full, int p0, void* stored, bool save,
                                   hipStream_t st) const {
    if (!kv8_) return EMBLA_ERR_UNSUPPORTED;
    std::vector<unsigned long long> regions;
    for (const Layer* L : full) {
        if (!L || L->kind != LayerKind::full) return EMBLA_ERR_INVALID;
        regions.push_back(L->kOffset);
        regions.push_back(L->vOffset);
    }
    if (regions.empty()) return EMBLA_ERR_INVALID;
    return embla_kv_block_copy(b_.cache, regions.data(), (int)full.size(), p0, maxContext_, 2, EMBLA_F32, stored,
                               save ? 1 : 0, st);
}

int AttentionEngine::copyWindowBlock(const std::vector<const Layer*>& sliding, int p0, void* stored, bool save,
                                     hipStream_t st) const {
    std::vector<unsigned long long> regions;
    for (const Layer* L : sliding) {
        if (!L || L->kind != LayerKind::sliding) return EMBLA_ERR_INVALID;
        regions.push_back(L->kOffset);
        regions.push_back(L->vOffset);
    }
    if (regions.empty()) return EMBLA_ERR_INVALID;
    return embla_ring_block_copy(b_.cache, regions.data(), (int)sliding.size(), p0, 4096, 4, stored, save ? 1 : 0, st);
}

int AttentionEngine::encodeToken(const float* logits, int vocab, uint32_t* tokens, uint32_t* greedy, int pos,
                                 int promptEnd, const Sampling& s, void* scratch, size_t scratchBytes,
                                 hipStream_t st) const {
    if (s.isGreedy())
        return embla_argmax(logits, tokens, vocab, greedy, pos, promptEnd, scratch, scratchBytes, st);
    const float top_p = s.topP < 1.0f ? s.topP : 1.0f;   // Sampling.init clamps it to [0, 1]
    return embla_sample(logits, tokens, vocab, greedy, pos, promptEnd, 1.0f / s.temperature, top_p, s.seed, scratch,
                        scratchBytes, st);
}

int PrefillEncoder::encode(const Layer& L, int p0, int T, hipStream_t st, bool kvOnly) const {
    constexpr int d = AttentionEngine::d;
    if (p0 < 0 || T <= 0 || p0 + T > maxContext_ || L.qkv.empty() || L.oproj.empty()) return EMBLA_ERR_INVALID;
    // the q/k/v GEMM, one call a segment (segmentGEMM, Prefill.swift:288)
    unsigned start = 0;
    for (const EmblaSeg& s : L.qkv) {
        const unsigned long long wo[3] = {s.w, s.s, s.b};
        const int rc = embla_gemm_q4(b_.W, wo, static_cast<const uint16_t*>(b_.hs) + s.x,
                                     static_cast<uint16_t*>(b_.qkv) + s.y, T, (int)(s.end - start), d, d, 4096,
                                     EMBLA_EPI_BF16, st);
        if (rc) return rc;
        start = s.end;
    }
    int rc = EMBLA_OK;
    const void* qg = at(b_.W, L.qGain);
    const void* kg = at(b_.W, L.kGain);
    if (L.kind == LayerKind::sliding) {   // Prefill.swift:291-313
        if (kvOnly) return EMBLA_OK;
        rc = embla_attn_sliding8_b(b_.qkv, qg, kg, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset), b_.o, p0, T, st);
    } else {                              // Prefill.swift:315-340, 378-407
        if (!L.kvJobs.empty()) {
            rc = kv8_ ? embla_kv_append(b_.qkv, b_.cache, L.kvJobs.data(), (int)L.kvJobs.size(), p0, maxContext_, T, st)
                      : embla_kv_append_bf16(b_.qkv, b_.cache, L.kvJobs.data(), (int)L.kvJobs.size(), p0, maxContext_,
                                             T, st);
            if (rc) return rc;
        }
        if (kvOnly) return EMBLA_OK;
        if (kv8_) {
            rc = embla_q_prep_b(b_.qkv, qg, kg, b_.qn, T, st);
            if (!rc) rc = embla_relu2_prefill(b_.qn, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset), b_.o, T, p0 + T,
                                              maxContext_, st);
        } else {   // attn_full_b over the bf16 caches (Prefill.swift:325-338)
            const EmblaAttnB ap{p0, 0, 0, maxContext_};
            rc = embla_attn_full_b(b_.qkv, qg, kg, at(b_.cache, L.kOffset), at(b_.cache, L.vOffset),
                                   static_cast<float*>(b_.qn), b_.counter, b_.o, &ap, T, st);
        }
    }
    if (rc) return rc;
    // the o-projection GEMM into the residual (Prefill.swift:337-339)
    const EmblaSeg& os = L.oproj[0];
    const unsigned long long wo[3] = {os.w, os.s, os.b};
    return embla_gemm_q4(b_.W, wo, b_.o, b_.x, T, d, d, d, d, L.oFirst ? EMBLA_EPI_F32_BF : EMBLA_EPI_ADD, st);
}

}  // namespace embla_host
