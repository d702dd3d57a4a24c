// The attention sub-layer of a decode step, host side, over the library's C ABI.
//
// Mirrors Engine.encodeAttention (Sources/EmblaMetal/Engine.swift:743-832) and the attention parts
// of Engine's state (layer kinds and cache offsets, Engine.swift:269-284, 441-485; the selection
// constants, Engine.swift:7-27): for one layer at position pos, the 4-bit q/k/v projection, the
// int8 append of the new k and v (full and sparse layers' KV jobs), the layer's attention (sliding
// window; full ReLU² with the scores a selecting layer needs and the top-k selection; sparse
// softmax over the selected rows of its block's full-layer cache), then the o-projection into the
// fp32 residual x. Where the reference encodes Metal dispatches with barriers between them, this
// issues stream-ordered calls on one HIP stream; the chunking is the library's.
//
// Ownership as the reference's: the caller owns every buffer (weights, cache, activations,
// workspaces); the engine keeps offsets and launch choices only, allocates nothing and returns the
// first failing call's error code (EMBLA_OK = 0).
#pragma once

#include <cstddef>
#include <cstdint>
#include <set>
#include <vector>

#include "embla_attn.h"

namespace embla_host {

/// Layer kinds (Engine.swift's Layer.kind).
enum class LayerKind { sliding, full, sparse };

/// One attention layer's offsets (Engine.swift:441-485): gains and the cache regions as byte
/// offsets; a sparse layer's regions are its block's full layer's (Engine.swift:461-462).
struct Layer {
    int index = 0;
    LayerKind kind = LayerKind::full;
    size_t qGain = 0, kGain = 0;        // byte offsets of the q and k gains in W (bf16 [128])
    size_t kOffset = 0, vOffset = 0;    // byte offsets of the layer's K and V regions in the cache
    int nGains = 2;                     // gains applied to q in the full and sparse layers
    std::vector<EmblaKVJob> kvJobs;     // the k/v appends this layer owns (full layers)
    std::vector<EmblaSeg> qkv, oproj;   // stacked 4-bit segments of the projections
    bool oFirst = false;                // a block's first layer: the o-projection sets x (EPI 3)
};

/// Device buffers of a step (Engine.swift:252-267): W weights, the cache, hs the projection input
/// (bf16 [2048]), qkv (bf16 [4096]), o (bf16 [16][128]), x the fp32 residual [2048], the split-K
/// workspace (embla_workspace_bytes(maxContext, 16) bytes), scores fp32 [2][maxContext], sel u32
/// [2][topk + recent] and the reference's counter words.
struct Buffers {
    void* W = nullptr;
    void* cache = nullptr;
    void* hs = nullptr;
    void* qkv = nullptr;
    void* o = nullptr;
    float* x = nullptr;
    float* apart = nullptr;
    float* scores = nullptr;
    uint32_t* sel = nullptr;
    uint32_t* counter = nullptr;
};

class AttentionEngine {
public:
    static constexpr int d = 2048, headDim = 128, topk = 1024, recent = 128;   // Engine.swift:7-27

    /// selects: the full layers that score every key for the sparse layers after them
    /// (Embla.selects). kv8: the full layers' caches in int8 with fp32 scales (the reference's
    /// default, Engine.kv8); false: bf16 caches (EMBLA_KV8=0), whose KV jobs carry element
    /// offsets (Engine.swift:457).
    AttentionEngine(int maxContext, Buffers buffers, std::set<int> selects, bool kv8 = true)
        : maxContext_(maxContext), b_(buffers), selects_(std::move(selects)), kv8_(kv8) {}

    /// Engine.encodeAttention: the layer's attention sub-layer at position pos. With kvOnly, only
    /// the q/k/v projection and the k/v append (a prompt token's last layer).
    int encodeAttention(const Layer& L, int pos, hipStream_t stream, bool kvOnly = false) const;

    /// The full layers' int8 keys and values of positions p0 ..< p0 + 128 (p0 % 128 == 0) to or
    /// from a stored block (Engine.fullSpans + copy, PrefixCache.swift:153-200; one launch for every
    /// layer): stored holds embla_kv_block_bytes(layers, 2, EMBLA_F32) bytes in fullSpans' order.
    /// int8 caches only (EMBLA_ERR_UNSUPPORTED without kv8).
    int copyFullBlock(const std::vector<const Layer*>& full, int p0, void* stored, bool save, hipStream_t stream) const;
    /// The sliding layers' ring slots of positions p0 ..< p0 + 128 (Engine.windowSpans' K/V spans):
    /// stored holds embla_ring_block_bytes(layers, 4) bytes.
    int copyWindowBlock(const std::vector<const Layer*>& sliding, int p0, void* stored, bool save,
                        hipStream_t stream) const;

    /// How a step picks its token (Engine.swift:1306-1325): greedy when temperature <= 0 or
    /// top-p <= 0.
    struct Sampling {
        float temperature = 0.0f, topP = 1.0f;
        uint32_t seed = 0;
        bool isGreedy() const { return temperature <= 0.0f || topP <= 0.0f; }
    };
    /// The step's token from the lm-head's fp32 logits (Engine.swift:972-987): the argmax or the
    /// top-p draw, written to greedy[pos], to tokens[pos + 1] past the prompt, and last to the
    /// polled word greedy[-1] (greedy points one word into its buffer). scratch:
    /// embla_sample_workspace_bytes(vocab) bytes.
    int encodeToken(const float* logits, int vocab, uint32_t* tokens, uint32_t* greedy, int pos, int promptEnd,
                    const Sampling& sampling, void* scratch, size_t scratchBytes, hipStream_t stream) const;

    /// Whether a layer at position pos selects (keys past topk + recent) and, for a full layer,
    /// scores (Engine.swift:796-798).
    bool selecting(int pos) const { return pos + 1 > topk + recent; }
    bool scoring(const Layer& L, int pos) const {
        return selecting(pos) && L.kind == LayerKind::full && selects_.count(L.index) > 0;
    }

private:
    int maxContext_;
    Buffers b_;
    std::set<int> selects_;
    bool kv8_;
};

/// Device buffers of a prefill chunk of up to T tokens (Prefill.swift's own buffers): hs bf16
/// [T][2048] the projection input, qkv bf16 [T][4096], qn bf16 [16][T][128] (the full layers'
/// prepared queries), o bf16 [T][2048], x fp32 [T][2048]; W and cache as the decode's.
struct PrefillBuffers {
    void* W = nullptr;
    void* cache = nullptr;
    void* hs = nullptr;
    void* qkv = nullptr;
    void* qn = nullptr;
    void* o = nullptr;
    float* x = nullptr;
    uint32_t* counter = nullptr;   // the reference's counter words (attn_full_b's argument; unused)
};

/// The attention parts of Prefill.encode (Sources/EmblaMetal/Prefill.swift:285-341, 378-407) for
/// one layer and a chunk of T tokens at positions p0 .. p0 + T - 1: the q/k/v GEMM per segment;
/// a sliding layer's ring append with its pre-ops and windowed attention (kv_sliding_b +
/// attn_sliding8_b); a full or sparse layer's int8 append, q preparation and causal ReLU² attention
/// with sink over every key (kv_append_b, q_prep_b, relu2_prefill_nax: the reference prefills its
/// sparse layers with the full layers' kernel too; without kv8, kv_append_b and attn_full_b over
/// bf16 caches, Prefill.swift:315-338, with qn as attn_full_b's part buffer); then the o-projection
/// GEMM into x.
class PrefillEncoder {
public:
    PrefillEncoder(int maxContext, PrefillBuffers buffers, bool kv8 = true)
        : maxContext_(maxContext), b_(buffers), kv8_(kv8) {}
    /// With kvOnly, only the q/k/v GEMM and the k/v append (the prompt's last layer, Prefill.swift:287,
    /// 323).
    int encode(const Layer& L, int p0, int T, hipStream_t stream, bool kvOnly = false) const;

private:
    int maxContext_;
    PrefillBuffers b_;
    bool kv8_;
};

}  // namespace embla_host
