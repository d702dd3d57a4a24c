// Host-side argument records shared by the C ABI layer (api.cpp) and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include "../../include/embla_attn.h"

namespace embla {

struct FullDecodeArgs {
    const uint16_t* q;   // prepared fp16 queries [n_q][128]
    const int8_t* kc;
    const int8_t* vc;
    float* part;         // [C][n_q][132] chunk partials
    float* scores;       // optional
    uint16_t* o;
    int S, CH, C, max_s, n_q, n_kv;
    bool relu2, scale32, out_bf16;
    // raw queries (ng >= 0): q holds bf16 rows [n_q][128] straight from the q/k/v projection; the
    // kernel applies the head norm with ng (0-2) gains g1, g2 and the bf16 rounding itself
    const uint16_t* g1 = nullptr;
    const uint16_t* g2 = nullptr;
    int ng = -1;
    bool merge = true;   // false: leave the chunk partials (C > 1) for a later merge
    // the decode step's own append (append): the new token's bf16 k, v rows [n_kv][128] quantised
    // into the writable regions kcw, vcw at position pos, and added as partial C; S = pos keys
    bool append = false;
    const uint16_t* knew = nullptr;
    const uint16_t* vnew = nullptr;
    int8_t* kcw = nullptr;
    int8_t* vcw = nullptr;
    int pos = 0;
    int norm_k = 0;
};
int launch_full_decode(const FullDecodeArgs& a, hipStream_t st);
/// Validates embla_decode_int8's arguments and fills a (chunking included) except a.part;
/// rc != 0 on a bad argument (api.cpp).
int full_decode_plan(const void* q, const void* kc, const void* vc, void* o, float* scores, int S, int max_s, int n_q,
                     int n_kv, int weights, int scale_dtype, int out_dtype, int chunk, FullDecodeArgs& a);
/// The new token's append and partial as the kernel's extra workgroup reads them.
struct DecodeAppend {
    const uint16_t* k;
    const uint16_t* v;
    int8_t* kc;
    int8_t* vc;
    int pos, norm_k;
};
/// The merge launch_full_decode ends with, on its own (a.C > 1, partials in a.part).
int launch_full_decode_merge(const FullDecodeArgs& a, hipStream_t st);
/// Merges C chunk partials into o [n_q][128]: fp32 records [C][n_q][132] whose sums carry a factor
/// oscale, or (h16) the int8 decode's records [C][n_q][68] (O / l as fp16, then m and l).
int launch_decode_merge(const float* part, uint16_t* o, int C, int n_q, bool relu2, bool out_bf16, float oscale,
                        hipStream_t st, bool h16 = false);

struct RingArgs {
    const uint16_t* q;       // head h's row at q + h * q_stride
    int q_stride;
    const uint16_t* k_new;   // kv head h at + h * 128
    const uint16_t* v_new;
    const uint16_t* qg;      // gains (pre-ops only)
    const uint16_t* kg;
    uint16_t* kring;         // [n_kv][R/32] tiles, ES = 2
    uint16_t* vring;
    float* part;
    uint16_t* o;
    int pos, W, R, CH, C, n_q, n_kv;
    bool bf16, preops;
};
int launch_ring_decode(const RingArgs& a, hipStream_t st);

struct SparseArgs {
    const uint16_t* q;       // [n_q][128]
    const uint16_t* kc;      // 16-bit rows [n_kv][max_s][128]
    const uint16_t* vc;
    const uint32_t* idx;     // rows of kv head h at idx + h * idx_stride (stride 0: one set); null: 0 .. nsel-1
    int idx_stride, nsel;
    float* part;
    uint16_t* o;
    int CH, C, max_s, n_q, n_kv;
    bool bf16;
    // Non-null sel_ws: rows 0 .. sel_topk - 1 are the wide select's output, its last step run by
    // each workgroup for the ranks it attends (idx unused, CH <= 256), and rows sel_topk .. nsel - 1
    // are keys sel_n .. (the recent ones). sel_out (optional) receives the selection in
    // select_keys' order; the select's epoch word is advanced once.
    const uint32_t* sel_ws = nullptr;
    int sel_n = 0, sel_topk = 0;
    uint32_t* sel_out = nullptr;
    uint32_t* sel_epoch = nullptr;
};
int launch_sparse_decode(const SparseArgs& a, hipStream_t st);
constexpr int kSparseFusedMaxCh = 256;    // keys a workgroup with the select's last step fused
constexpr int kWideSelectMaxN = 32768;    // candidates a set of the wide select

/// Gathered softmax attention over an int8 cache: query row r (position p0 + r) attends the keys
/// idx[r][0 .. nsel) (at idx + r * idx_row_stride + kv head * idx_kv_stride) when p0 + r + 1 > nsel,
/// else keys 0 .. p0 + r. The cache is row-major ([n_kv][max_s][128] int8, the sparse prefill's) or
/// MFMA tiles (the full layer's decode cache: tiles), then the scales (fp16, or fp32 with
/// scale32). Keys split into C chunks of CH: C > 1 writes partials (one row, R == 1) for the merge.
struct SparseRows8Args {
    const uint16_t* q;       // row r, head h at q + r * q_row_stride + h * 128 (fp16 or bf16)
    long q_row_stride;
    const int8_t* kc;
    const int8_t* vc;
    const uint32_t* idx;
    long idx_row_stride, idx_kv_stride;
    int nsel, p0, R;
    uint16_t* o;             // row r, head h at o + r * o_row_stride + h * 128
    long o_row_stride;
    float* part;             // [C][n_q][132] when C > 1
    int CH, C;
    int max_s, n_q, n_kv;
    bool q_bf16, o_bf16, tiles, scale32;
};
int launch_sparse_rows8(const SparseRows8Args& a, hipStream_t st);

/// Approximate index scores of T rows (4 fp16 index heads of 64 dims, fp32 weights) against keys
/// 0 .. ld-1 (zero past nk), as the top 16 bits of their order bits, and each key chunk's largest
/// key norm (kmax[c], chunk c = keys c * kchunk ..).
struct IndexMfmaArgs {
    const uint16_t* qi;   // [T][4][64]
    const float* w;       // [T][4]
    const uint16_t* ki;   // [nk][64]
    uint16_t* keys;       // [T][ld]
    float* kmax;          // [ld / kchunk]
    int T, nk, ld, kchunk;
    int lim0;             // row t's candidates are keys < t + lim0; the rest are stored as 0
};
int launch_index_mfma(const IndexMfmaArgs& a, hipStream_t st);

/// Row t (position p0 + t, S = p0 + t + 1 keys) selects, when S > topk + recent, the topk keys of
/// [0, S - recent) by the spec score, in select_keys' order, then the recent ones: idx[t][..].
struct BandSelectArgs {
    const uint16_t* keys;  // [T][ld] from index_mfma
    int ld;
    const uint16_t* qi;
    const float* w;
    const uint16_t* ki;
    const float* kmax;
    int nchunks;
    uint32_t* idx;
    int idx_stride;
    int T, p0, topk, recent;
    uint32_t* ovf;         // [T][2]: a row's band bounds {kin, kout} when its band overflows, else {0, 0}
};
int launch_select_band(const BandSelectArgs& a, hipStream_t st);
int launch_select_topk(const float* scores, int score_stride, uint32_t* idx, int idx_stride, int S, int n_sets,
                       int topk, int recent, hipStream_t st);
struct PrefillArgs {
    const uint16_t* q;       // row (token t, head h) at q + t * q_tok_stride + h * q_head_stride
    long q_tok_stride, q_head_stride;
    const int8_t* kc;        // int8 regions (tiles, then scales)
    const int8_t* vc;
    uint16_t* o;             // row (t, h) at o + t * o_tok_stride + h * o_head_stride
    long o_tok_stride, o_head_stride;
    int T, p0, max_s, n_q, n_kv, window;
    int nsplit;              // key-range splits (> 1: partial rows in part, then a merge)
    float* part;             // [nsplit][T][n_q] records of 68 floats: O / l (128 fp16), m, l, pad
    bool relu2, scale32, q_bf16, out_bf16;
    // 16-bit ring source (kring/vring non-null): keys at slot p % R, no scales, MFMA in the ring's type
    const uint16_t* kring;
    const uint16_t* vring;
    int R;
    const uint16_t* qg;      // q pre-ops (norm with gains, RoPE, bf16), ring mode only; null: none
};
int launch_prefill_int8(const PrefillArgs& a, hipStream_t st);
int launch_prefill_ring(const PrefillArgs& a, hipStream_t st);
/// Prefill over the int8 region a.kc / a.vc through its staged fp16 copy k16, v16 ([n_kv][R] tiles
/// of 16-bit elements, R a multiple of 128 >= p0 + T): the staging pass, then the attention.
int launch_prefill_prestaged(const PrefillArgs& a, uint16_t* k16, uint16_t* v16, int R, hipStream_t st);

int launch_index_scores(const uint16_t* qi, const float* w, const uint16_t* ki, float* scores, int n, int n_ih,
                        hipStream_t st, uint32_t* sw = nullptr);
/// Words (4 bytes) of the wide select's workspace: two histogram buffers (WSEL_NCP copies of 256
/// coarse bins), counters (first digit, keys above it, epoch), the candidate counts of the
/// classify workgroups, the bitmap and their candidate regions (1024 pairs each), then the scorer
/// workgroups' fine-bin rows.
#ifndef WSEL_NCP
#define WSEL_NCP 16   // histogram copies of the wide select (C4 step: 8 -> 32.1 us, 16 -> 29.5, 32 -> 29.6, 64 -> 31.4)
#endif
constexpr size_t kWideSelectFine = 2 * WSEL_NCP * 256 + 64 + 32768 / 1024 + 32768 / 32 + 2 * 32768;
constexpr int kWideSelectScorers = 128;   // scorer workgroups at most (32768 keys, 256 a workgroup)
/// Workgroups of index_scores_kernel for n keys (256 keys a workgroup, at most 1024): the scorer's
/// grid, and with the wide select the number of fine-bin rows it leaves.
__host__ __device__ constexpr int index_score_blocks(int n) {
    return ((n + 63) / 64 + 3) / 4 < 1 ? 1 : (((n + 63) / 64 + 3) / 4 > 1024 ? 1024 : ((n + 63) / 64 + 3) / 4);
}
/// + the scorer workgroups' own fine-bin rows (uint16 [kWideSelectScorers][4096])
constexpr size_t kWideSelectWords = kWideSelectFine + (size_t)kWideSelectScorers * 4096 / 2;
constexpr size_t kWideSelectEpoch = 2 * WSEL_NCP * 256 + 3;   // the epoch word's index
constexpr size_t kWideSelectRecounts = 2 * WSEL_NCP * 256 + 4;   // calls that found a stale histogram
/// Index scores of keys [0, S - recent) and the first steps of their exact top-k on many
/// workgroups (one set): the scores' histogram, then the first digit of the topk-th value, the
/// bitmap of keys above it and the candidates in it. The last step is the consumer's
/// (SparseArgs::sel_ws, wsel_slice), which also advances the epoch. sw: kWideSelectWords words,
/// zero before the first call.
int launch_wide_select(const uint16_t* qi, const float* w, const uint16_t* ki, float* scores, int S, int n_ih,
                       int topk, int recent, uint32_t* sw, hipStream_t st);

struct KVQuantArgs {
    const uint16_t* k;   // [T] rows of k, row stride `stride` elements, kv head h at h * 128
    const uint16_t* v;
    int stride;
    int T, p0, n_kv, max_s;
    int8_t* kc;
    int8_t* vc;
    bool in_bf16, scale32, norm_k;
    bool row_major;      // rows [n_kv][max_s][128] (the sparse layer's gathered cache), else MFMA tiles
};
int launch_kv_quant(const KVQuantArgs& a, hipStream_t st);

struct QPrepArgs {
    const uint16_t* qraw;   // bf16 [T] rows, row stride `stride`, head h at h * 128
    const uint16_t* g1;     // optional gains (bf16 [128])
    const uint16_t* g2;
    int ng, stride, T, n_q;
    uint16_t* out;          // [T][n_q][128] fp16 or bf16; head-major [n_q][T][128] with head_major
    bool out_bf16;
    bool head_major = false;
};
int launch_q_prep(const QPrepArgs& a, hipStream_t st);

struct RingAppendArgs {
    const uint16_t* k;       // rows t at + t * stride, head h at + h * 128 (16-bit)
    const uint16_t* v;
    int stride, T, p0, n_kv, R;
    uint16_t* kring;
    uint16_t* vring;
    const uint16_t* kg;      // gains: bf16 pre-ops on K (norm, RoPE); null: copy
    bool norm_k = false;     // without gains: K RMS-normed (no gains, no RoPE) and rounded to bf16
};
int launch_ring_append(const RingAppendArgs& a, hipStream_t st);

/// Decode over a bf16 full-layer cache in the 16-bit tile layout (decode_full16.hip).
struct Full16Args {
    const uint16_t* q;       // raw bf16 queries [n_q][128], normed with ng gains in the kernel
    const uint16_t* g1;
    const uint16_t* g2;
    int ng;
    const uint16_t* kc;      // [n_kv][max_s/32] tiles of 32 x 128 bf16
    const uint16_t* vc;
    const uint32_t* idx;     // SEL: rows [n_kv][S]; null: keys 0 .. S-1
    float* part;             // [C][n_q][132] chunk partials
    float* scores;           // optional [n_kv][max_s]: max over a kv head's query heads of q·k
    uint16_t* o;             // bf16 [n_q][128]
    int S, CH, C, max_s, n_q, n_kv;
    bool relu2;
};
int launch_full16_decode(const Full16Args& a, hipStream_t st);

/// A prefix-cache block copy (blocks.hip): 128 positions of every listed layer's K and V region.
constexpr int kMaxBlockLayers = 64;
struct BlockCopyArgs {
    char* cache;
    char* stored;
    unsigned long long off[2 * kMaxBlockLayers];   // byte offsets of each layer's K, V region
    int n_layers, n_kv, max_s, p0;                 // the ring: max_s = ring length, p0 = slot
    int elem;          // bytes an element: 1 (int8 cache) or 2 (16-bit ring)
    int row_units;     // 16-byte units of a head's 128 rows: 128 * 128 * elem / 16
    int scale_bytes;   // bytes a scale (0: none)
    int scale_units;   // 16-byte units of a head's 128 scales
    int save;          // cache -> stored, else stored -> cache
};
int launch_block_copy(const BlockCopyArgs& a, hipStream_t st);

/// The 4-bit projections (gemv_q4.hip): stacked segments, as gemv.metal's Seg.
constexpr int kMaxGemvSegs = 8;
struct GemvSeg {
    unsigned long long w, s, b;   // byte offsets in W of the segment's words, scales, biases
    unsigned int end, x, y, pad;  // end row (exclusive, a multiple of 4); input, output element offsets
};
struct GemvArgs {
    const void* W;
    const void* X;   // bf16
    void* Y;
    GemvSeg seg[kMaxGemvSegs];
    int nseg, K;
};
int launch_gemv_q4(const GemvArgs& a, int epi, hipStream_t st);

/// The prefill projections (gemm_q4.hip): Y [T][ldy] = X [T][ldx] W^T, W 4-bit at byte offsets.
struct GemmArgs {
    const void* W;
    unsigned long long wo, so, bo;   // byte offsets in W of the words, scales, biases
    const uint16_t* X;               // bf16
    void* Y;
    int T, O, K, ldx, ldy;
};
int launch_gemm_q4(const GemmArgs& a, int epi, hipStream_t st);

/// The sampling tail (sample.hip). Workspace: the capped row as bf16, then the block maxima and
/// their indices (64 each) and 64 block records of 32 bytes, then a 1024-word candidate list a block.
inline size_t sample_ws_off_blk(int V) { return ((size_t)V * 2 + 255) / 256 * 256; }
inline size_t sample_ws_off_cand(int V) { return sample_ws_off_blk(V) + 2560; }
inline size_t sample_ws_bytes(int V) { return sample_ws_off_cand(V) + (size_t)((V + 1023) / 1024) * 4096; }
int launch_argmax(const float* logits, int V, uint32_t* token, uint32_t* greedy, int pos, int prompt, char* ws,
                  hipStream_t st);
int launch_sample(const float* logits, int V, uint32_t* token, uint32_t* greedy, int pos, int prompt, float inv_t,
                  float top_p, uint32_t seed, char* ws, hipStream_t st);

}  // namespace embla
