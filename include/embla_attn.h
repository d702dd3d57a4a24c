/* embla_attn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Every entry point takes device pointers the caller owns, a hipStream_t, and returns 0 or a
 * negative EMBLA_ERR_* code. Arguments are validated on the host before any launch; nothing
 * throws or aborts across this boundary, nothing allocates, nothing synchronises the host.
 * Calls are stream-ordered and asynchronous. A workspace (split-K partials) is thread-compatible,
 * not thread-safe: one in-flight call per workspace. Calls keep no state in it between calls, so
 * they can be captured in a HIP graph.
 *
 * Head dim is 128. Cache layouts (one layer): an int8 K (or V) region is the 32-key tiles of
 * every kv head, [n_kv][max_s/32][4096] bytes, then the scales [n_kv][max_s] (fp16 or fp32).
 * Inside a tile the bytes are in MFMA lane order, so a wave reads each tile as contiguous 1 KB
 * runs (element (key k, dim d) of a tile; ES = element size):
 *   K: k = 16t + m: byte ((t*2ES + p/16) * 64 + m + 16*(d/32)) * 16 + p%16, p = (d%32)*ES
 *   V: k = 16t + 4g + i, d = 8n + u: byte ((p/16) * 64 + n + 16g) * 16 + p%16, p = (8u+4t+i)*ES
 * A region has the byte size and scale offset of the reference's KV8 layout
 * (Sources/EmblaMetal/Kernels/common.metal:53-63; Engine.swift:277-281), so an engine's per-layer
 * offsets hold. max_s must be a multiple of 32. 16-bit rings use the same tiles with ES = 2.
 */
#ifndef EMBLA_ATTN_H
#define EMBLA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define EMBLA_OK 0
#define EMBLA_ERR_INVALID (-1)     /* an argument out of range (checked on the host) */
#define EMBLA_ERR_UNSUPPORTED (-2) /* a combination no kernel is built for */
#define EMBLA_ERR_HIP (-3)         /* the HIP runtime reported an error at launch */
#define EMBLA_ERR_WORKSPACE (-4)   /* workspace missing or too small */

/* element types */
#define EMBLA_F16 0
#define EMBLA_BF16 1
#define EMBLA_F32 2

/* attention weights */
#define EMBLA_SOFTMAX 0    /* softmax(q·k / sqrt(128)) */
#define EMBLA_RELU2_SINK 1 /* w = relu(q·k / sqrt(128))^2, o = Σ w v / (sqrt(128) + Σ w) */

/* Mirrors AttnParams (Sources/EmblaMetal/Kernels/attention.metal:8-16; Engine.swift:37-39)
 * field for field. CH = 0 lets the library choose the chunking. */
typedef struct EmblaAttnParams {
    int32_t S, CH, C, maxS, pos, ng, pad0, pad1;
} EmblaAttnParams;

/* Mirrors AttnB (prefill.metal:217; Prefill.swift:327-328) field for field. */
typedef struct EmblaAttnB {
    int32_t p0, CH, C, maxS;
} EmblaAttnB;

/* Mirrors KVJob (attention.metal:108-111; Engine.swift:35): element offsets of k and v in qkv
 * and byte offsets of the layer's K and V regions in the cache. */
typedef struct EmblaKVJob {
    uint32_t k, v, kc, vc;
} EmblaKVJob;

/* Library version, for a host to check it loaded what it was built against. */
int embla_version(void);

/* Bytes of workspace for decode calls with up to max_s keys and n_q query heads. */
size_t embla_workspace_bytes(int max_s, int n_q);
/* Zeroes a workspace's reserved header (optional; kept for engines that initialise buffers). */
int embla_workspace_init(void* ws, size_t ws_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- decode, int8 cache
 * One query token attends keys 0 .. S-1 of an int8 layer cache, split over chunks of keys whose
 * partials a second kernel merges (one launch when a single chunk covers S). Replaces the dispatches of attn_full8 and
 * attn_sparse8 without selection (attention.metal:235-363, 448-584) made by
 * Engine.encodeAttention (Engine.swift:795-818).
 *   q       fp16 [n_q][128], prepared (normed/gained where the model does that)
 *   o       [n_q][128] in out_dtype (EMBLA_F16 or EMBLA_BF16)
 *   scores  optional [n_kv][max_s] fp32: max over a kv head's query heads of q·k·scale_k
 *           (the reference's SCORES output, attention.metal:295-305); only with RELU2_SINK
 *   weights EMBLA_SOFTMAX or EMBLA_RELU2_SINK; scale_dtype EMBLA_F16 or EMBLA_F32
 *   chunk   keys a workgroup (multiple of 32), 0 = library's choice */
int embla_decode_int8(const void* q, const void* kc, const void* vc, void* o, float* scores,
                      int S, int max_s, int n_q, int n_kv, int weights, int scale_dtype,
                      int out_dtype, int chunk, void* ws, size_t ws_bytes, hipStream_t stream);

/* embla_decode_int8 as its two launches, for a caller that merges later or times the split-K
 * kernel alone: _partials runs the chunks (at least two) and leaves their partials in ws;
 * _merge reads them and writes o. Same arguments as embla_decode_int8 (the merge's S, max_s,
 * n_q, n_kv, weights, out_dtype and chunk as the partials call's); nothing may touch ws between
 * the two. No counterpart in the reference, whose arrive_last step merges inside the kernel
 * (common.metal:86-99). */
int embla_decode_int8_partials(const void* q, const void* kc, const void* vc, float* scores, int S, int max_s,
                               int n_q, int n_kv, int weights, int scale_dtype, int out_dtype, int chunk, void* ws,
                               size_t ws_bytes, hipStream_t stream);
int embla_decode_int8_merge(void* o, int S, int max_s, int n_q, int n_kv, int weights, int out_dtype, int chunk,
                            void* ws, size_t ws_bytes, hipStream_t stream);

/* embla_decode_int8 without a workspace argument, for callers that cannot allocate (code under
 * HIP graph capture, serving loops or harnesses that forbid hipMalloc). No counterpart in the
 * reference. The split-K partials go to a file-scope device array of
 * embla_decode_int8_noalloc_max_bytes() bytes (4.125 MiB: C chunks x n_q x 528 B must fit, or the
 * call returns EMBLA_ERR_WORKSPACE). The call allocates nothing; each GPU holds one array for the
 * life of the process, resolved on that GPU's first call. Calls that overlap on one GPU (other
 * streams or threads) share that array and race; calls ordered on one stream do not. */
int embla_decode_int8_noalloc(const void* q, const void* kc, const void* vc, void* o, float* scores, int S,
                              int max_s, int n_q, int n_kv, int weights, int scale_dtype, int out_dtype,
                              int chunk, hipStream_t stream);
size_t embla_decode_int8_noalloc_max_bytes(void);

/* Reference-signature full layer (attn_full8, attention.metal:235-363; bound at Engine.swift:
 * 800-818): raw bf16 q [16][128] normed with p->ng gains g1, g2 (common.metal:13-26) and rounded
 * to bf16, ReLU² with sink over the int8 cache of 2 kv heads with fp32 scales; o bf16 [16][128].
 * scores may be NULL (the SCORES=0 pipeline). part: a workspace of embla_workspace_bytes(maxS, 16)
 * bytes; `counter` (the reference's split-K counters) is accepted and not used: the chunk
 * partials are merged by a second kernel. */
int embla_attn_full8(const void* qraw, const void* g1, const void* g2, const void* kc,
                     const void* vc, float* part, float* scores, uint32_t* counter, void* o,
                     const EmblaAttnParams* p, hipStream_t stream);

/* ---------------------------------------------------------------- sliding window over a ring
 * One query token attends the last min(pos + 1, window) positions, the current one included, of
 * a 16-bit ring of `ring` slots a kv head (position p at slot p % ring; K and V in the tile layout
 * with ES = 2); the current k, v are written into slot pos % ring. Softmax, scale 1/sqrt(128).
 * q [n_q][128], k_new, v_new [n_kv][128], o [n_q][128], all in dtype (EMBLA_F16 or EMBLA_BF16).
 * window <= ring, ring a multiple of 32; chunk: ring keys a workgroup (0 = library's choice);
 * ws as embla_decode_int8 (sized for max_s = ring), unused when one chunk covers the window.
 * The BASELINE config C2 (fp16 ring of 8192, window 1024) runs through this. */
int embla_sliding_decode(const void* q, const void* k_new, const void* v_new, void* kring, void* vring,
                         void* o, int pos, int window, int ring, int n_q, int n_kv, int dtype, int chunk,
                         void* ws, size_t ws_bytes, hipStream_t stream);

/* Reference-signature sliding layer (attn_sliding, attention.metal:26-102; bound at
 * Engine.swift:771-780): qkv bf16 [q 16*128 | k 4*128 | v 4*128]; q and k RMS-normed with gains
 * qg / kg (ng = 1) and rotated (RoPE, common.metal:39-47), rounded to bf16; window 128 over a bf16
 * ring of 4096 (kc, vc in the tile layout); o bf16 [16][128]. */
int embla_attn_sliding(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o,
                       int pos, hipStream_t stream);

/* ---------------------------------------------------------------- sparse layers: selection
 * Index scores (the BASELINE configs' indexer): scores[j] = Σ_h w_h relu(qi_h·ki_j)² for
 * j < n, qi fp16 [n_ih][64], w fp32 [n_ih], ki fp16 [n][64], n_ih in {1, 2, 4}. The fp32 order
 * is fixed (so the top-k is reproducible): 8 fma chains over dims 8k .. 8k+7, combined as
 * ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)); r = max(dot, 0); s = fma(w_h, r*r, s) from h = 0. */
int embla_index_scores(const void* qi, const float* w, const void* ki, float* scores, int n, int n_ih,
                       hipStream_t stream);

/* Exact top-k (select_keys, attention.metal:647-744), n_sets sets: among keys [0, S - recent) of
 * set i (scores + i * score_stride) the topk largest (order-preserving float bits; ties go to the
 * lower index), written to idx + i * idx_stride as: keys above the topk-th value in index order,
 * then the first keys equal to it in index order, then S - recent .. S - 1. Requires
 * S > topk + recent and S - recent <= 33024. */
int embla_select_topk(const float* scores, int score_stride, uint32_t* idx, int idx_stride, int S, int n_sets,
                      int topk, int recent, hipStream_t stream);

/* Reference-signature select_keys (attention.metal:680-744, bound at Engine.swift:819-827):
 * 2 sets, scores [2][maxS], idx [2][1152], topk 1024, recent 128. */
int embla_select_keys(const float* scores, uint32_t* idx, int S, int maxS, hipStream_t stream);

/* Softmax decode over gathered 16-bit rows (attn_sparse with SEL, attention.metal:370-441): kv head
 * h attends rows idx[h * idx_stride + j], j < nsel (idx_stride 0: one set for every kv head; idx
 * NULL: rows 0 .. nsel-1) of row-major caches kc, vc [n_kv][max_s][128] in dtype; q, o
 * [n_q][128]. ws: embla_workspace_bytes(32 * chunks, n_q), unused with one chunk. */
int embla_sparse_decode(const void* q, const void* kc, const void* vc, const uint32_t* idx, int idx_stride,
                        int nsel, void* o, int max_s, int n_q, int n_kv, int dtype, int chunk, void* ws,
                        size_t ws_bytes, hipStream_t stream);

/* Bytes of workspace for embla_sparse_layer_decode: zero-fill it before its first use (every call
 * leaves its counters clean for the next). A workspace that is not clean (never zeroed,
 * overwritten, or left by a call stopped between its kernels) never yields a wrong selection: the
 * select checks that its histogram counts exactly this call's keys and otherwise recounts them
 * from the scores (that call is slower; the next is clean again). The 32-bit word at
 * embla_sparse_workspace_recount_offset(max_s, n_q) counts such calls. */
size_t embla_sparse_workspace_bytes(int max_s, int n_q);
/* Byte offset, in embla_sparse_layer_decode's workspace, of its count of recounted calls (no
 * counterpart in the reference: it lets a caller audit the workspace's state). */
size_t embla_sparse_workspace_recount_offset(int max_s, int n_q);
/* The workspace's audit (no counterpart in the reference): waits for the stream, returns
 * EMBLA_ERR_WORKSPACE if any call since the last audit found the workspace not clean (its
 * selection was still exact: the select recounted), EMBLA_OK if none did, and clears the count.
 * The only entry point that synchronises the host. */
int embla_sparse_workspace_audit(void* ws, size_t ws_bytes, int max_s, int n_q, hipStream_t stream);

/* One sparse-layer decode step (config C4): with S > 1152 keys, index scores of keys
 * [0, S - 128), the top 1024 plus the latest 128, then attention over those 1152 rows; with
 * S <= 1152 attention over every key (Engine.swift:796-818). */
int embla_sparse_layer_decode(const void* q, const void* qi, const float* w, const void* ki, const void* kc,
                              const void* vc, void* o, int S, int max_s, int n_q, int n_kv, int n_ih, int dtype,
                              void* ws, size_t ws_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- batched prefill, int8 cache
 * T tokens at positions p0 .. p0+T-1 attend keys 0 .. their position (window > 0: only the last
 * `window` positions, the own one included) of an int8 layer cache that already holds them.
 * Query row (t, h) at q + t * q_tok_stride + h * q_head_stride (elements, q_dtype), output row at
 * o + t * o_tok_stride + h * o_head_stride (o_dtype). weights: EMBLA_SOFTMAX, or EMBLA_RELU2_SINK
 * (threshold 0, sink sqrt(128), as relu2_prefill_nax, attn_nax.metal:61-364). n_q / n_kv in {4, 8}.
 * ws (optional, embla_prefill_workspace_bytes(T, n_q)): lets the key range split in two (partial
 * rows merged by a second launch) so the GPU holds two waves a SIMD; NULL: one pass. */
int embla_prefill_int8(const void* q, int q_dtype, long q_tok_stride, long q_head_stride, const void* kc,
                       const void* vc, void* o, int o_dtype, long o_tok_stride, long o_head_stride, int T, int p0,
                       int max_s, int n_q, int n_kv, int weights, int scale_dtype, int window, void* ws,
                       size_t ws_bytes, hipStream_t stream);

/* Bytes of the optional prefill workspace for T tokens and n_q query heads. */
size_t embla_prefill_workspace_bytes(int T, int n_q);

/* Bytes of a prefill workspace that also holds an fp16 copy of the layer's keys 0 .. p0+T-1 (no
 * counterpart in the reference, whose threadgroups each widen the int8 rows they stage,
 * attn_nax.metal:26-56): embla_prefill_int8 / embla_prefill_full given at least this much convert
 * the region once into it, bit-identical products, and attend over the copy (softmax, fp16
 * scales, bf16 q and out, n_q = 4 n_kv, no window; other calls ignore the extra bytes). */
size_t embla_prefill_staged_workspace_bytes(int T, int p0, int n_q, int n_kv);

/* Full-layer prefill chunk (config C5 full): the chunk's bf16 K and V [T][n_kv][128] quantised into
 * the int8 cache (fp16 per-token absmax scales) at p0 .., then causal softmax attention of the bf16
 * queries [T][n_q][128] over keys 0 .. p0 + t; o bf16 [T][n_q][128]; ws as embla_prefill_int8. */
int embla_prefill_full(const void* q, const void* k, const void* v, void* kc, void* vc, void* o, int T, int p0,
                       int max_s, int n_q, int n_kv, void* ws, size_t ws_bytes, hipStream_t stream);

/* Reference-signature relu2_prefill_nax (attn_nax.metal:61-364, bound at Prefill.swift:389-406):
 * qn bf16 [16][Tq][128] from q_prep_b, the int8 cache of 2 kv heads (fp32 scales), keys 0 .. Tk-1,
 * the chunk being the last Tq of them; out bf16 token-major [Tq][2048]. */
int embla_relu2_prefill(const void* qn, const void* kc, const void* vc, void* o, int Tq, int Tk, int maxS,
                        hipStream_t stream);

/* ---------------------------------------------------------------- batched prefill, 16-bit ring
 * 16-bit K, V rows of T positions p0 .. into a ring (slot p % ring, tile layout with ES = 2).
 * kg != NULL (bf16 only): K rows are RMS-normed with gains kg, rotated (RoPE at their position)
 * and rounded to bf16 first, as kv_sliding_b (prefill.metal:103-125). Rows at (t * stride + h * 128). */
int embla_ring_append(const void* k, const void* v, int dtype, int stride, int T, int p0, int n_kv, void* kring,
                      void* vring, int ring, const void* kg, hipStream_t stream);

/* Sliding-window prefill over a 16-bit ring that already holds the chunk: T tokens at p0 .. attend
 * their last `window` positions (the own one included), softmax. dtype EMBLA_BF16 or EMBLA_F16 for
 * q, ring and o; strides as embla_prefill_int8. qg != NULL (bf16): q is normed with gains qg,
 * rotated and rounded to bf16 in the kernel (attn_sliding8_b, prefill.metal:428-548). Requires
 * window - 1 + T <= ring. ws optional (embla_prefill_workspace_bytes). */
int embla_prefill_ring(const void* q, int dtype, long q_tok_stride, long q_head_stride, const void* kring,
                       const void* vring, int ring, void* o, long o_tok_stride, long o_head_stride, int T, int p0,
                       int n_q, int n_kv, int window, const void* qg, void* ws, size_t ws_bytes, hipStream_t stream);

/* Sliding-layer prefill chunk (config C5 sliding): bf16 K, V [T][n_kv][128] appended to the bf16 ring,
 * then windowed softmax attention of q [T][n_q][128]; o bf16 [T][n_q][128]. */
int embla_prefill_sliding(const void* q, const void* k, const void* v, void* kring, void* vring, void* o, int T,
                          int p0, int ring, int window, int n_q, int n_kv, void* ws, size_t ws_bytes,
                          hipStream_t stream);

/* Reference-signature sliding prefill: kv_sliding_b then attn_sliding8_b (prefill.metal:103-125,
 * 428-548; Prefill.swift:291-313): qkv bf16 [T][4096], gains qg, kg, bf16 rings kc, vc of 4096 slots
 * (tile layout), window 128; o bf16 token-major [T][2048]. */
int embla_attn_sliding8_b(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o, int p0, int T,
                          hipStream_t stream);

/* attn_sliding_b (prefill.metal:129-180), the reference's scalar sliding prefill chosen with
 * SLIDING8=0 (Prefill.swift:27-31, 311-312): the same ring writes and the same attention as
 * embla_attn_sliding8_b, which it calls. */
int embla_attn_sliding_b(const void* qkv, const void* qg, const void* kg, void* kc, void* vc, void* o, int p0, int T,
                         hipStream_t stream);

/* ---------------------------------------------------------------- sparse-layer batched prefill
 * Config C5's sparse layer: T rows at p0 .. (q bf16 [T][n_q][128]); the chunk's K, V (bf16
 * [T][n_kv][128]) are quantised into a ROW-MAJOR int8 cache (kc, vc: [n_kv][max_s][128] int8, then
 * fp16 scales [n_kv][max_s]: the layout a gathering reader wants). Row t (S = p0 + t + 1 keys)
 * selects, when S > 1152, the top 1024 of keys [0, S - 128) by the ReLU² index score (index queries
 * qi fp16 [T][4][64], weights w f32 [T][4], index keys ki fp16 [p0 + T][64]; the score is
 * embla_index_scores' spec, bit for bit) plus the latest 128, in select_keys' order, else all S
 * keys; softmax attention over those rows gives o bf16 [T][n_q][128]. idx (optional, [T][1152]
 * u32) receives the selection. ws: embla_sparse_prefill_workspace_bytes(T, p0). Requires
 * p0 + T - 128 <= 32768. */
size_t embla_sparse_prefill_workspace_bytes(int T, int p0);
int embla_prefill_sparse(const void* q, const void* k, const void* v, const void* qi, const float* w, const void* ki,
                         void* kc, void* vc, void* o, uint32_t* idx, int T, int p0, int max_s, int n_q, int n_kv,
                         void* ws, size_t ws_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- quantise-and-append
 * T new positions p0 .. p0+T-1 of K and V rows into an int8 layer cache (write_row8,
 * common.metal:72-84; kv_append / kv_append_b, attention.metal:113-140, prefill.metal:182-212):
 * a = max|x|, q = rint(x * 127 / a), scale = a / 127 stored in scale_dtype. k and v point at row 0
 * head 0; row t head h is at (t * stride + h * 128) elements; in_dtype EMBLA_BF16 or EMBLA_F16
 * (bf16 inputs are rounded to bf16 after the norm, as the reference's bf()). norm_k: RMS-norm K
 * rows first (no gains, eps 2^-23), as the reference's full layers. */
int embla_kv_quant_append(const void* k, const void* v, int in_dtype, int stride, int T, int p0,
                          int n_kv, void* kc, void* vc, int max_s, int scale_dtype, int norm_k,
                          hipStream_t stream);

/* Reference-signature sparse layer decode (attn_sparse8, attention.metal:448-584; Engine.swift:
 * 799-818): q as embla_attn_full8 (raw bf16 with ng gains), 2 kv heads of the block's full layer's
 * int8 cache (tile layout, fp32 scales), softmax. idx == NULL (SEL = 0): keys 0 .. p->S-1; else
 * (SEL = 1) the rows idx[kv head][0 .. p->S) (u32 [2][p->S], as select_keys writes them), gathered
 * from the tiles. part/counter as embla_attn_full8; o bf16 [16][128]. */
int embla_attn_sparse8(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                       float* part, const uint32_t* idx, uint32_t* counter, void* o, const EmblaAttnParams* p,
                       hipStream_t stream);

/* ---------------------------------------------------------------- bf16 full-layer caches
 * The reference's full and sparse layers without KV8 (EMBLA_KV8=0, Engine.swift:162-163, 223-226,
 * 278): the caches hold bf16 K and V, `maxS` rows a kv head of 2, in the 16-bit tile layout of the
 * rings ([2][maxS/32] tiles of 32 x 128 bf16, no scales), the same bytes as the reference's
 * 2 · maxS · 128 · 2 a region. */

/* kv_append / kv_append_b without KV8 (attention.metal:113-140, prefill.metal:182-212; bound at
 * Engine.swift:782-793, Prefill.swift:315-322): T tokens of qkv rows (4096 bf16 each, position
 * pm_pos + t); K RMS-normed without gains and rounded to bf16, V copied; jobs[i].kc / .vc are
 * ELEMENT offsets of the layer's K and V regions in cache (Engine.swift:457). */
int embla_kv_append_bf16(const void* qkv, void* cache, const EmblaKVJob* jobs, int njobs, int pm_pos,
                         int maxS, int T, hipStream_t stream);

/* attn_full without KV8 (attention.metal:148-220; bound at Engine.swift:800-818): as
 * embla_attn_full8 over bf16 caches; scores (optional) the max over the 8 query heads of q·k. */
int embla_attn_full(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                    float* part, float* scores, uint32_t* counter, void* o, const EmblaAttnParams* p,
                    hipStream_t stream);

/* attn_sparse without KV8 (attention.metal:370-441): as embla_attn_sparse8 over bf16 caches;
 * idx NULL: every key 0 .. p->S-1, else the rows idx[kv head][0 .. p->S) gathered from the tiles. */
int embla_attn_sparse(const void* qraw, const void* g1, const void* g2, const void* kc, const void* vc,
                      float* part, const uint32_t* idx, uint32_t* counter, void* o, const EmblaAttnParams* p,
                      hipStream_t stream);

/* attn_full_b (prefill.metal:214-282; bound at Prefill.swift:325-338): T tokens of qkv bf16
 * [T][4096] at positions p->p0 .., q normed with both gains (g1, g2) and rounded to bf16, ReLU² with
 * sink over keys 0 .. p->p0 + t of the bf16 caches; o bf16 [T][2048]. part: the reference's part
 * buffer ([T][C][16][129] fp32, at least T · 16 · 128 · 2 bytes), used for the prepared queries;
 * p->CH and p->C are not used (one pass over every key of a row); counter is not used. */
int embla_attn_full_b(const void* qkv, const void* g1, const void* g2, const void* kc, const void* vc,
                      float* part, uint32_t* counter, void* o, const EmblaAttnB* p, int T, hipStream_t stream);

/* Reference-signature kv_append (attention.metal:113-140 / prefill.metal:182-212, bound at
 * Engine.swift:782-793, Prefill.swift:315-322): T tokens of qkv rows (4096 bf16 each, position
 * pm_pos + t), njobs jobs of 2 kv heads, int8 cache with fp32 scales at byte offsets
 * jobs[i].kc / .vc of cache; maxS rows a kv head. */
int embla_kv_append(const void* qkv, void* cache, const EmblaKVJob* jobs, int njobs, int pm_pos,
                    int maxS, int T, hipStream_t stream);

/* embla_decode_int8 with the q preparation folded in (softmax weights): q is the raw bf16 q of
 * the q/k/v projection [n_q][128], head-normed with ng (0-2) bf16 gains and rounded to bf16 inside
 * the decode kernel, as the reference's attention kernels do (common.metal:13-26 called from
 * attention.metal:235-363), instead of a separate embla_q_prep launch. Combinations: n_q / n_kv = 4,
 * fp16 scales, bf16 output; n_q / n_kv = 8, fp32 scales, bf16 output. */
int embla_decode_int8_qraw(const void* qraw, const void* g1, const void* g2, int ng, const void* kc, const void* vc,
                           void* o, int S, int max_s, int n_q, int n_kv, int scale_dtype, int out_dtype, int chunk,
                           void* ws, size_t ws_bytes, hipStream_t stream);

/* One decode step of a full layer with its own append, in one launch and a merge: the new token's
 * k and v (bf16 [n_kv][128] at element offsets k_off, v_off of qkv; q_off, k_off, v_off multiples
 * of 8 and qkv 16-byte aligned) quantised into the int8 cache
 * at position pos exactly as embla_kv_quant_append does (norm_k: K RMS-normed first; scales of
 * scale_dtype), and the softmax decode of q (raw bf16 [n_q][128] at q_off, head-normed with ng
 * gains as embla_decode_int8_qraw) over keys 0 .. pos, the new one included. The cached keys are
 * read by the split-K workgroups while one more workgroup a kv head appends the new row and adds
 * it as a partial: the append needs no launch of its own (the reference encodes kv_append and the
 * attention as two dispatches, Engine.swift:782-818). Combinations: n_q / n_kv = 4, fp16 scales,
 * bf16 output. ws: embla_workspace_bytes(max_s, n_q). */
int embla_decode_step_int8(const void* qkv, int q_off, int k_off, int v_off, const void* g1, const void* g2, int ng,
                           void* kc, void* vc, void* o, int pos, int max_s, int n_q, int n_kv, int scale_dtype,
                           int norm_k, int out_dtype, int chunk, void* ws, size_t ws_bytes, hipStream_t stream);

/* Query preparation (head_norm with ng gains + bf16 rounding; attention.metal:167-169,
 * prefill.metal:406-426): qraw bf16 rows of `stride` elements, n_q heads, T tokens ->
 * out [T][n_q][128] in out_dtype. */
int embla_q_prep(const void* qraw, const void* g1, const void* g2, int ng, int stride, int T,
                 int n_q, void* out, int out_dtype, hipStream_t stream);

/* Reference-signature q_prep_b (prefill.metal:406-426, bound at Prefill.swift:381-388): the full
 * layer's queries of qkv bf16 [T][4096] normed with both gains and rounded to bf16, head-major
 * qn [16][T][128], the input embla_relu2_prefill takes. */
int embla_q_prep_b(const void* qkv, const void* g1, const void* g2, void* qn, int T, hipStream_t stream);

/* ---------------------------------------------------------------- prefix-cache blocks
 * Save/restore of 128-position blocks between the layer caches and a stored block buffer, one
 * launch for every layer (Engine.fullSpans / windowSpans / copy, PrefixCache.swift:147-200). The
 * stored bytes are, per layer, K then V; per kv head its 128 rows (in the cache's tile order),
 * then each head's 128 scales: the reference's span order. regions: [n_layers][2] byte offsets of
 * each layer's K and V region in `cache` (16-byte aligned). save != 0 copies cache -> stored,
 * else stored -> cache. */

/* Bytes of a stored block of n_layers full layers (int8 rows, scales of scale_dtype). */
size_t embla_kv_block_bytes(int n_layers, int n_kv, int scale_dtype);

/* Positions p0 .. p0+127 (p0 % 128 == 0) of full layers' int8 caches [n_kv][max_s] (fullSpans). */
int embla_kv_block_copy(void* cache, const unsigned long long* regions, int n_layers, int p0, int max_s, int n_kv,
                        int scale_dtype, void* stored, int save, hipStream_t stream);

/* Bytes of a stored sliding-layer checkpoint of n_layers rings (16-bit elements). */
size_t embla_ring_block_bytes(int n_layers, int n_kv);

/* Ring slots (p0 % ring) .. +127 (p0 and ring multiples of 128) of sliding layers' 16-bit rings
 * [n_kv][ring][128] (windowSpans' K/V spans; the engram rows are outside this library). */
int embla_ring_block_copy(void* cache, const unsigned long long* regions, int n_layers, int p0, int ring, int n_kv,
                          void* stored, int save, hipStream_t stream);

/* ---------------------------------------------------------------- 4-bit projections
 * The q/k/v producer and o-projection consumer of the attention sub-layer (gemv.metal:1-92,
 * gemm.metal:1-134): W in MLX's affine 4-bit layout, words [O][K/8] (nibble q of word c is the
 * weight of column 8c + q), bf16 scales and biases [O][K/64] (w = s * nibble + b); x bf16. */

/* Epilogues (gemv.metal:77-88): y = bf16(acc); y = bf16(relu(bf16(acc))^2); y (fp32) += bf16(acc);
 * y (fp32) = bf16(acc); y (fp32) = acc. */
enum { EMBLA_EPI_BF16 = 0, EMBLA_EPI_RELU2 = 1, EMBLA_EPI_ADD = 2, EMBLA_EPI_F32_BF = 3, EMBLA_EPI_F32 = 4 };

/* A segment of stacked rows (gemv.metal's Seg, 29-35): byte offsets in W of its words, scales and
 * biases; its end row in the stack (exclusive, a multiple of 4); the element offsets of its input
 * in X (a multiple of 8) and of its first output in Y. */
typedef struct {
    unsigned long long w, s, b;
    unsigned int end, x, y, pad;
} EmblaSeg;

/* y = W x for one token over nseg (<= 8) stacked segments, K columns (2048 or 4096), one launch
 * (gemv.metal with MIX = 0: q, k and v of a layer, or the o-projection with EMBLA_EPI_ADD). */
int embla_gemv_q4(const void* W, const void* X, void* Y, const EmblaSeg* segs, int nseg, int K, int epi,
                  hipStream_t stream);

/* Y = X W^T for T tokens (gemm.metal with EXPERTS = GATHER = 0): X [T][ldx] bf16 (ldx a multiple of
 * 8), W's words, scales and biases at byte offsets wo[0], wo[1], wo[2] (16, 2, 2-byte aligned),
 * O rows, K inputs (a multiple of 64), Y [T][ldy] in the epilogue's type. */
int embla_gemm_q4(const void* W, const unsigned long long* wo, const void* X, void* Y, int T, int O, int K,
                  int ldx, int ldy, int epi, hipStream_t stream);

/* ---------------------------------------------------------------- sampling tail
 * The token of a step from V (<= 65536) fp32 logits, each softcapped in bf16 as
 * bf(bf(tanh(bf(bf(l) / 15))) * 15). Outputs as the reference's: greedy[pos] = the token; past the
 * prompt (pos + 1 >= prompt_len) token[pos + 1] = the token; last, greedy[-1] =
 * (pos + 1) << 16 | token, written at system scope after the others for a host that polls it.
 * `greedy` points one word into its buffer (the reference binds it at byte offset 4). logits
 * 16-byte aligned. Workspace: embla_sample_workspace_bytes(V) bytes, no zeroing needed. */
size_t embla_sample_workspace_bytes(int V);

/* The greedy token: the first index of the largest softcapped logit (misc.metal:86-128, the
 * `argmax` dispatch of Engine.swift:972-987). */
int embla_argmax(const float* logits, uint32_t* token, int V, uint32_t* greedy, int pos, int prompt_len, void* ws,
                 size_t ws_bytes, hipStream_t stream);

/* A draw from softmax(c / T) cut to its top-p nucleus by the Gumbel-max trick (misc.metal:196-298,
 * the `sample` dispatch of Engine.swift:972-987, SampleParams {1/T, top-p, seed}): inv_t = 1/T > 0,
 * 0 < top_p <= 1; the noise of token i is a hash of (seed, pos, i), so a draw is a function of its
 * inputs. Callers wanting greedy decoding (T <= 0 or top-p <= 0, Sampling.isGreedy) call
 * embla_argmax. */
int embla_sample(const float* logits, uint32_t* token, int V, uint32_t* greedy, int pos, int prompt_len, float inv_t,
                 float top_p, uint32_t seed, void* ws, size_t ws_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* EMBLA_ATTN_H */
