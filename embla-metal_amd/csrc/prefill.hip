// Batched prefill attention over an int8 KV cache: T new tokens at positions p0 .. p0+T-1 attend
// keys 0 .. their own position (causal; optionally only the last `window` positions).
//
// Follows relu2_prefill_nax and attn_full_b (Sources/EmblaMetal/Kernels/attn_nax.metal:61-364,
// prefill.metal:214-282): ReLU² with sink (p = relu(s·scale)², out = Σp·v / (√128 + Σp)) for the
// reference's full layer, softmax (scale 1/√128) for the BASELINE configs; the int8 rows are
// staged once a workgroup as exact 16-bit integers (attn_nax.metal:26-56), each key's scale
// multiplies its score and each value row's scale its weight (attn_nax.metal:231-246, 294).
//
// MI355X design: a workgroup is (32 tokens, kv head) with one wave a query head (GQ waves), so the
// staged K/V tiles serve GQ * 32 query rows. S^T = K·Q^T runs on v_mfma_f32_32x32x16_f16 with the
// query rows as MFMA columns: lane (row r = l % 32, half h = l / 32) then holds one query row's 16
// scores a 32-key block, so the online softmax state (m, l) and the output O^T rows live in that
// lane: the row maximum needs one cross-lane step (xor 32) and rescaling O needs none. O^T += V^T·P^T
// takes P^T straight from the score registers (its k-slots are chosen to match the score items)
// and V^T from LDS, where V is staged as an fp16 copy of its global lane-order tile, which already
// holds 8 keys of one dim contiguous. K and V tiles are double-buffered in LDS: the next 64 keys'
// global loads are in flight while the current ones are multiplied.
#include "common.hpp"
#include "embla_internal.hpp"

#include <type_traits>

namespace embla {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int PBK = 64;            // keys a staged tile
constexpr int KROW = HD + 8;       // LDS row stride of K (fp16 elements): conflict-free 16 B reads
// V is staged as an fp16 copy of its global tile order: a 32-key tile is 8 rows u (dim % 8) of 64
// lane slots (n + 16g) of 16 bytes, each slot the 8 keys {16t + 4g + i} of dim 8n + u. Rows are
// padded by 16 bytes so the A-operand reads (8 lanes, rows u = 0..7) hit distinct banks.
constexpr int VUROW = 64 * 8 + 8;  // fp16 elements a padded row u
constexpr int VTILE = 8 * VUROW;   // fp16 elements a staged 32-key V tile

__device__ __forceinline__ f16_t mfma32(h8v a, h8v b, f16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
/// 32x32x16 on 16-byte operands holding fp16 (BF = false) or bf16 (BF = true) values.
template <bool BF>
__device__ __forceinline__ f16_t mfma32x(u4_t a, u4_t b, f16_t c) {
    if constexpr (BF) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
}

struct __attribute__((aligned(16))) PrefillSmem {
    _Float16 k[2][PBK * KROW];
    _Float16 vt[2][2 * VTILE];
    float ks[2][PBK], vs[2][PBK];
};

constexpr int PPS = HD + 4;        // floats a split partial row: O[128], m, l, pad
int launch_prefill_tail(const PrefillArgs& a, hipStream_t st);

// RING: K/V from a 16-bit ring (no scales; S = K·Q^T on the MFMA in the ring's type, BF = bf16;
// V staged as fp16); else from an int8 region (fp16 MFMA). PRE: q normed with gains, rotated, bf16-rounded in-kernel.
template <int GQ, bool RELU2, bool SCALE32, bool QBF, bool OBF, bool RING = false, bool BF = false, bool PRE = false>
__global__ __launch_bounds__(64 * GQ, 2) void prefill_int8_kernel(PrefillArgs a) {
    constexpr int NT = 64 * GQ;
    __shared__ PrefillSmem sm;
    const int tb = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 31, h = lane >> 5;
    const int hq = kvh * GQ + w;
    const int tok0 = tb * 32, tok = tok0 + r;                 // this lane's query row
    const bool row_ok = tok < a.T;
    const int pos = a.p0 + min(tok, a.T - 1);                  // its position
    const int last_tok = min(tok0 + 31, a.T - 1);
    const int hi = a.p0 + last_tok;                            // last key the block needs
    int lo = 0;
    if (a.window > 0) lo = max(0, a.p0 + tok0 - a.window + 1);
    const int kfirst = lo & ~(PBK - 1);
    const int ntot = (hi - kfirst) / PBK + 1;
    // split z of nsplit takes an equal share of the block's key tiles (the prefix splits evenly)
    const int z = blockIdx.z, t_lo = ntot * z / a.nsplit, t_hi = ntot * (z + 1) / a.nsplit;
    const int kstart = kfirst + t_lo * PBK;
    const int ntiles = t_hi - t_lo;

    const float c = RELU2 ? 0.08838834764831845f : 0.08838834764831845f * 1.4426950408889634f;
    const size_t nrow = (size_t)a.n_kv * a.max_s * HD;
    const char* ksb = (const char*)(a.kc + nrow);
    const char* vsb = (const char*)(a.vc + nrow);

    // ---- staging: each thread moves 16-byte pieces of the two 32-key global tiles of a 64-key tile
    constexpr int ES = RING ? 2 : 1;
    constexpr int PIECES = 2 * 256 * ES;          // 16-byte pieces a 64-key tile, K (same for V)
    constexpr int PER = PIECES / NT;              // pieces a thread
    u4_t kr[PER], vr[PER];
    uint32_t sr = 0;                              // a scale (threads 0 .. 2*PBK-1)
    auto tile_addr = [&](int key) -> size_t {     // byte offset of the 32-key tile holding key
        if constexpr (RING) return tile_base(kvh, a.R, key % a.R, 2);
        // a 64-key tile's second half may lie past max_s (max_s % 64 == 32): read the first
        // half again; those keys are past every row's position and masked
        else return tile_base(kvh, a.max_s, min(key, a.max_s - 32), 1);
    };
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = tid + NT * i, gt = q / (256 * ES);
            const size_t off = tile_addr(k0 + 32 * gt) + (size_t)(q % (256 * ES)) * 16;
            if constexpr (RING) {
                kr[i] = ld16((const char*)a.kring + off);
                vr[i] = ld16((const char*)a.vring + off);
            } else {
                kr[i] = ld16(a.kc + off);
                vr[i] = ld16(a.vc + off);
            }
        }
        if constexpr (!RING) {
            if (tid < 2 * PBK) {
                const int key = k0 + (tid & (PBK - 1));
                const char* sb = tid < PBK ? ksb : vsb;
                const size_t si = (size_t)kvh * a.max_s + min(key, a.max_s - 1);
                sr = SCALE32 ? *(const uint32_t*)(sb + si * 4) : (uint32_t)*(const uint16_t*)(sb + si * 2);
            }
        }
    };
    auto sstore = [&](int b) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = tid + NT * i, gt = q / (256 * ES), j = (q % (256 * ES)) >> 6, l = q & 63;
            if constexpr (RING) {
                // K piece (j, l): key 16 (j / 4) + l % 16, dims 32 (l / 16) + 8 (j % 4) .. + 7
                const int key = 32 * gt + 16 * (j >> 2) + (l & 15), d0 = 32 * (l >> 4) + 8 * (j & 3);
                *(u4_t*)(sm.k[b] + key * KROW + d0) = kr[i];
                // V piece (j = u, l): row u of slot l, 8 keys: a copy (bf16 widened to fp16, so P
                // keeps fp16's 11-bit significand in the P·V product)
                u4_t vv = vr[i];
                if constexpr (BF) vv = __builtin_bit_cast(u4_t, bf8_to_h8(vv));
                *(u4_t*)(sm.vt[b] + gt * VTILE + j * VUROW + l * 8) = vv;
            } else {
                // K piece (j, l): key 16 (j / 2) + l % 16, dims 32 (l / 16) + 16 (j % 2) .. + 15
                const int key = 32 * gt + 16 * (j >> 1) + (l & 15), d0 = 32 * (l >> 4) + 16 * (j & 1);
                *(h8_t*)(sm.k[b] + key * KROW + d0) = i8x8_to_h8(kr[i][0], kr[i][1]);
                *(h8_t*)(sm.k[b] + key * KROW + d0 + 8) = i8x8_to_h8(kr[i][2], kr[i][3]);
                // V piece (j, l): rows u = 2j, 2j + 1 of slot l, 8 keys each: straight copies as fp16
                _Float16* base = sm.vt[b] + gt * VTILE + l * 8;
                *(h8_t*)(base + (2 * j) * VUROW) = i8x8_to_h8(vr[i][0], vr[i][1]);
                *(h8_t*)(base + (2 * j + 1) * VUROW) = i8x8_to_h8(vr[i][2], vr[i][3]);
            }
        }
        if (tid < 2 * PBK) {
            const float v = RING ? 1.0f : (SCALE32 ? __uint_as_float(sr) : h2f((uint16_t)sr));
            // scores: scale_k * (1/sqrt(128)) [* log2 e]; weights: scale_v [* 64 into fp16's range]
            if (tid < PBK) sm.ks[b][tid] = v * c;
            else sm.vs[b][tid - PBK] = RELU2 ? v : v * 64.0f;
        }
    };

    // ---- Q^T as the B operand: lane (row r, half h), k-step s: dims 16s + 8h .. + 7 (16-bit,
    // in the MFMA's type)
    u4_t qb[8];
    {
        const uint16_t* qr = a.q + (size_t)min(tok, a.T - 1) * a.q_tok_stride + (size_t)hq * a.q_head_stride;
#pragma unroll
        for (int s = 0; s < 8; s++) qb[s] = ld16(qr + 16 * s + 8 * h);
        if constexpr (PRE) {
            // head_norm with the q gains, RoPE at the row's position, bf16 (attn_sliding8_b,
            // prefill.metal:450-456): the row's dims are split over lanes h = 0, 1 (xor 32); the
            // rotation pairs d and d + 32 (d < 32) sit in the same lane (k-steps s and s + 2)
            float x[64];
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    x[8 * s + 2 * i] = bf2f(qb[s][i] & 0xFFFF);
                    x[8 * s + 2 * i + 1] = bf2f(qb[s][i] >> 16);
                }
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 64; e++) ss += x[e] * x[e];
            ss += shfl_xor(ss, 32);
            const float rn = 1.0f / sqrtf(ss / 128.0f + 1.1920929e-07f);
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) x[8 * s + e] = x[8 * s + e] * (rn * (1.0f + bf2f(a.qg[16 * s + 8 * h + e])));
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int d = 16 * s + 8 * h + e;   // < 32, partner d + 32 at k-step s + 2
                    float sn, cs;
                    sincosf(-(float)pos * (float)exp2(-(double)d / 32.0 * 13.287712379549449), &sn, &cs);
                    const float x1 = x[8 * s + e], x2 = x[8 * (s + 2) + e];
                    x[8 * s + e] = x1 * cs - x2 * sn;
                    x[8 * (s + 2) + e] = x1 * sn + x2 * cs;
                }
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    qb[s][i] = (uint32_t)f2bf(x[8 * s + 2 * i]) | ((uint32_t)f2bf(x[8 * s + 2 * i + 1]) << 16);
        } else if constexpr (!RING && QBF) {
#pragma unroll
            for (int s = 0; s < 8; s++) qb[s] = __builtin_bit_cast(u4_t, bf8_to_h8(qb[s]));
        }
    }

    float m = NEG_INF, lsum = 0.0f;
    f16_t O[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) O[i][e] = 0.0f;

    if (ntiles > 0) {
        gload(kstart);
        sstore(0);
    }
    __syncthreads();
    for (int it = 0; it < ntiles; it++) {
        const int b = it & 1, k0 = kstart + it * PBK;
        if (it + 1 < ntiles) gload(k0 + PBK);   // in flight during this tile's products
        const bool full_tile = k0 + PBK - 1 <= a.p0 + tok0 && (a.window == 0 || k0 >= a.p0 + last_tok - a.window + 1);
        // keys above kmax or at/below kmin are masked; a tile every row sees whole masks nothing
        const int kmax = full_tile ? 0x7FFFFFFF : pos;
        const int kmin = (full_tile || a.window == 0) ? -0x7FFFFFFF : pos - a.window;
        // S^T for keys k0 + 32kb + {8b + 4h + i}: the lane's 16 items e = 4b + i. Both blocks'
        // products are issued before either block's softmax, so one chain runs under the other's
        // VALU work.
        auto s_block = [&](int kb) -> f16_t {
            const u4_t* krow = (const u4_t*)(sm.k[b] + (32 * kb + r) * KROW) + h;
            f16_t st = mfma32x<BF>(krow[0], qb[0], (f16_t){});
#pragma unroll
            for (int s = 1; s < 8; s++) st = mfma32x<BF>(krow[2 * s], qb[s], st);
            return st;
        };
        auto run_block = [&](int kb, const f16_t& st) {
            const f4_t* ks4 = (const f4_t*)(sm.ks[b] + 32 * kb + 4 * h);   // [2b]: keys 8b + 4h ..
            const f4_t* vs4 = (const f4_t*)(sm.vs[b] + 32 * kb + 4 * h);
            float pw[16];   // P^T values (with the V scales), item e
            if constexpr (RELU2) {
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    const f4_t kq = ks4[2 * bb], vq = vs4[2 * bb];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int e = 4 * bb + i;
                        const int key = k0 + 32 * kb + 8 * bb + 4 * h + i;
                        const bool ok = key <= kmax && key > kmin;
                        const float t = fmaxf(st[e] * kq[i], 0.0f);
                        const float p = ok ? t * t : 0.0f;
                        lsum += p;
                        pw[4 * bb + i] = p * vq[i];
                    }
                }
            } else {
                float x[16];
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    const f4_t kq = ks4[2 * bb];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        x[4 * bb + i] = st[4 * bb + i] * kq[i];
                    }
                }
                if (!full_tile) {   // uniform: only the diagonal (and window-edge) tiles
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int key = k0 + 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                        x[e] = key <= kmax && key > kmin ? x[e] : NEG_INF;
                    }
                }
                float mt = fmaxf(x[0], x[1]);
#pragma unroll
                for (int e = 2; e < 16; e += 2) mt = fmaxf(mt, fmaxf(x[e], x[e + 1]));
                mt = fmaxf(mt, shfl_xor(mt, 32));
                // the running maximum moves only when a row's grows by more than 2^8: weights stay
                // <= 256 (fp16-safe after the 64 * scale_v prescale), O and l share the stale m
                if (__any(mt > m + 8.0f)) {
                    const float mn = fmaxf(m, mt);
                    const float corr = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                    lsum *= corr;
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) O[i][e] *= corr;
                    m = mn;
                }
                // a masked key gives exp2(-inf) = 0; a row whose every key so far is masked keeps
                // m = -inf: subtracting +inf instead keeps its weights 0 (not exp2(-inf + inf))
                const float msub = m == NEG_INF ? -NEG_INF : m;
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    const f4_t vq = vs4[2 * bb];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float p = __builtin_amdgcn_exp2f(x[4 * bb + i] - msub);
                        lsum += p;
                        pw[4 * bb + i] = p * vq[i];
                    }
                }
            }
            // P^T B operands (fp16) of the two 16-key k-steps: step s = items b = s (slots 0..3)
            // and b = 2 + s (slots 4..7)
            u4_t pb[2];
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int q2 = 0; q2 < 4; q2++) {
                    const int e0 = (q2 < 2 ? 4 * s : 4 * (2 + s)) + 2 * (q2 & 1);
                    pb[s][q2] = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)pw[e0], (_Float16)pw[e0 + 1]});
                }
            // O^T (dims 32i + {8b + 4h + i}) += V^T P^T over two 16-key k-steps: in step s lane
            // (dim 32i + r, h) takes slot (n = dim / 8, g = 2s + h) of row u = dim % 8, whose 8 keys
            // {8s + 4h + i, 16 + 8s + 4h + i} are the P^T items b = s and b = 2 + s
            const u4_t* vt = (const u4_t*)(sm.vt[b] + kb * VTILE);
#pragma unroll
            for (int s = 0; s < 2; s++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int dim = 32 * i + r;
                    O[i] = mfma32x<false>(vt[(dim & 7) * (VUROW / 8) + (dim >> 3) + 16 * (2 * s + h)], pb[s], O[i]);
                }
            }
        };
        const f16_t s0 = s_block(0), s1 = s_block(1);
        run_block(0, s0);
        run_block(1, s1);
        if (it + 1 < ntiles) {
            // buffer b ^ 1 was last read in the previous iteration, which every wave finished
            // before that iteration's barrier: one barrier a tile
            sstore(b ^ 1);
            __syncthreads();
        }
    }

    // ---- normalise and store: lane (row r, half h) holds dims 32i + 8b + 4h .. + 3
    lsum += shfl_xor(lsum, 32);
    if (!row_ok) return;
    if (a.nsplit > 1) {   // this split's partial row: unnormalised O, m, l
        float* pp = a.part + (((size_t)z * a.T + tok) * a.n_q + hq) * PPS;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int bb = 0; bb < 4; bb++)
                *(f4_t*)(pp + 32 * i + 8 * bb + 4 * h) = (f4_t){O[i][4 * bb], O[i][4 * bb + 1], O[i][4 * bb + 2], O[i][4 * bb + 3]};
        if (h == 0) { pp[HD] = m; pp[HD + 1] = lsum; }
        return;
    }
    const float inv = RELU2 ? 1.0f / (11.313708498984761f + lsum) : 1.0f / (64.0f * lsum);
    uint16_t* orow = a.o + (size_t)tok * a.o_tok_stride + (size_t)hq * a.o_head_stride;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const int d = 32 * i + 8 * bb + 4 * h;
            u2_t pk;
            pk[0] = (uint32_t)f2a<OBF>(O[i][4 * bb] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 1] * inv) << 16);
            pk[1] = (uint32_t)f2a<OBF>(O[i][4 * bb + 2] * inv) | ((uint32_t)f2a<OBF>(O[i][4 * bb + 3] * inv) << 16);
            *(u2_t*)(orow + d) = pk;
        }
}

/// Merges the nsplit partial rows of (token, head) = (blockIdx.x * 4 + wave, blockIdx.y): a wave
/// a row, two dims a lane.
template <bool RELU2, bool OBF>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
    const int lane = threadIdx.x & 63, tok = blockIdx.x * 4 + (threadIdx.x >> 6), hq = blockIdx.y;
    if (tok >= a.T) return;
    float M = RELU2 ? 0.0f : NEG_INF;
    if constexpr (!RELU2)
        for (int z = 0; z < a.nsplit; z++) M = fmaxf(M, a.part[(((size_t)z * a.T + tok) * a.n_q + hq) * PPS + HD]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
    for (int z = 0; z < a.nsplit; z++) {
        const float* pp = a.part + (((size_t)z * a.T + tok) * a.n_q + hq) * PPS;
        const float mz = pp[HD];
        const float f = RELU2 ? 1.0f : (mz == NEG_INF ? 0.0f : exp2f(mz - M));
        L += pp[HD + 1] * f;
        o0 += pp[2 * lane] * f;
        o1 += pp[2 * lane + 1] * f;
    }
    const float inv = RELU2 ? 1.0f / (11.313708498984761f + L) : 1.0f / (64.0f * L);
    uint16_t* orow = a.o + (size_t)tok * a.o_tok_stride + (size_t)hq * a.o_head_stride;
    *(uint32_t*)(orow + 2 * lane) = (uint32_t)f2a<OBF>(o0 * inv) | ((uint32_t)f2a<OBF>(o1 * inv) << 16);
}

int launch_prefill_int8(const PrefillArgs& a, hipStream_t st) {
    const int gq = a.n_q / a.n_kv;
    const dim3 grid((a.T + 31) / 32, a.n_kv, a.nsplit);
#define EMBLA_PF(GQ, R, S32, QBF, OBF) \
    hipLaunchKernelGGL((prefill_int8_kernel<GQ, R, S32, QBF, OBF>), grid, dim3(64 * GQ), 0, st, a)
    if (gq == 4 && !a.relu2 && !a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(4, false, false, true, true);
    else if (gq == 4 && !a.relu2 && !a.scale32 && !a.q_bf16 && !a.out_bf16) EMBLA_PF(4, false, false, false, false);
    else if (gq == 8 && a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, true, true, true, true);
    else if (gq == 8 && !a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, false, true, true, true);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_PF
    return launch_prefill_tail(a, st);
}

int launch_prefill_ring(const PrefillArgs& a, hipStream_t st) {
    const int gq = a.n_q / a.n_kv;
    const dim3 grid((a.T + 31) / 32, a.n_kv, a.nsplit);
#define EMBLA_PR(BF, PRE) \
    hipLaunchKernelGGL((prefill_int8_kernel<4, false, false, BF, BF, true, BF, PRE>), grid, dim3(256), 0, st, a)
    if (gq != 4 || a.relu2) return EMBLA_ERR_UNSUPPORTED;
    if (a.q_bf16 && a.out_bf16 && a.qg) EMBLA_PR(true, true);
    else if (a.q_bf16 && a.out_bf16) EMBLA_PR(true, false);
    else if (!a.q_bf16 && !a.out_bf16 && !a.qg) EMBLA_PR(false, false);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_PR
    return launch_prefill_tail(a, st);
}

int launch_prefill_tail(const PrefillArgs& a, hipStream_t st) {
    if (a.nsplit > 1) {
        const dim3 mg((a.T + 3) / 4, a.n_q);
        if (a.relu2) hipLaunchKernelGGL((prefill_merge_kernel<true, true>), mg, dim3(256), 0, st, a);
        else if (a.out_bf16) hipLaunchKernelGGL((prefill_merge_kernel<false, true>), mg, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((prefill_merge_kernel<false, false>), mg, dim3(256), 0, st, a);
    }
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
