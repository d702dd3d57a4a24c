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
// takes P^T straight from the score registers (its k-slots match the score items) and V^T from
// LDS, where V is staged transposed. K and V tiles are double-buffered in LDS: the next 64 keys'
// global loads are in flight while the current ones are multiplied.
#include "common.hpp"
#include "embla_internal.hpp"

namespace embla {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int PBK = 64;            // keys a staged tile
constexpr int KROW = HD + 8;       // LDS row stride of K (fp16 elements): conflict-free 16 B reads
constexpr int VROW = PBK + 8;      // LDS row stride of V^T

__device__ __forceinline__ f16_t mfma32(h8v a, h8v b, f16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct PrefillSmem {
    _Float16 k[2][PBK * KROW];
    _Float16 vt[2][HD * VROW];
    float ks[2][PBK], vs[2][PBK];
};

template <int GQ, bool RELU2, bool SCALE32, bool QBF, bool OBF>
__global__ __launch_bounds__(64 * GQ) void prefill_int8_kernel(PrefillArgs a) {
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
    const int kstart = lo & ~(PBK - 1);
    const int ntiles = (hi - kstart) / PBK + 1;

    const size_t nrow = (size_t)a.n_kv * a.max_s * HD;
    const char* ksb = (const char*)(a.kc + nrow);
    const char* vsb = (const char*)(a.vc + nrow);

    // ---- staging: each thread moves 16-byte pieces of the two 32-key global tiles of a 64-key tile
    constexpr int PIECES = 2 * 256;               // 16-byte pieces a 64-key tile, K (same for V)
    constexpr int PER = PIECES / NT;              // pieces a thread
    u4_t kr[PER], vr[PER];
    uint32_t sr = 0;                              // a scale (threads 0 .. 2*PBK-1)
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = tid + NT * i, gt = q >> 8;
            // a 64-key tile's second half may lie past max_s (max_s % 64 == 32): read the first
            // half again; those keys are past every row's position and masked
            const size_t base = tile_base(kvh, a.max_s, min(k0 + 32 * gt, a.max_s - 32), 1) + (size_t)(q & 255) * 16;
            kr[i] = ld16(a.kc + base);
            vr[i] = ld16(a.vc + base);
        }
        if (tid < 2 * PBK) {
            const int key = k0 + (tid & (PBK - 1));
            const char* sb = tid < PBK ? ksb : vsb;
            const size_t si = (size_t)kvh * a.max_s + min(key, a.max_s - 1);
            sr = SCALE32 ? *(const uint32_t*)(sb + si * 4) : (uint32_t)*(const uint16_t*)(sb + si * 2);
        }
    };
    auto sstore = [&](int b) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = tid + NT * i, gt = q >> 8, j = (q & 255) >> 6, l = q & 63;
            // K piece (j, l): key 16 (j / 2) + l % 16, dims 32 (l / 16) + 16 (j % 2) .. + 15
            {
                const int key = 32 * gt + 16 * (j >> 1) + (l & 15), d0 = 32 * (l >> 4) + 16 * (j & 1);
                const h8_t lo8 = i8x8_to_h8(kr[i][0], kr[i][1]), hi8 = i8x8_to_h8(kr[i][2], kr[i][3]);
                *(h8_t*)(sm.k[b] + key * KROW + d0) = lo8;
                *(h8_t*)(sm.k[b] + key * KROW + d0 + 8) = hi8;
            }
            // V piece (j, l): dims 8 (l % 16) + 2j + {0, 1}, each with keys {16t + 4 (l / 16) + i}
            {
                const int n = l & 15, g = l >> 4;
#pragma unroll
                for (int uu = 0; uu < 2; uu++) {
                    const h8_t v8 = i8x8_to_h8(vr[i][2 * uu], vr[i][2 * uu + 1]);   // items e = 4t + i
                    const int dim = 8 * n + 2 * j + uu;
                    _Float16* row = sm.vt[b] + dim * VROW + 32 * gt + 4 * g;
                    *(h4_t*)(row) = (h4_t){v8[0], v8[1], v8[2], v8[3]};
                    *(h4_t*)(row + 16) = (h4_t){v8[4], v8[5], v8[6], v8[7]};
                }
            }
        }
        if (tid < 2 * PBK) {
            const float v = SCALE32 ? __uint_as_float(sr) : h2f((uint16_t)sr);
            if (tid < PBK) sm.ks[b][tid] = v;
            else sm.vs[b][tid - PBK] = v;
        }
    };

    // ---- Q^T as the B operand: lane (row r, half h), k-step s: dims 16s + 8h .. + 7 (fp16)
    h8v qb[8];
    {
        const uint16_t* qr = a.q + (size_t)min(tok, a.T - 1) * a.q_tok_stride + (size_t)hq * a.q_head_stride;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const u4_t raw = ld16(qr + 16 * s + 8 * h);
            qb[s] = QBF ? __builtin_bit_cast(h8v, bf8_to_h8(raw)) : __builtin_bit_cast(h8v, raw);
        }
    }
    const float c = RELU2 ? 0.08838834764831845f : 0.08838834764831845f * 1.4426950408889634f;

    float m = NEG_INF, lsum = 0.0f;
    f16_t O[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) O[i][e] = 0.0f;

    gload(kstart);
    sstore(0);
    __syncthreads();
    for (int it = 0; it < ntiles; it++) {
        const int b = it & 1, k0 = kstart + it * PBK;
        if (it + 1 < ntiles) gload(k0 + PBK);   // in flight during this tile's products
        const bool full_tile = k0 + PBK - 1 <= a.p0 + tok0 && (a.window == 0 || k0 >= a.p0 + last_tok - a.window + 1);
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            // S^T for keys k0 + 32kb + {8 (e / 4) + 4h + e % 4}: lane's 16 items
            f16_t st;
#pragma unroll
            for (int e = 0; e < 16; e++) st[e] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const h8v kv = *(const h8v*)(sm.k[b] + (32 * kb + r) * KROW + 16 * s + 8 * h);
                st = mfma32(kv, qb[s], st);
            }
            float x[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int kk = 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                const int key = k0 + kk;
                const bool ok = full_tile || (key <= pos && (a.window == 0 || key > pos - a.window));
                x[e] = ok ? st[e] * sm.ks[b][kk] * c : NEG_INF;
            }
            h8v pb[2];   // P^T B operands of the two 16-key k-steps (items 8s .. 8s + 7)
            if constexpr (RELU2) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int kk = 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                    const float t = fmaxf(x[e], 0.0f);
                    const float p = x[e] == NEG_INF ? 0.0f : t * t;
                    lsum += p;
                    pb[e >> 3][e & 7] = (_Float16)(p * sm.vs[b][kk]);
                }
            } else {
                float mt = NEG_INF;
#pragma unroll
                for (int e = 0; e < 16; e++) mt = fmaxf(mt, x[e]);
                mt = fmaxf(mt, shfl_xor(mt, 32));
                const float mn = fmaxf(m, mt);
                if (__any(mn > m)) {
                    const float corr = m == NEG_INF ? 0.0f : exp2f(m - mn);
                    lsum *= corr;
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) O[i][e] *= corr;
                    m = mn;
                }
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int kk = 32 * kb + 8 * (e >> 2) + 4 * h + (e & 3);
                    const float p = x[e] == NEG_INF ? 0.0f : exp2f(x[e] - m);
                    lsum += p;
                    pb[e >> 3][e & 7] = (_Float16)(p * sm.vs[b][kk] * 64.0f);
                }
            }
            // O^T (dims 32i + {8 (e / 4) + 4h + e % 4}) += V^T P^T over the two 16-key k-steps
#pragma unroll
            for (int s = 0; s < 2; s++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const _Float16* vrow = sm.vt[b] + (32 * i + r) * VROW + 32 * kb + 16 * s + 4 * h;
                    const h4_t v0 = *(const h4_t*)vrow, v1 = *(const h4_t*)(vrow + 8);
                    const h8v av = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    O[i] = mfma32(av, pb[s], O[i]);
                }
            }
        }
        if (it + 1 < ntiles) {
            __syncthreads();          // every wave is done with buffer b ^ 1 (its previous tile)
            sstore(b ^ 1);
            __syncthreads();
        }
    }

    // ---- normalise and store: lane (row r, half h) holds dims 32i + 8b + 4h .. + 3
    lsum += shfl_xor(lsum, 32);
    if (!row_ok) return;
    const float inv = RELU2 ? 1.0f / (0.0f + (11.313708498984761f + lsum)) : 1.0f / (64.0f * lsum);
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

int launch_prefill_int8(const PrefillArgs& a, hipStream_t st) {
    const int gq = a.n_q / a.n_kv;
    const dim3 grid((a.T + 31) / 32, a.n_kv);
#define EMBLA_PF(GQ, R, S32, QBF, OBF) \
    hipLaunchKernelGGL((prefill_int8_kernel<GQ, R, S32, QBF, OBF>), grid, dim3(64 * GQ), 0, st, a)
    if (gq == 4 && !a.relu2 && !a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(4, false, false, true, true);
    else if (gq == 4 && !a.relu2 && !a.scale32 && !a.q_bf16 && !a.out_bf16) EMBLA_PF(4, false, false, false, false);
    else if (gq == 8 && a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, true, true, true, true);
    else if (gq == 8 && !a.relu2 && a.scale32 && a.q_bf16 && a.out_bf16) EMBLA_PF(8, false, true, true, true);
    else return EMBLA_ERR_UNSUPPORTED;
#undef EMBLA_PF
    return hipGetLastError() == hipSuccess ? EMBLA_OK : EMBLA_ERR_HIP;
}

}  // namespace embla
