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
};
int launch_full_decode(const FullDecodeArgs& a, hipStream_t st);

struct KVQuantArgs {
    const uint16_t* k;   // [T] rows of k, row stride `stride` elements, kv head h at h * 128
    const uint16_t* v;
    int stride;
    int T, p0, n_kv, max_s;
    int8_t* kc;
    int8_t* vc;
    bool in_bf16, scale32, norm_k;
};
int launch_kv_quant(const KVQuantArgs& a, hipStream_t st);

struct QPrepArgs {
    const uint16_t* qraw;   // bf16 [T] rows, row stride `stride`, head h at h * 128
    const uint16_t* g1;     // optional gains (bf16 [128])
    const uint16_t* g2;
    int ng, stride, T, n_q;
    uint16_t* out;          // [T][n_q][128] fp16 or bf16
    bool out_bf16;
};
int launch_q_prep(const QPrepArgs& a, hipStream_t st);

}  // namespace embla
