#!/usr/bin/env python3
"""bench.py — MI355X attention hot path of embla-metal, one GPU.

Headline (BASELINE.json metric "attention µs/layer + HBM GB/s at 32k decode"): config C3, one
decode step of full-layer attention over int8 KV caches at context 32768 (16 query / 4 kv heads,
head dim 128, fp16 scales), through a stack of 16 layers with 16 distinct caches (545 MB, beyond
the 256 MB MALL, so every layer streams from HBM). A step is the 16 layers' attention calls
(split-K decode + merge), captured once as a HIP graph and replayed; inputs are resident in HBM.
`value` is algorithmic HBM bytes a step / time (1040·L + 8192 bytes a layer).

Also reported: the C3 context sweep (4096, 16384, 32768; µs a layer), C2 sliding-window decode
(512 steps over an fp16 ring of 8192, window 1024), C4 sparse-layer decode at 32k (indexer, exact
top-k, attention over 1152 gathered rows), and the CPU baseline: the C oracle
(oracle/oracle.c, a scalar fp32 restatement) timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "embla-metal_amd"))

METRIC = "attention µs/layer + HBM GB/s at 32k decode; prefill attn TFLOP/s @2048"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0   # dense bf16/fp16 MFMA, MI355X


def main_kernel_bytes(L: int) -> int:
    """Algorithmic bytes of C3's split-K kernel: K and V int8 rows + fp16 scales, q fp16."""
    return L * 4 * 2 * (128 + 2) + 16 * 128 * 2


def layer_bytes(L: int) -> int:
    """Algorithmic bytes of one C3 layer: K and V int8 rows + fp16 scales, q and o fp16."""
    return L * 4 * 2 * (128 + 2) + 16 * 128 * 2 * 2


def make_caches(torch, n_layers: int, max_s: int, n_kv: int = 4, seed_layer0: int | None = 2):
    """n_layers (K region, V region) pairs of int8 tiles + fp16 scales U[0.005, 0.02]. Layer 0
    comes from the seeded SplitMix64 draw of config C3 (kept for the parity check); the rest are
    drawn on the device."""
    from embla_attn import layout, synth
    nrow = n_kv * max_s * 128
    regions = []
    case = None
    for i in range(n_layers):
        if i == 0 and seed_layer0 is not None:
            case = synth.decode_int8_case(seed=seed_layer0, S=max_s, n_kv=n_kv)
            kc = torch.from_numpy(layout.pack_region(case["K"], case["ks"], max_s, "k")).cuda()
            vc = torch.from_numpy(layout.pack_region(case["V"], case["vs"], max_s, "v")).cuda()
        else:
            g = torch.Generator(device="cuda")
            g.manual_seed(1000 + i)
            kc = torch.empty(nrow + n_kv * max_s * 2, dtype=torch.uint8, device="cuda")
            vc = torch.empty_like(kc)
            for t in (kc, vc):
                t[:nrow].random_(0, 256, generator=g)
                t[nrow:].view(torch.float16).uniform_(0.005, 0.02, generator=g)
        regions.append((kc, vc))
    return regions, case


LAST_MEDIAN_MS = [0.0]   # the median replay of the last time_graph call


def time_graph(torch, fn, steps: int, warmup: int):
    """Captures fn() once as a graph, replays `warmup` untimed then `steps` timed replays between
    synchronisations; returns (seconds, ms a replay by events)."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn()   # eager once (first-touch), outside the graph
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(steps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    LAST_MEDIAN_MS[0] = per[steps // 2]
    return wall, ev[0].elapsed_time(ev[steps]) / steps


def time_calls(torch, fn, n: int, reps: int, warmup: int) -> float:
    """ms a call of fn, n calls captured in one graph (a graph of a short call would time its own
    launch)."""
    def run():
        for _ in range(n):
            fn()
    return time_graph(torch, run, reps, warmup)[1] / n


def bench_c3(torch, steps, warmup, n_layers=16, contexts=(4096, 16384, 32768)):
    from embla_attn import ops
    max_s = max(contexts)
    regions, case = make_caches(torch, n_layers, max_s)
    q = torch.from_numpy(case["q"]).cuda().view(torch.float16)
    ws = ops.Workspace(max_s, 16)
    outs = [torch.empty((16, 128), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    res = {}
    for L in contexts:
        def step(L=L):
            for i in range(n_layers):
                ops.decode_int8(q, regions[i][0], regions[i][1], L, max_s, 4, ws=ws, out=outs[i])
        wall, ms = time_graph(torch, step, steps if L == max_s else max(10, steps // 2), warmup)
        res[L] = dict(ms_per_step=ms, us_per_layer=ms * 1000 / n_layers, wall_s=wall,
                      us_per_layer_median=LAST_MEDIAN_MS[0] * 1000 / n_layers,
                      gbs=layer_bytes(L) * n_layers / (ms * 1e-3) / 1e9)
    # the split-K kernel alone (no merge), the dominant kernel of the roofline: 16 launches a graph
    L = max_s
    def main_only():
        for i in range(n_layers):
            ops.decode_int8_partials(q, regions[i][0], regions[i][1], L, max_s, 4, ws)
    _, ms_main = time_graph(torch, main_only, steps, warmup)
    main_us = ms_main * 1000 / n_layers
    # parity of layer 0 at the headline context against the oracle (checked, not timed)
    return res, case, outs[0], regions, main_us


def bench_c3_single(torch, regions, case, L=32768, reps=30):
    """One C3 layer call alone (split-K pass + merge, captured as a one-layer graph), each replay
    after a 512 MB fill that evicts the L2s and the MALL, so its 34 MB come from HBM with nothing
    before or after it in the graph: the isolated cold-cache layer time (median of `reps`)."""
    from embla_attn import ops
    q = torch.from_numpy(case["q"]).cuda().view(torch.float16)
    ws = ops.Workspace(L, 16)
    out = torch.empty((16, 128), dtype=torch.float16, device="cuda")
    big = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    kc, vc = regions[0]
    ops.decode_int8(q, kc, vc, L, L, 4, ws=ws, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.decode_int8(q, kc, vc, L, L, 4, ws=ws, out=out)
    times = []
    for _ in range(reps):
        big.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1000)
    times.sort()
    us = times[len(times) // 2]
    return dict(us_cold_median=us, us_cold_min=times[0], gbs=layer_bytes(L) / (us * 1e-6) / 1e9,
                tokens_per_s=1e6 / us, reps=reps)


def bench_read_floor(torch, n_layers=16, max_s=32768, n_kv=4, reps=20):
    """The practical floor of one decode layer's split-K pass: a plain streaming read of the same
    bytes (K and V rows + fp16 scales of 32768 keys, 34,078,720 B) in one launch, 16 distinct
    buffers in one graph (545 MB, beyond the 256 MB MALL); the best of three grid sizes."""
    from embla_attn import ops
    nbytes = 2 * n_kv * max_s * (128 + 2)
    bufs = []
    for i in range(n_layers):
        b = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        b.random_(0, 256, generator=torch.Generator(device="cuda").manual_seed(500 + i))
        bufs.append(b)
    sink = torch.empty(4096, dtype=torch.int32, device="cuda")
    best = None
    for grid in (512, 1024, 2048):
        def run(grid=grid):
            for b in bufs:
                ops.stream_read(b, sink, grid)
        _, ms = time_graph(torch, run, reps, 3)
        us = ms * 1000 / n_layers
        if best is None or us < best[1]:
            best = (grid, us)
    del bufs
    return dict(bytes=nbytes, grid=best[0], us_per_launch=best[1], gbs=nbytes / (best[1] * 1e-6) / 1e9)


def bench_mfma_ceiling(torch, reps=5):
    """The dense fp16 MFMA rate the chip sustains: the bench-only probe's back-to-back
    v_mfma_f32_32x32x16_f16 (4 independent chains a wave, no memory traffic), 512 workgroups of 4
    waves for about as long as C5's full prefill (~0.7 ms a launch); the best of `reps` launches."""
    from embla_attn import ops
    grid, iters = 512, 4000
    sink = torch.empty(grid * 4, dtype=torch.float32, device="cuda")
    ops.mfma_rate(grid, 100, sink)
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ops.mfma_rate(grid, iters, sink)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        best = ms if best is None else min(best, ms)
    flops = grid * 4 * 4 * iters * 32768.0
    tf = flops / (best * 1e-3) / 1e12
    return dict(what="back-to-back v_mfma_f32_32x32x16_f16, no memory traffic (the bench-only probe)",
                ms=best, tflops=tf, frac_of_peak=tf / (MFMA_PEAK_TFLOPS))


def bench_c2(torch, n_steps=512, reps=5):
    """Config C2: 512 consecutive decode steps over an fp16 ring of 8192, window 1024, each
    appending one K/V pair; one graph of the 512 steps."""
    from embla_attn import ops
    R, W, n_kv, n_q = 8192, 1024, 4, 16
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    kring = torch.randn(n_kv * R * 128, generator=g, device="cuda").half()
    vring = torch.randn(n_kv * R * 128, generator=g, device="cuda").half()
    qs = torch.randn(n_steps, n_q, 128, generator=g, device="cuda").half()
    ks = torch.randn(n_steps, n_kv, 128, generator=g, device="cuda").half()
    vs = torch.randn(n_steps, n_kv, 128, generator=g, device="cuda").half()
    out = torch.empty(n_q, 128, dtype=torch.float16, device="cuda")
    ws = ops.Workspace(R, n_q)
    p0 = R   # the history fills the ring; step s is position R + s

    def run():
        for s in range(n_steps):
            ops.sliding_decode(qs[s], ks[s], vs[s], kring, vring, p0 + s, W, R, n_kv, ws=ws, out=out)
    wall, ms = time_graph(torch, run, reps, 1)
    us = ms * 1000 / n_steps
    return dict(us_per_step=us, tokens_per_s=1e6 / us, steps=n_steps,
                gbs_cache_resident=2 * W * n_kv * 128 * 2 / (us * 1e-6) / 1e9)


def bench_c4(torch, reps=20, n_layers=16):
    """Config C4: a sparse-layer decode step at context 32768 (index scores, exact top-1024 +
    latest 128, attention over the 1152 gathered fp16 rows); 16 steps in one graph, each over its
    own index keys (the seeded keys rolled by 2048 l positions, so each selects other rows; a
    graph of one step would time the graph launch)."""
    from embla_attn import ops, synth
    c = synth.sparse_case(seed=3, ctx=32768)
    dev = lambda a, dt=None: (torch.from_numpy(a).cuda().view(dt) if dt is not None else torch.from_numpy(a).cuda())
    q, qi, w, ki = dev(c["q"], torch.float16), dev(c["qi"], torch.float16), dev(c["w"]), dev(c["ki"], torch.float16)
    K, V = dev(c["K"], torch.float16), dev(c["V"], torch.float16)
    ws = ops.SparseWorkspace(32768, 16)
    out = torch.empty(16, 128, dtype=torch.float16, device="cuda")

    kis = [ki] + [torch.roll(ki, 2048 * l, 0).contiguous() for l in range(1, n_layers)]

    def run():
        for l in range(n_layers):
            ops.sparse_layer_decode(q, qi, w, kis[l], K, V, 32768, 32768, 4, ws, out=out)
    wall, ms = time_graph(torch, run, reps, 3)
    us = ms * 1000 / n_layers
    nbytes = 32768 * 64 * 2 + 1152 * 4 * 2 * 128 * 2
    return dict(us_per_layer=us, tokens_per_s=1e6 / us, algorithmic_bytes=nbytes, layers_a_graph=n_layers,
                gbs=nbytes / (us * 1e-6) / 1e9)


def bench_blocks(torch, reps=20):
    """Prefix-cache block save + restore: 16 blocks (positions 16384 + 128 i ..,
    i < 16) of 16 full layers at C3's shape (4 kv heads, 32768 positions, int8 + fp16 scales), each
    saved then restored, in one graph (a graph of a single pair would time the graph launch);
    bytes = each copy's reads and writes."""
    from embla_attn import layout, ops
    n_layers, n_kv, max_s, p0 = 16, 4, 32768, 16384
    rb = (layout.region_bytes(n_kv, max_s, 2) + 255) // 256 * 256
    cache = torch.zeros(2 * n_layers * rb, dtype=torch.uint8, device="cuda")
    regions = [[(2 * l) * rb, (2 * l + 1) * rb] for l in range(n_layers)]
    nbytes = ops.lib().embla_kv_block_bytes(n_layers, n_kv, ops.F16)
    nblk = 16
    stored = torch.empty(nblk * nbytes, dtype=torch.uint8, device="cuda")

    def run():
        for i in range(nblk):
            ops.kv_block_copy(cache, regions, p0 + 128 * i, max_s, n_kv, stored[i * nbytes:], True)
            ops.kv_block_copy(cache, regions, p0 + 128 * i, max_s, n_kv, stored[i * nbytes:], False)
    wall, ms = time_graph(torch, run, reps, 3)
    us = ms * 1000 / nblk
    moved = 2 * 2 * nbytes   # a save and a restore, each reading and writing the block
    return dict(block_bytes=nbytes, us_save_restore=us, gbs=moved / (us * 1e-6) / 1e9)


def bench_gemv(torch, reps=20):
    """The decode projections either side of attention: per layer q/k/v (3072 rows)
    and the o-projection (2048 rows, accumulating into an fp32 residual) of one token, K = 2048,
    4-bit weights in MLX's layout; 48 distinct layers (283 MB of weights, beyond the 256 MB MALL)
    in one graph. Algorithmic bytes: the weights' words, scales and biases."""
    from embla_attn import ops
    n_layers, K = 48, 2048
    rows_qkv, rows_o = 3072, 2048

    def mat_bytes(O):
        return O * K // 2, O * K // 64 * 2

    lw = sum(mat_bytes(O)[0] + 2 * mat_bytes(O)[1] for O in (rows_qkv, rows_o))
    W = torch.randint(0, 256, (n_layers * lw,), dtype=torch.uint8, device="cuda")
    # scales and biases small and finite: overwrite them with bf16 0.01 and -0.075
    segs = []
    at = 0
    for l in range(n_layers):
        lay = []
        for O in (rows_qkv, rows_o):
            wb, sb = mat_bytes(O)
            w0, s0, b0 = at, at + wb, at + wb + sb
            W[s0:s0 + sb].view(torch.bfloat16).fill_(0.01)
            W[b0:b0 + sb].view(torch.bfloat16).fill_(-0.075)
            lay.append((w0, s0, b0, O, 0, 0))
            at += wb + 2 * sb
        segs.append(lay)
    x = torch.randn(K, device="cuda").bfloat16()
    qkv = torch.empty(rows_qkv, dtype=torch.bfloat16, device="cuda")
    resid = torch.zeros(rows_o, dtype=torch.float32, device="cuda")

    def run():
        for l in range(n_layers):
            ops.gemv_q4(W, x, qkv, [segs[l][0]], K, ops.EPI_BF16)
            ops.gemv_q4(W, x, resid, [segs[l][1]], K, ops.EPI_ADD)
    wall, ms = time_graph(torch, run, reps, 3)
    us = ms * 1000 / n_layers
    return dict(layers=n_layers, weight_bytes_layer=lw, us_per_layer=us, gbs=lw / (us * 1e-6) / 1e9,
                frac_hbm=lw / (us * 1e-6) / 1e9 / HBM_PEAK_GBS)


def bench_gemm(torch, reps=10):
    """The prefill projections either side of attention: C5's 2048-token chunk
    through q/k/v (3072 rows) and the o-projection (2048 rows, accumulating into an fp32
    residual), K = 2048, 4-bit weights in MLX's layout; 4 pairs a graph. FLOPs 2 T O K."""
    from embla_attn import ops
    T, K = 2048, 2048
    mats = []
    for O in (3072, 2048):
        wb, sb = O * K // 2, O * K // 64 * 2
        W = torch.randint(0, 256, (wb + 2 * sb,), dtype=torch.uint8, device="cuda")
        W[wb:wb + sb].view(torch.bfloat16).fill_(0.01)
        W[wb + sb:].view(torch.bfloat16).fill_(-0.075)
        mats.append((W, (0, wb, wb + sb), O))
    x = torch.randn(T, K, device="cuda").bfloat16()
    a = torch.randn(T, 2048, device="cuda").bfloat16()
    qkv = torch.empty(T, 3072, dtype=torch.bfloat16, device="cuda")
    resid = torch.zeros(T, 2048, dtype=torch.float32, device="cuda")

    def run():
        ops.gemm_q4(mats[0][0], mats[0][1], x, qkv, T, 3072, K, ops.EPI_BF16)
        ops.gemm_q4(mats[1][0], mats[1][1], a, resid, T, 2048, K, ops.EPI_ADD)
    ms = time_calls(torch, run, 4, reps, 2)
    flops = 2.0 * T * K * (3072 + 2048)
    return dict(gflop=flops / 1e9, ms=ms, tflops=flops / (ms * 1e-3) / 1e12,
                mfma_util=flops / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS)


def bench_step(torch, regions, L=32768, reps=20, fused=True):
    """The whole attention sub-layer decode step of one token over C3's 16-layer
    stack at context L, captured as one graph: per layer the 4-bit q/k/v projection, the int8 append
    of the new k and v at position L - 1, the split-K decode over L positions with the q head norm
    inside its kernel (bf16 out) and the 4-bit o-projection into the fp32 residual. fused: the
    append inside the decode launch (embla_decode_step_int8, 4 kernels a layer), else its own
    launch (5). Algorithmic bytes a layer: the cache as in C3 plus the weights."""
    from embla_attn import ops
    n_layers, D, n_q, n_kv, max_s = len(regions), 2048, 16, 4, 32768

    def mat_bytes(O):
        return O * D // 2, O * D // 64 * 2

    lw = sum(mat_bytes(O)[0] + 2 * mat_bytes(O)[1] for O in (3072, D))
    W = torch.randint(0, 256, (n_layers * lw,), dtype=torch.uint8, device="cuda")
    segs, at = [], 0
    for l in range(n_layers):
        lay = []
        for O in (3072, D):
            wb, sb = mat_bytes(O)
            W[at + wb:at + wb + sb].view(torch.bfloat16).fill_(0.002)
            W[at + wb + sb:at + wb + 2 * sb].view(torch.bfloat16).fill_(-0.015)
            lay.append((at, at + wb, at + wb + sb, O, 0, 0))
            at += wb + 2 * sb
        segs.append(lay)
    x = torch.randn(D, device="cuda").bfloat16()
    qkv = torch.empty(3072, dtype=torch.bfloat16, device="cuda")
    o = torch.empty(n_q, 128, dtype=torch.bfloat16, device="cuda")
    resid = torch.empty(D, dtype=torch.float32, device="cuda")
    ws = ops.Workspace(max_s, n_q)

    def run():
        resid.zero_()
        for l in range(n_layers):
            kc, vc = regions[l]
            ops.gemv_q4(W, x, qkv, [segs[l][0]], D, ops.EPI_BF16)
            if fused:
                ops.decode_step_int8(qkv, 0, 2048, 2560, kc, vc, L - 1, max_s, n_q, n_kv, ws, out=o)
            else:
                ops.kv_quant_append(qkv[2048:2560], qkv[2560:3072], 1, L - 1, n_kv, kc, vc, max_s)
                ops.decode_int8_qraw(qkv[:2048], kc, vc, L, max_s, n_kv, ws=ws, out=o)
            ops.gemv_q4(W, o, resid, [segs[l][1]], D, ops.EPI_ADD)
    wall, ms = time_graph(torch, run, reps, 3)
    us = ms * 1000 / n_layers
    nbytes = layer_bytes(L) + lw
    return dict(context=L, layers=n_layers, kernels_per_layer=4 if fused else 5, bytes_layer=nbytes, us_per_layer=us,
                gbs=nbytes / (us * 1e-6) / 1e9, frac_hbm=nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS)


def bench_sampling(torch, reps=10):
    """The sampling tail on a 65536-token row: the greedy token, a top-p draw over
    few candidates (a peaked row: 316 tokens within 1/16384 of the top) and a draw that bisects
    over every token (a flat row); 32 positions a graph. Latency-bound: µs a call."""
    from embla_attn import ops
    V, n = 65536, 32
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    flat = torch.randn(V, device="cuda", generator=g)
    peaked = torch.randn(V, device="cuda", generator=g) - 6
    hot = torch.randperm(V, device="cuda", generator=g)[:300]
    peaked[hot] = torch.rand(300, device="cuda", generator=g) * 6 + 2
    st = ops.SampleState(V, n + 2)
    res = {}
    for name, fn in [
        ("greedy_us", lambda p: ops.argmax(flat, st, p)),
        ("draw_candidates_us", lambda p: ops.sample(peaked, st, p, 1.0, 0.9, 7)),
        ("draw_all_tokens_us", lambda p: ops.sample(flat, st, p, 1.0, 0.9, 7)),
    ]:
        def run(fn=fn):
            for p in range(n):
                fn(p)
        _, ms = time_graph(torch, run, reps, 2)
        res[name] = ms * 1000 / n
    res["vocab"] = V
    return res


def prefill_flops(p0: int, T: int, n_q: int = 16, window: int = 0) -> float:
    """Algorithmic FLOPs of causal prefill attention: 4·128 a (query row, key) pair (QK and PV)."""
    pairs = 0
    for i in range(T):
        n = p0 + i + 1
        pairs += min(n, window) if window else n
    return pairs * n_q * 4 * 128


def bench_c5(torch, reps=10):
    """Config C5 full layer: a 2048-token chunk after 30720 cached int8 positions: the fused
    quantise-and-append + causal attention, and the attention alone."""
    from embla_attn import ops
    p0, T, max_s, n_kv = 30720, 2048, 32768, 4
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    nrow = n_kv * max_s * 128
    kc = torch.empty(nrow + n_kv * max_s * 2, dtype=torch.uint8, device="cuda")
    vc = torch.empty_like(kc)
    for t in (kc, vc):
        t[:nrow].random_(0, 256, generator=g)
        t[nrow:].view(torch.float16).uniform_(0.005, 0.02, generator=g)
    q = torch.randn(T, 16, 128, generator=g, device="cuda").bfloat16()
    kn = torch.randn(T, n_kv, 128, generator=g, device="cuda").bfloat16()
    vn = torch.randn(T, n_kv, 128, generator=g, device="cuda").bfloat16()
    out = torch.empty(T, 16, 128, dtype=torch.bfloat16, device="cuda")
    flops = prefill_flops(p0, T)
    ws = ops.PrefillWorkspace(T, 16, staged_p0=p0)
    # ~0.2 s of the attention first: the shader clock ramps over the first hundreds of ms of MFMA
    # load, and whichever call was timed first read ~10% slow
    time_graph(torch, lambda: ops.prefill_int8(q, kc, vc, T, p0, max_s, n_kv, out=out, ws=ws), 300, 2)
    _, ms_fused = time_graph(torch, lambda: ops.prefill_full(q, kn, vn, kc, vc, T, p0, max_s, n_kv, out=out, ws=ws), reps, 2)
    _, ms_attn = time_graph(torch, lambda: ops.prefill_int8(q, kc, vc, T, p0, max_s, n_kv, out=out, ws=ws), reps, 2)
    full = dict(gflop=flops / 1e9, ms_attention=ms_attn, tflops_attention=flops / (ms_attn * 1e-3) / 1e12,
                mfma_util_attention=flops / (ms_attn * 1e-3) / 2.5e15, ms_fused=ms_fused,
                tflops_fused=flops / (ms_fused * 1e-3) / 1e12, tokens_per_s=T / (ms_fused * 1e-3))
    # sliding layer: the same chunk, window 1024, over a bf16 ring of 8192 (append + attention)
    R, W = 8192, 1024
    kring = torch.randn(n_kv * R * 128, generator=g, device="cuda").bfloat16()
    vring = torch.randn(n_kv * R * 128, generator=g, device="cuda").bfloat16()
    sflops = 4.0 * 128 * 16 * sum(min(W, p0 + t + 1) for t in range(T))
    ms_sl = time_calls(torch, lambda: ops.prefill_sliding(q, kn, vn, kring, vring, T, p0, R, W, n_kv, out=out, ws=ws),
                       8, reps, 2)
    ms_sla = time_calls(torch, lambda: ops.prefill_ring(q, kring, vring, T, p0, R, W, n_kv, out=out, ws=ws), 8, reps, 2)
    sliding = dict(window=W, ring=R, gflop=sflops / 1e9, ms_attention=ms_sla,
                   tflops_attention=sflops / (ms_sla * 1e-3) / 1e12,
                   mfma_util_attention=sflops / (ms_sla * 1e-3) / 2.5e15, ms_fused=ms_sl,
                   tokens_per_s=T / (ms_sl * 1e-3))
    # sparse layer: the same chunk, per-row top-1024 + latest 128 by the index score, over a
    # row-major int8 cache (quantise-and-append, MFMA indexer, exact band select, gathered attention)
    kr = torch.empty(nrow + n_kv * max_s * 2, dtype=torch.uint8, device="cuda")
    vr = torch.empty_like(kr)
    for t in (kr, vr):
        t[:nrow].random_(0, 256, generator=g)
        t[nrow:].view(torch.float16).uniform_(0.005, 0.02, generator=g)
    qi = torch.randn(T, 4, 64, generator=g, device="cuda").half()
    wi = torch.rand(T, 4, generator=g, device="cuda")
    ki = torch.randn(p0 + T, 64, generator=g, device="cuda").half()
    sws = ops.SparsePrefillWorkspace(T, p0)
    ms_sp = time_calls(torch, lambda: ops.prefill_sparse(q, kn, vn, qi, wi, ki, kr, vr, T, p0, max_s, n_kv, sws,
                                                         out=out), 2, reps, 2)
    att = 4.0 * 128 * 16 * T * 1152
    idxf = 4.0 * 128 * sum(p0 + t + 1 - 128 for t in range(T))
    sparse = dict(gflop_attention=att / 1e9, gflop_indexer=idxf / 1e9, ms_layer=ms_sp,
                  tflops_layer=(att + idxf) / (ms_sp * 1e-3) / 1e12,
                  mfma_util_layer=(att + idxf) / (ms_sp * 1e-3) / 2.5e15, tokens_per_s=T / (ms_sp * 1e-3))
    return dict(full, sliding=sliding, sparse=sparse)


def _cpu_threads():
    """Host threads the baseline uses: OMP_NUM_THREADS when set (the GPU box sets it to its CPU
    share), else every core this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def _timed(fn, budget_s, min_n=2, max_n=200):
    out, n, t0 = None, 0, time.perf_counter()
    while n < min_n or (time.perf_counter() - t0 < budget_s and n < max_n):
        out = fn()
        n += 1
    return (time.perf_counter() - t0) / n, n, out


def cpu_baseline(case, L, budget_s=6.0):
    """The oracle's C restatement of the reference's math (oracle/oracle.c) built at -O3
    -march=native with OpenMP (liborc_omp.so: threads over query heads, prefill rows and index
    keys; the same results as the checker build), timed on this host's cores: C3 whole layers at
    context L (GB/s, the headline's unit), plus C2 (decode steps over the 1024-position window),
    C4 (one sparse-layer step: index scores, top-k, attention over the 1152 rows) and C5 full,
    sliding and sparse (samples of the 2048-row chunk, scaled to TFLOP/s). The reference itself
    has no CPU attention path (all of it is Metal)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np
    import orc
    from embla_attn import synth
    orc.use_openmp(True)
    threads = _cpu_threads()
    os.environ["OMP_NUM_THREADS"] = str(threads)
    q = synth.f16_val(case["q"])
    K, V = case["K"][:, :L], case["V"][:, :L]
    ks, vs = synth.f16_val(case["ks"][:, :L]), synth.f16_val(case["vs"][:, :L])
    dt3, n3, out = _timed(lambda: orc.decode_int8(q, K, ks, V, vs), budget_s)
    # C4: one sparse-layer decode step at context 32768
    c4 = synth.sparse_case(seed=3, ctx=32768)
    ctx = 32768

    q4, K4, V4 = synth.f16_val(c4["q"]), synth.f16_val(c4["K"]), synth.f16_val(c4["V"])

    def c4_step():
        sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:ctx - 128])
        sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), ctx)
        return orc.decode_rows(q4, K4, V4, sel.astype(np.int32))
    dt4, n4, _ = _timed(c4_step, budget_s / 2)
    # C5 full: 64 consecutive rows from the middle of the chunk (row i attends p0 + i + 1 keys),
    # threads over the rows, scaled to TFLOP/s by their exact pair count
    p0, T, r0, nr = 30720, 2048, 992, 64
    c5 = synth.prefill_case(seed=4, p0=p0, T=T)
    Kc = np.concatenate([c5["K"], np.zeros((4, T, 128), np.int8)], 1)
    Vc = np.concatenate([c5["V"], np.zeros((4, T, 128), np.int8)], 1)
    ksc = np.concatenate([synth.f16_val(c5["ks"]), np.full((4, T), 0.01, np.float32)], 1)
    vsc = np.concatenate([synth.f16_val(c5["vs"]), np.full((4, T), 0.01, np.float32)], 1)
    qf = synth.bf16_val(c5["q"][r0:r0 + nr])
    flops_rows = float(sum((p0 + r0 + i + 1) * 16 * 512 for i in range(nr)))

    def c5_rows():
        return orc.prefill_int8(qf, Kc, ksc, Vc, vsc, p0 + r0)
    dt5, n5, _ = _timed(c5_rows, budget_s / 2, min_n=1, max_n=5)
    # C2: decode steps over a window of 1024 positions of an fp16 ring (the values of an N(0,1)
    # fp16 history; the oracle attends positions pos - 1023 .. pos)
    g = np.random.default_rng(1)
    Kr = g.standard_normal((4, 8192, 128)).astype(np.float16).astype(np.float32)
    Vr = g.standard_normal((4, 8192, 128)).astype(np.float16).astype(np.float32)
    q2 = g.standard_normal((16, 128)).astype(np.float16).astype(np.float32)
    win = np.arange(8192 - 1024, 8192, dtype=np.int32)
    dt2, n2, _ = _timed(lambda: orc.decode_rows(q2, Kr, Vr, win), budget_s / 4)
    # C5 sliding: a 64-row sample of the chunk, each row over its 1024-position window (scaled
    # to TFLOP/s by the rows' pair count)
    qs5 = g.standard_normal((nr, 16, 128)).astype(np.float16).astype(np.float32)

    def c5_sliding_rows():
        for i in range(nr):
            orc.decode_rows(qs5[i], Kr, Vr, win)
    dt6, n6, _ = _timed(c5_sliding_rows, budget_s / 4, min_n=1, max_n=400)
    sl_flops = float(nr * 1024 * 16 * 512)
    # C5 sparse: 4 rows of the chunk at positions near its end, each its own index scores over
    # ~32K keys, select_keys, attention over its 1152 rows (int8 cache, fp16 scales)
    ki5 = g.standard_normal((p0 + T, 64)).astype(np.float16).view(np.uint16)
    qi5 = g.standard_normal((4, 4, 64)).astype(np.float16).view(np.uint16)
    wi5 = g.random((4, 4)).astype(np.float32)
    q5s = synth.bf16_val(c5["q"][T - 4:T])

    def c5_sparse_rows():
        for i in range(4):
            S = p0 + T - 4 + i + 1
            sc = orc.index_scores(qi5[i], wi5[i], ki5[:S - 128])
            sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
            orc.prefill_int8(q5s[i:i + 1], Kc, ksc, Vc, vsc, S - 1, rows_sel=sel[None])
    dt7, n7, _ = _timed(c5_sparse_rows, budget_s / 4, min_n=1, max_n=400)
    sp_flops = float(sum(4 * 128 * (p0 + T - 4 + i + 1 - 128) + 4 * 128 * 16 * 1152 for i in range(4)))
    orc.use_openmp(False)
    cores = os.cpu_count()
    base = dict(cores=threads, host_cpus=cores, kind="port", build="oracle/oracle.c, gcc -O3 -march=native -fopenmp")
    c3 = dict(value=layer_bytes(L) / dt3 / 1e9, unit="GB/s", **base,
              sample=f"{n3} whole C3 layers at context {L} (16 q / 4 kv heads), {dt3 * 1e6:.0f} us a layer, "
                     f"{threads} OpenMP threads over the 16 query heads")
    more = {
        "c4_sparse": dict(value=dt4 * 1e6, unit="us/layer", sample=f"{n4} C4 sparse-layer steps at context 32768 "
                          "(index scores of 32640 keys over threads, serial top-k, attention over 1152 rows)"),
        "c5_prefill_full": dict(value=flops_rows / dt5 / 1e12, unit="TFLOP/s",
                                sample=f"{n5} passes over rows {r0}..{r0 + nr - 1} of the C5 chunk "
                                       f"({flops_rows / 1e9:.2f} GFLOP a pass, {dt5 * 1e3:.0f} ms), threads over rows"),
        "c2_sliding": dict(value=dt2 * 1e6, unit="us/step", tokens_per_s=1.0 / dt2,
                           sample=f"{n2} C2 decode steps (16 q / 4 kv heads, window 1024 of an fp16 ring of 8192)"),
        "c5_prefill_sliding": dict(value=sl_flops / dt6 / 1e12, unit="TFLOP/s", tokens_per_s=nr / dt6,
                                   sample=f"{n6} passes over {nr} rows of the C5 chunk, each over its 1024-position "
                                          f"window ({sl_flops / 1e9:.2f} GFLOP a pass, {dt6 * 1e3:.0f} ms)"),
        "c5_prefill_sparse": dict(value=sp_flops / dt7 / 1e12, unit="TFLOP/s", tokens_per_s=4 / dt7,
                                  sample=f"{n7} passes over 4 rows at the end of the C5 chunk: index scores over "
                                         f"their ~32K keys, select_keys, attention over the 1152 rows "
                                         f"({sp_flops / 1e9:.3f} GFLOP a pass, {dt7 * 1e3:.0f} ms)"),
    }
    c3["more"] = more
    return c3, out


def traffic_probe(torch, reps=6):
    """Dispatches for the HBM traffic counters: a C3 decode call at 32k (split-K kernel + merge)
    and a 64 MB device copy (the counters' calibration), each after a 512 MB fill that evicts the
    caches, so both read from HBM."""
    from embla_attn import ops
    regions, case = make_caches(torch, 2, 32768)
    q = torch.from_numpy(case["q"]).cuda().view(torch.float16)
    ws = ops.Workspace(32768, 16)
    out = torch.empty((16, 128), dtype=torch.float16, device="cuda")
    src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    big = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    for i in range(reps):
        big.zero_()
        ops.decode_int8(q, regions[i % 2][0], regions[i % 2][1], 32768, 32768, 4, ws=ws, out=out)
        big.zero_()
        dst.copy_(src)
    torch.cuda.synchronize()


def measured_traffic():
    """HBM bytes a C3 decode launch moves, from the committed counter summary (FETCH_SIZE scaled by
    the copy calibration, plus WRITE_SIZE), or None."""
    f = ROOT / "profiles" / "decode_c3_hbm_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def profile_case(torch, name, calls=5):
    """Only dispatches one workload's calls, eagerly, for rocprofv3 --pmc runs (the last dispatch
    is read): 'c5_full' = C5's full-layer attention (embla_prefill_int8, 2048 rows after 30720
    int8 positions); 'gemm_prefill' = the q/k/v projection GEMM of C5's chunk (T 2048, O 3072,
    K 2048); 'c5_sparse' = C5's sparse layer (embla_prefill_sparse: indexer, band select,
    gathered attention); 'c4' = C4 sparse-layer decode steps at context 32768 (scorer, classify,
    the attention with the select's last step, merge). Prints nothing."""
    from embla_attn import ops
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    if name == "c5_full":
        p0, T, max_s, n_kv = 30720, 2048, 32768, 4
        nrow = n_kv * max_s * 128
        kc = torch.empty(nrow + n_kv * max_s * 2, dtype=torch.uint8, device="cuda")
        vc = torch.empty_like(kc)
        for t in (kc, vc):
            t[:nrow].random_(0, 256, generator=g)
            t[nrow:].view(torch.float16).uniform_(0.005, 0.02, generator=g)
        q = torch.randn(T, 16, 128, generator=g, device="cuda").bfloat16()
        out = torch.empty(T, 16, 128, dtype=torch.bfloat16, device="cuda")
        ws = ops.PrefillWorkspace(T, 16, staged_p0=p0)
        for _ in range(calls):
            ops.prefill_int8(q, kc, vc, T, p0, max_s, n_kv, out=out, ws=ws)
    elif name == "gemm_prefill":
        T, K, O = 2048, 2048, 3072
        wb, sb = O * K // 2, O * K // 64 * 2
        W = torch.randint(0, 256, (wb + 2 * sb,), dtype=torch.uint8, device="cuda", generator=g)
        W[wb:wb + sb].view(torch.bfloat16).fill_(0.01)
        W[wb + sb:].view(torch.bfloat16).fill_(-0.075)
        x = torch.randn(T, K, device="cuda", generator=g).bfloat16()
        y = torch.empty(T, O, dtype=torch.bfloat16, device="cuda")
        for _ in range(calls):
            ops.gemm_q4(W, (0, wb, wb + sb), x, y, T, O, K, ops.EPI_BF16)
    elif name == "c5_sparse":
        p0, T, n_kv = 30720, 2048, 4
        max_s = p0 + T
        nrow = n_kv * max_s * 128
        kr = torch.empty(nrow + n_kv * max_s * 2, dtype=torch.uint8, device="cuda")
        vr = torch.empty_like(kr)
        for t in (kr, vr):
            t[:nrow].random_(0, 256, generator=g)
            t[nrow:].view(torch.float16).uniform_(0.005, 0.02, generator=g)
        q = torch.randn(T, 16, 128, generator=g, device="cuda").bfloat16()
        kn = torch.randn(T, n_kv, 128, generator=g, device="cuda").bfloat16()
        vn = torch.randn(T, n_kv, 128, generator=g, device="cuda").bfloat16()
        qi = torch.randn(T, 4, 64, generator=g, device="cuda").half()
        wi = torch.rand(T, 4, generator=g, device="cuda")
        ki = torch.randn(p0 + T, 64, generator=g, device="cuda").half()
        out = torch.empty(T, 16, 128, dtype=torch.bfloat16, device="cuda")
        sws = ops.SparsePrefillWorkspace(T, p0)
        for _ in range(calls):
            ops.prefill_sparse(q, kn, vn, qi, wi, ki, kr, vr, T, p0, max_s, n_kv, sws, out=out)
    elif name == "c4":
        from embla_attn import synth
        c = synth.sparse_case(seed=3, ctx=32768)
        dev = lambda a, dt=None: (torch.from_numpy(a).cuda().view(dt) if dt is not None else torch.from_numpy(a).cuda())
        q, qi, w, ki = dev(c["q"], torch.float16), dev(c["qi"], torch.float16), dev(c["w"]), dev(c["ki"], torch.float16)
        K, V = dev(c["K"], torch.float16), dev(c["V"], torch.float16)
        ws = ops.SparseWorkspace(32768, 16)
        out = torch.empty(16, 128, dtype=torch.float16, device="cuda")
        kis = [ki] + [torch.roll(ki, 2048 * l, 0).contiguous() for l in range(1, 16)]
        for _ in range(calls):
            for l in range(16):
                ops.sparse_layer_decode(q, qi, w, kis[l], K, V, 32768, 32768, 4, ws, out=out)
    else:
        raise SystemExit(f"unknown profile case {name}")
    torch.cuda.synchronize()


def render_table(d):
    """The current-numbers table (markdown) of a bench line: each config's time, throughput and
    roofline fraction, the floors measured beside them, and the CPU baselines."""
    r = lambda x, n=2: f"{x:,.{n}f}"
    c5, sl, sp = d["c5_prefill_full"], d["c5_prefill_sliding"], d["c5_prefill_sparse"]
    rows = [
        ("C3 decode, 32K, 16-layer stack (`value`)", f"{r(d['us_per_layer'], 2)} µs/layer",
         f"{r(d['value'], 0)} GB/s; {r(d['tokens_per_s'], 0)} tokens/s through 16 layers, {r(d['tokens_per_s_one_layer'], 0)} through one",
         f"{d['layer_roofline']['frac']:.3f} of HBM"),
        ("C3 split-K kernel (`roofline`)", f"{r(d['roofline']['launch_us'], 2)} µs/launch",
         f"{r(d['roofline']['achieved'], 0)} GB/s; traffic {d['roofline']['traffic'] / d['roofline']['per_launch_bytes']:.3f}x algorithmic",
         f"{d['roofline']['frac']:.3f} of HBM"),
        ("C3 one layer alone, cold caches", f"{r(d['c3_single_layer_cold']['us_cold_median'], 2)} µs",
         f"{r(d['c3_single_layer_cold']['gbs'], 0)} GB/s", f"{d['c3_single_layer_cold']['gbs'] / HBM_PEAK_GBS:.3f} of HBM"),
        ("C3 sweep 4K / 16K", f"{r(d['c3_sweep_us_per_layer']['4096'])} / {r(d['c3_sweep_us_per_layer']['16384'])} µs/layer",
         f"{r(d['c3_sweep_gbs']['4096'], 0)} / {r(d['c3_sweep_gbs']['16384'], 0)} GB/s", "launch-bound at 4K"),
        ("HBM read floor (probe, one 34 MB launch)", f"{r(d['hbm_read_floor']['us_per_launch'])} µs",
         f"{r(d['hbm_read_floor']['gbs'], 0)} GB/s; split-K = {d['hbm_read_floor']['split_k_launch_over_floor']:.2f}x it",
         f"{d['hbm_read_floor']['frac_of_peak']:.3f} of HBM"),
        ("C2 sliding decode (512 steps, one graph)", f"{r(d['c2_sliding']['us_per_step'])} µs/step",
         f"{r(d['c2_sliding']['tokens_per_s'], 0)} tokens/s", "latency (2 MB cache-resident)"),
        ("C4 sparse-layer decode, 32K", f"{r(d['c4_sparse']['us_per_layer'])} µs/layer",
         f"{r(d['c4_sparse']['tokens_per_s'], 0)} tokens/s", f"{d['c4_sparse']['gbs'] / HBM_PEAK_GBS:.3f} of HBM (latency)"),
        ("C5 full prefill attention", f"{r(c5['ms_attention'], 3)} ms", f"{r(c5['tflops_attention'], 0)} TFLOP/s; "
         f"fused with the append {r(c5['ms_fused'], 3)} ms, {r(c5['tokens_per_s'], 0)} tokens/s",
         f"{c5['mfma_util_attention']:.3f} of bf16 MFMA ({c5['frac_of_sustained_mfma']:.2f} of the MFMA-only probe)"),
        ("C5 sliding prefill attention", f"{r(sl['ms_attention'], 4)} ms", f"{r(sl['tflops_attention'], 0)} TFLOP/s",
         f"{sl['mfma_util_attention']:.3f} of bf16 MFMA"),
        ("C5 sparse prefill layer", f"{r(sp['ms_layer'], 3)} ms", f"{r(sp['tflops_layer'], 0)} TFLOP/s (indexer + attention)",
         f"{sp['mfma_util_layer']:.3f} of bf16 MFMA (gather address work)"),
        ("MFMA-only probe", f"{r(d['mfma_ceiling']['ms'], 3)} ms", f"{r(d['mfma_ceiling']['tflops'], 0)} TFLOP/s",
         f"{d['mfma_ceiling']['frac_of_peak']:.3f} of bf16 MFMA"),
        ("decode sub-layer step (q/k/v GEMV, decode with append, o GEMV)",
         f"{r(d['decode_sublayer_step_graph']['us_per_layer'])} µs/layer", f"{r(d['decode_sublayer_step_graph']['gbs'], 0)} GB/s",
         f"{d['decode_sublayer_step_graph']['frac_hbm']:.3f} of HBM"),
        ("4-bit projections, decode (GEMV)", f"{r(d['qkv_o_projections_decode']['us_per_layer'])} µs/layer",
         f"{r(d['qkv_o_projections_decode']['gbs'], 0)} GB/s", f"{d['qkv_o_projections_decode']['frac_hbm']:.3f} of HBM (launch-bound)"),
        ("4-bit projections, prefill (GEMM)", f"{r(d['qkv_o_projections_prefill']['ms'], 4)} ms",
         f"{r(d['qkv_o_projections_prefill']['tflops'], 0)} TFLOP/s", f"{d['qkv_o_projections_prefill']['mfma_util']:.3f} of bf16 MFMA"),
        ("sampling tail, V = 65536", f"{r(d['sampling_tail']['greedy_us'])} / {r(d['sampling_tail']['draw_candidates_us'])} / "
         f"{r(d['sampling_tail']['draw_all_tokens_us'])} µs", "greedy / draw (few candidates) / draw (all tokens)", "latency"),
        ("KV block save + restore (2.13 MB)", f"{r(d['kv_block_save_restore']['us_save_restore'])} µs",
         f"{r(d['kv_block_save_restore']['gbs'], 0)} GB/s", "launch-bound"),
    ]
    out = ["| workload | time | throughput | bound, fraction |", "|---|---:|---|---|"]
    out += [f"| {a} | {b} | {c} | {e} |" for a, b, c, e in rows]
    cb = d.get("cpu_baseline")
    if cb:
        out += ["", f"CPU baseline (`cpu_baseline`, the C oracle on {cb['cores']} host threads, kind \"{cb['kind']}\"):", "",
                "| workload | CPU | GPU / CPU |", "|---|---:|---:|",
                f"| C3 layer | {r(cb['value'], 2)} GB/s | {d['value'] / cb['value']:,.0f}x |"]
        more, gpu = cb["more"], {"c4_sparse": d["c4_sparse"]["us_per_layer"], "c2_sliding": d["c2_sliding"]["us_per_step"],
                                 "c5_prefill_full": c5["tflops_attention"], "c5_prefill_sliding": sl["tflops_attention"],
                                 "c5_prefill_sparse": sp["tflops_layer"]}
        for k, v in more.items():
            ratio = v["value"] / gpu[k] if v["unit"].startswith("us") else gpu[k] / v["value"]
            out.append(f"| {k} | {r(v['value'], 4 if v['unit'] == 'TFLOP/s' else 1)} {v['unit']} | {ratio:,.0f}x |")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline (C3 at 32k, 16-layer graph) and print its JSON line; "
                         "for kernel-trace profiles of the headline alone")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only dispatch C3 decode layers and a 64 MB copy (each after a cache-evicting "
                         "fill) for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs; prints nothing else")
    ap.add_argument("--table", metavar="JSON",
                    help="print the current-numbers table (markdown) of a saved bench line and exit (no GPU)")
    ap.add_argument("--profile-case", choices=["c5_full", "gemm_prefill", "c5_sparse", "c4"],
                    help="only dispatch one workload's calls (for rocprofv3 --pmc runs); prints nothing")
    args = ap.parse_args()
    if args.table:
        print(render_table(json.loads(Path(args.table).read_text().strip().splitlines()[-1])))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the attention hot path runs on a "
                                   "single MI355X (multi-GPU sharding is design only); run with --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    from embla_attn import _lib
    _lib.lib()   # the HIP library must load; there is no fallback path
    if args.traffic_probe:
        traffic_probe(torch)
        return
    if args.profile_case:
        profile_case(torch, args.profile_case)
        return

    L = 32768
    if args.headline_only:
        res, case, out0, _, main_us = bench_c3(torch, args.steps, args.warmup, contexts=(L,))
        h = res[L]
        print(json.dumps({"metric": METRIC, "value": round(h["gbs"], 1), "unit": "GB/s",
                          "us_per_layer": round(h["us_per_layer"], 3), "main_kernel_us": round(main_us, 3),
                          "steps": args.steps}))
        return
    res, case, out0, regions, main_us = bench_c3(torch, args.steps, args.warmup)
    single = bench_c3_single(torch, regions, case)
    floor = bench_read_floor(torch)
    step = bench_step(torch, regions)
    step["us_per_layer_append_own_launch"] = bench_step(torch, regions, fused=False)["us_per_layer"]
    sampling = bench_sampling(torch)
    c2 = bench_c2(torch)
    c4 = bench_c4(torch)
    c5 = bench_c5(torch)
    mfma_ceiling = bench_mfma_ceiling(torch)
    c5["frac_of_sustained_mfma"] = c5["tflops_attention"] / mfma_ceiling["tflops"]
    blocks = bench_blocks(torch)
    gemv = bench_gemv(torch)
    gemm = bench_gemm(torch)
    head = res[L]
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "C3 full-layer int8 decode, context 32768, 16-layer stack of distinct caches",
                   "context": L, "layers": 16, "q_heads": 16, "kv_heads": 4, "head_dim": 128,
                   "kv": "int8 + fp16 scales", "graph": True},
        "us_per_layer": round(head["us_per_layer"], 3),
        # decode throughput of one token: through the 16-layer stack, and through one layer
        "tokens_per_s": round(1e6 / (16 * head["us_per_layer"]), 1),
        "tokens_per_s_one_layer": round(1e6 / head["us_per_layer"], 1),
        "c3_single_layer_cold": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in single.items()},
        # the dominant kernel (the split-K pass over the cache, 16 launches a graph timed by events
        # on the launching stream); the whole layer call (with the merge and the launch gaps) is
        # value / layer_roofline
        "roofline": {
            "bound": "hbm",
            "achieved": round(main_kernel_bytes(L) / (main_us * 1e-6) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(main_kernel_bytes(L) / (main_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "kernel": "full_decode_kernel (the split-K pass of one layer's decode, C3 at 32768)",
            "per_launch_bytes": main_kernel_bytes(L),
            "launch_us": round(main_us, 3),
        },
        "layer_roofline": {
            "achieved": round(layer_bytes(L) / (head["us_per_layer"] * 1e-6) / 1e9, 1),
            "frac": round(layer_bytes(L) / (head["us_per_layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "kernels": "full_decode_kernel + decode_merge_kernel (one layer's decode call)",
            "per_call_bytes": layer_bytes(L),
        },
        "hbm_read_floor": {
            "what": "a plain streaming read of one layer's K+V bytes in one launch (the bench-only probe library), "
                    "16 distinct buffers a graph: the practical floor of the split-K pass at this size",
            "bytes": floor["bytes"], "grid": floor["grid"], "us_per_launch": round(floor["us_per_launch"], 3),
            "gbs": round(floor["gbs"], 1), "frac_of_peak": round(floor["gbs"] / HBM_PEAK_GBS, 4),
            "split_k_launch_over_floor": round(main_us / floor["us_per_launch"], 3),
        },
        "c3_sweep_us_per_layer": {str(k): round(v["us_per_layer"], 3) for k, v in res.items()},
        "c3_sweep_gbs": {str(k): round(v["gbs"], 1) for k, v in res.items()},
        "c3_sweep_us_per_layer_median": {str(k): round(v["us_per_layer_median"], 3) for k, v in res.items()},
        "c2_sliding": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in c2.items()},
        "c4_sparse": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in c4.items()},
        "c5_prefill_full": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in c5.items()
                            if k not in ("sliding", "sparse")},
        "mfma_ceiling": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in mfma_ceiling.items()},
        "c5_prefill_sparse": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in c5["sparse"].items()},
        "kv_block_save_restore": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in blocks.items()},
        "qkv_o_projections_decode": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in gemv.items()},
        "decode_sublayer_step_graph": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in step.items()},
        "sampling_tail": {k: (round(v, 3) if isinstance(v, float) else v) for k, v in sampling.items()},
        "qkv_o_projections_prefill": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in gemm.items()},
        "c5_prefill_sliding": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in c5["sliding"].items()},
    }
    if not args.no_cpu:
        cb, ref = cpu_baseline(case, L)
        line["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cb.items()}
        got = out0.float().cpu().numpy()
        line["parity_max_abs_err_layer0"] = float(np.abs(got - ref).max())
    print(json.dumps(line))


if __name__ == "__main__":
    main()
