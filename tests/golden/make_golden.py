"""Writes the golden fixtures of this directory: oracle outputs (oracle/oracle.c) on seeded
SplitMix64 inputs of the BASELINE configs at small sizes, with a SHA-256 digest of the inputs.

The reference (Swift + Metal) ships no attention vectors and cannot run here, so these fixtures
pin the oracle and the input generator against drift (tests/test_oracle.py re-derives them on the
CPU) and give the GPU tests expected outputs that do not need the C oracle at run time.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "embla-metal_amd"))


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def c1_decode(orc, synth):
    """C1: one decode step, 16 q / 4 kv heads, context 1024, int8 KV + fp16 scales, seed 0."""
    c = synth.decode_int8_case(seed=0, S=1024)
    out = orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    return dict(out=out.astype(np.float32), digest=digest(c["q"], c["K"], c["ks"], c["V"], c["vs"]))


def c4_select(orc, synth):
    """C4 at context 4096: index scores of the 3968 candidates and the 1152 selected rows."""
    c = synth.sparse_case(seed=3, ctx=4096)
    sc = orc.index_scores(c["qi"], c["w"], c["ki"][:4096 - 128])
    sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), 4096)
    return dict(scores=sc.astype(np.float32), sel=sel.astype(np.uint32), digest=digest(c["qi"], c["w"], c["ki"]))


def quant_rows(orc, synth):
    """int8 quantise-and-append of 64 bf16 rows (N(0,1) times 1..4), as the configs' append."""
    g = synth.SplitMix64(77)
    x = synth.bf16_bits((g.normal(64 * 128) * np.repeat(np.arange(1, 5), 16 * 128)).astype(np.float32)).reshape(64, 128)
    q = np.empty((64, 128), np.int8)
    s = np.empty(64, np.float32)
    for i in range(64):
        q[i], s[i] = orc.quant_row(synth.bf16_val(x[i]), round_bf=True)
    return dict(x=x, q=q, scale=s, digest=digest(x))


def c5_prefill(orc, synth):
    """C5 full layer at p0 = 300, T = 40 (causal softmax over the int8 cache after the chunk's
    quantise-and-append): the oracle output of every row."""
    c = synth.prefill_case(seed=4, p0=300, T=40)
    n_kv, p0, T = 4, 300, 40
    K = np.concatenate([c["K"], np.zeros((n_kv, T, 128), np.int8)], 1)
    V = np.concatenate([c["V"], np.zeros((n_kv, T, 128), np.int8)], 1)
    ks = np.concatenate([synth.f16_val(c["ks"]), np.zeros((n_kv, T), np.float32)], 1)
    vs = np.concatenate([synth.f16_val(c["vs"]), np.zeros((n_kv, T), np.float32)], 1)
    for h in range(n_kv):
        for t in range(T):
            K[h, p0 + t], sk = orc.quant_row(synth.bf16_val(c["kn"][t, h]), round_bf=True)
            V[h, p0 + t], sv = orc.quant_row(synth.bf16_val(c["vn"][t, h]), round_bf=True)
            ks[h, p0 + t] = synth.f16_val(synth.f16_bits(np.float32(sk)))
            vs[h, p0 + t] = synth.f16_val(synth.f16_bits(np.float32(sv)))
    out = orc.prefill_int8(synth.bf16_val(c["q"]), K, ks, V, vs, p0)
    return dict(out=out.astype(np.float32), digest=digest(c["K"], c["ks"], c["V"], c["vs"], c["q"], c["kn"], c["vn"]))


def c2_window(orc, synth):
    """C2's math at a small size: one query over the last 96 of 300 fp16 rows."""
    g = synth.SplitMix64(1)
    K = synth.f16_bits(g.normal(4 * 300 * 128)).reshape(4, 300, 128)
    V = synth.f16_bits(g.normal(4 * 300 * 128)).reshape(4, 300, 128)
    q = synth.f16_bits(g.normal(16 * 128)).reshape(16, 128)
    out = orc.decode_rows(synth.f16_val(q), synth.f16_val(K), synth.f16_val(V), np.arange(204, 300, dtype=np.int32))
    return dict(out=out.astype(np.float32), digest=digest(K, V, q))


def c5_sparse_selection(orc, synth, rows=None):
    """C5 sparse at full size (seed 4, p0 = 30720, T = 2048): for every row t, the SHA-256 of the
    1152 selected positions (u32, select_keys' order) over the index scores of its keys
    [0, p0 + t + 1 - 128). rows: only those rows (the others' digests stay empty), for a quick
    re-derivation."""
    p0, T = 30720, 2048
    c = synth.sparse_prefill_case(seed=4, p0=p0, T=T)
    out = np.zeros((T, 32), np.uint8)
    for t in range(T) if rows is None else rows:
        S = p0 + t + 1
        sc = orc.index_scores(c["qi"][t], c["w"][t], c["ki"][:S - 128])
        sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S).astype(np.uint32)
        out[t] = np.frombuffer(hashlib.sha256(sel.tobytes()).digest(), np.uint8)
    return dict(row_sha256=out, digest=digest(c["qi"], c["w"], c["ki"]))


FIXTURES = {"c1_decode": c1_decode, "c4_select_4k": c4_select, "quant_rows": quant_rows,
            "c5_prefill_small": c5_prefill, "c2_window_small": c2_window,
            "c5_sparse_selection": c5_sparse_selection}


def main():
    import orc
    from embla_attn import synth
    only = sys.argv[1:]
    for name, fn in FIXTURES.items():
        if only and name not in only:
            continue
        d = fn(orc, synth)
        np.savez_compressed(HERE / f"{name}.npz", **d)
        print(name, {k: (v.shape if hasattr(v, "shape") else v) for k, v in d.items()})


if __name__ == "__main__":
    main()
