"""Seeded synthetic inputs of the benchmark configurations (SplitMix64, as the reference's tests
seed their fixtures: Tests/EmblaMetalTests/GEMV4Tests.swift:35-46).

Draws, in a fixed order per configuration:
  uniform  u = (z >> 11) * 2^-53
  normal   Box-Muller on consecutive uniform pairs (u1, u2): sqrt(-2 ln(1 - u1)) cos(2π u2), in
           fp64, then rounded (RNE) to fp16 or bf16
  int8     (z mod 255) - 127, in [-127, 127]
"""
from __future__ import annotations

import numpy as np

GOLD = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


class SplitMix64:
    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            z = self.state + np.arange(1, n + 1, dtype=np.uint64) * GOLD
            self.state = self.state + np.uint64(n) * GOLD
            z = (z ^ (z >> np.uint64(30))) * M1
            z = (z ^ (z >> np.uint64(27))) * M2
            return z ^ (z >> np.uint64(31))

    def uniform(self, n: int) -> np.ndarray:
        return (self.next(n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)

    def normal(self, n: int) -> np.ndarray:
        u = self.uniform(2 * n)
        u1, u2 = u[0::2], u[1::2]
        return np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)

    def int8(self, n: int) -> np.ndarray:
        return ((self.next(n) % np.uint64(255)).astype(np.int16) - 127).astype(np.int8)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """fp64/fp32 -> fp16 bits (RNE, via numpy's IEEE conversion)."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).view(np.uint16)


def f16_val(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """-> bf16 bits, RNE from the fp32 value (BFloat16.swift:4-9)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)) >> np.uint64(16)
    return r.astype(np.uint16)


def bf16_val(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def decode_int8_case(seed: int, S: int, n_q: int = 16, n_kv: int = 4, lo: float = 0.005,
                     hi: float = 0.02) -> dict:
    """Configs 1 and 3: q fp16 N(0,1); K, V int8 U{-127..127}; fp16 scales U[lo, hi].
    Draw order: q, K, K scales, V, V scales."""
    g = SplitMix64(seed)
    q = f16_bits(g.normal(n_q * 128)).reshape(n_q, 128)
    K = g.int8(n_kv * S * 128).reshape(n_kv, S, 128)
    ks = f16_bits(lo + (hi - lo) * g.uniform(n_kv * S)).reshape(n_kv, S)
    V = g.int8(n_kv * S * 128).reshape(n_kv, S, 128)
    vs = f16_bits(lo + (hi - lo) * g.uniform(n_kv * S)).reshape(n_kv, S)
    return dict(q=q, K=K, ks=ks, V=V, vs=vs, S=S, n_q=n_q, n_kv=n_kv)


def sparse_case(seed: int, ctx: int, n_q: int = 16, n_kv: int = 4, n_ih: int = 4) -> dict:
    """Config C4: index heads qi fp16 [n_ih][64] N(0,1), weights w U(0,1) fp32 [n_ih], index keys
    ki fp16 [ctx][64] N(0,1), q fp16 [n_q][128] N(0,1), K, V fp16 [n_kv][ctx][128] N(0,1).
    Draw order: qi, w, ki, q, K, V."""
    g = SplitMix64(seed)
    qi = f16_bits(g.normal(n_ih * 64)).reshape(n_ih, 64)
    w = g.uniform(n_ih).astype(np.float32)
    ki = f16_bits(g.normal(ctx * 64)).reshape(ctx, 64)
    q = f16_bits(g.normal(n_q * 128)).reshape(n_q, 128)
    K = f16_bits(g.normal(n_kv * ctx * 128)).reshape(n_kv, ctx, 128)
    V = f16_bits(g.normal(n_kv * ctx * 128)).reshape(n_kv, ctx, 128)
    return dict(qi=qi, w=w, ki=ki, q=q, K=K, V=V, S=ctx, n_q=n_q, n_kv=n_kv)


def prefill_case(seed: int, p0: int, T: int, n_q: int = 16, n_kv: int = 4, lo: float = 0.005,
                 hi: float = 0.02) -> dict:
    """Config C5: an int8 prefix of p0 positions (K, V int8 U{-127..127}, fp16 scales U[lo, hi],
    as C3) and a chunk of T tokens: bf16 Q [T][n_q][128], K, V [T][n_kv][128] drawn from N(0,1).
    Draw order: prefix K, K scales, V, V scales, then Q, K, V of the chunk."""
    g = SplitMix64(seed)
    K = g.int8(n_kv * p0 * 128).reshape(n_kv, p0, 128)
    ks = f16_bits(lo + (hi - lo) * g.uniform(n_kv * p0)).reshape(n_kv, p0)
    V = g.int8(n_kv * p0 * 128).reshape(n_kv, p0, 128)
    vs = f16_bits(lo + (hi - lo) * g.uniform(n_kv * p0)).reshape(n_kv, p0)
    q = bf16_bits(g.normal(T * n_q * 128).astype(np.float32)).reshape(T, n_q, 128)
    kn = bf16_bits(g.normal(T * n_kv * 128).astype(np.float32)).reshape(T, n_kv, 128)
    vn = bf16_bits(g.normal(T * n_kv * 128).astype(np.float32)).reshape(T, n_kv, 128)
    return dict(K=K, ks=ks, V=V, vs=vs, q=q, kn=kn, vn=vn, p0=p0, T=T, n_q=n_q, n_kv=n_kv)


def sparse_prefill_case(seed: int, p0: int, T: int, n_q: int = 16, n_kv: int = 4, n_ih: int = 4) -> dict:
    """Config C5's sparse layer: prefill_case's cache prefix and chunk, then the indexer: fp16
    index queries [T][n_ih][64] and keys [p0 + T][64] drawn from N(0,1), weights [T][n_ih] from
    U(0,1). Draw order: prefill_case's, then qi, w, ki."""
    c = prefill_case(seed, p0, T, n_q, n_kv)
    g = SplitMix64(seed + 1000)
    c["qi"] = f16_bits(g.normal(T * n_ih * 64)).reshape(T, n_ih, 64)
    c["w"] = g.uniform(T * n_ih).astype(np.float32).reshape(T, n_ih)
    c["ki"] = f16_bits(g.normal((p0 + T) * 64)).reshape(p0 + T, 64)
    return c


def q4_weights(g: "SplitMix64", O: int, K: int) -> tuple:
    """A 4-bit matrix in MLX's affine layout: words uint32 [O][K/8] of uniform nibbles, bf16
    scales U[0.005, 0.015] and biases -7.5 scale (weights centred on 0) [O][K/64], as bits."""
    words = (g.uniform(O * K // 8) * 2 ** 32).astype(np.uint64).astype(np.uint32).reshape(O, K // 8)
    sc = 0.005 + 0.01 * g.uniform(O * K // 64)
    s = bf16_bits(sc.astype(np.float32)).reshape(O, K // 64)
    b = bf16_bits((-7.5 * bf16_val(s).reshape(-1)).astype(np.float32)).reshape(O, K // 64)
    return words, s, b
