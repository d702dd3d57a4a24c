"""ctypes wrapper of liborc.so, the C oracle. TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker, never by the product.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liborc.so"
LIB_OMP = HERE / "liborc_omp.so"
_lib = None
_path = LIB

P = np.ctypeslib.ndpointer


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def use_openmp(on: bool = True) -> None:
    """Switches this module to liborc_omp.so (the same source at -O3 -march=native with OpenMP
    threads; the same results), the build bench.py times as the CPU baseline."""
    global _lib, _path
    _path = LIB_OMP if on else LIB
    _lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not _path.exists():
            build()
        L = C.CDLL(str(_path))
        f32 = P(np.float32, flags="C")
        i8 = P(np.int8, flags="C")
        u16 = P(np.uint16, flags="C")
        u32 = P(np.uint32, flags="C")
        i32 = P(np.int32, flags="C")
        opt = C.c_void_p
        L.orc_head_norm.argtypes = [f32, opt, opt, C.c_int, C.c_int, f32]
        L.orc_rope.argtypes = [f32, C.c_int]
        L.orc_rope_freq.argtypes = [C.c_int]
        L.orc_rope_freq.restype = C.c_float
        L.orc_quant_row.argtypes = [f32, C.c_int, C.c_int, i8, P(np.float32)]
        L.orc_decode_int8.argtypes = [f32, i8, f32, i8, f32, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, opt, f32, opt]
        L.orc_decode_f32.argtypes = [f32, f32, f32, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, opt, f32, opt]
        L.orc_decode_rows.argtypes = [f32, f32, f32, C.c_int, C.c_int, C.c_int, i32, C.c_int,
                                      C.c_int, f32]
        L.orc_order_bits.argtypes = [C.c_float]
        L.orc_order_bits.restype = C.c_uint32
        L.orc_select_keys.argtypes = [f32, C.c_int, C.c_int, C.c_int, u32]
        L.orc_index_scores.argtypes = [u16, f32, u16, C.c_int, C.c_int, f32]
        L.orc_prefill_int8.argtypes = [f32, i8, f32, i8, f32, C.c_int, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, opt, C.c_int, f32]
        L.orc_q4_matvec.argtypes = [u32, u16, u16, u16, C.c_int, C.c_int, C.c_int, f32]
        L.orc_softcap.argtypes = [C.c_float]
        L.orc_softcap.restype = C.c_float
        L.orc_argmax.argtypes = [f32, C.c_int]
        L.orc_argmax.restype = C.c_uint32
        L.orc_mix32.argtypes = [C.c_uint32]
        L.orc_mix32.restype = C.c_uint32
        L.orc_sample.argtypes = [f32, C.c_int, C.c_int, C.c_float, C.c_float, C.c_uint32, P(np.int32)]
        L.orc_sample.restype = C.c_uint32
        L.orc_sample_many.argtypes = [f32, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_uint32, u32, i32]
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f32_to_bf16.restype = C.c_uint16
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def head_norm(x, g1=None, g2=None, ng=0, round_bf=True):
    x = _c(x, np.float32)
    out = np.empty(128, np.float32)
    g1 = None if g1 is None else _c(g1, np.float32)
    g2 = None if g2 is None else _c(g2, np.float32)
    lib().orc_head_norm(x, _ptr(g1), _ptr(g2), ng, int(round_bf), out)
    return out


def rope(x, pos):
    x = _c(x, np.float32).copy()
    lib().orc_rope(x, pos)
    return x


def quant_row(x, norm=False, round_bf=False):
    x = _c(x, np.float32)
    q = np.empty(128, np.int8)
    s = np.zeros(1, np.float32)
    lib().orc_quant_row(x, int(norm), int(round_bf), q, s)
    return q, float(s[0])


def decode_int8(q, K, ks, V, vs, weights=0, rows=None, n_sel=None, want_scores=False):
    """q [n_q][128] f32; K, V int8 [n_kv][S_cache][128]; ks, vs f32 [n_kv][S_cache]."""
    q = _c(q, np.float32)
    K = _c(K, np.int8)
    V = _c(V, np.int8)
    ks = _c(ks, np.float32)
    vs = _c(vs, np.float32)
    n_q = q.shape[0]
    n_kv, S_cache, _ = K.shape
    S = S_cache if rows is None else n_sel
    rows_c = None if rows is None else _c(rows, np.uint32)
    out = np.empty((n_q, 128), np.float32)
    scores = np.empty((n_kv, S_cache), np.float32) if want_scores else None
    lib().orc_decode_int8(q, K, ks, V, vs, S, S_cache, n_q, n_kv, weights, _ptr(rows_c), out, _ptr(scores))
    return (out, scores) if want_scores else out


def decode_f32(q, K, V, S=None, weights=0, rows=None, want_scores=False):
    """q [n_q][128]; K, V [n_kv][S_cache][128] fp32 values of bf16 rows; rows u32 [n_kv][S]."""
    q = _c(q, np.float32)
    K = _c(K, np.float32)
    V = _c(V, np.float32)
    n_q = q.shape[0]
    n_kv, S_cache, _ = K.shape
    rows_c = None if rows is None else _c(rows, np.uint32)
    if S is None:
        S = rows_c.shape[-1] if rows_c is not None else S_cache
    out = np.empty((n_q, 128), np.float32)
    scores = np.empty((n_kv, S_cache), np.float32) if want_scores else None
    lib().orc_decode_f32(q, K, V, S, S_cache, n_q, n_kv, weights, _ptr(rows_c), out, _ptr(scores))
    return (out, scores) if want_scores else out


def decode_rows(q, K, V, pos_list, per_head=False):
    q = _c(q, np.float32)
    K = _c(K, np.float32)
    V = _c(V, np.float32)
    pl = _c(pos_list, np.int32)
    n_q = q.shape[0]
    n_kv, S_cache, _ = K.shape
    n = pl.shape[-1]
    out = np.empty((n_q, 128), np.float32)
    lib().orc_decode_rows(q, K, V, S_cache, n_q, n_kv, pl, n, int(per_head), out)
    return out


def order_bits(f):
    return int(lib().orc_order_bits(float(f)))


def select_keys(scores, S, topk=1024, recent=128):
    sc = _c(scores, np.float32)
    out = np.empty(topk + recent, np.uint32)
    lib().orc_select_keys(sc, S, topk, recent, out)
    return out


def index_scores(qi_bits, w, ki_bits):
    """qi fp16 bits [n_ih][64], w f32 [n_ih], ki fp16 bits [n][64] -> f32 [n]."""
    qi = _c(qi_bits, np.uint16)
    ki = _c(ki_bits, np.uint16)
    w = _c(w, np.float32)
    n = ki.shape[0]
    out = np.empty(n, np.float32)
    lib().orc_index_scores(qi, w, ki, n, qi.shape[0], out)
    return out


def prefill_int8(q, K, ks, V, vs, p0, weights=0, window=0, rows_sel=None):
    """q [T][n_q][128] f32; K, V int8 [n_kv][S_cache][128]; ks, vs f32 [n_kv][S_cache]."""
    q = _c(q, np.float32)
    K = _c(K, np.int8)
    V = _c(V, np.int8)
    ks = _c(ks, np.float32)
    vs = _c(vs, np.float32)
    T, n_q, _ = q.shape
    n_kv, S_cache, _ = K.shape
    rs = None if rows_sel is None else _c(rows_sel, np.uint32)
    nsel = 0 if rs is None else rs.shape[1]
    out = np.empty((T, n_q, 128), np.float32)
    lib().orc_prefill_int8(q, K, ks, V, vs, T, p0, S_cache, n_q, n_kv, weights, window, _ptr(rs), nsel, out)
    return out


def q4_matvec(w, s, b, x, epi=4, y=None):
    """y = W x for W in MLX's 4-bit affine layout: w uint32 [O][K/8], s, b bf16 bits [O][K/64],
    x bf16 bits [K]; epilogue epi (2 accumulates into y)."""
    w = _c(w, np.uint32)
    O, K = w.shape[0], w.shape[1] * 8
    out = np.zeros(O, np.float32) if y is None else np.ascontiguousarray(y, np.float32).copy()
    lib().orc_q4_matvec(w.reshape(-1), _c(s, np.uint16).reshape(-1), _c(b, np.uint16).reshape(-1),
                        _c(x, np.uint16).reshape(-1), O, K, epi, out)
    return out


def softcap(logits):
    """bf(bf(tanh(bf(bf(l) / 15))) * 15) of each logit (misc.metal:101)."""
    f = lib().orc_softcap
    return np.array([f(float(v)) for v in np.asarray(logits, np.float32).reshape(-1)], np.float32)


def argmax(logits) -> int:
    """The greedy token: first index of the largest softcapped logit (misc.metal:86-128)."""
    lg = _c(logits, np.float32).reshape(-1)
    return int(lib().orc_argmax(lg, lg.size))


def sample(logits, pos, inv_t, top_p, seed):
    """The top-p Gumbel draw of misc.metal:196-298 -> (token, fragile)."""
    lg = _c(logits, np.float32).reshape(-1)
    fr = np.zeros(1, np.int32)
    tok = lib().orc_sample(lg, lg.size, pos, inv_t, top_p, seed & 0xFFFFFFFF, fr)
    return int(tok), bool(fr[0])


def sample_many(logits, pos0, n, inv_t, top_p, seed):
    """Draws at positions pos0 .. pos0 + n - 1 -> (tokens, fragile flags)."""
    lg = _c(logits, np.float32).reshape(-1)
    tok = np.zeros(n, np.uint32)
    fr = np.zeros(n, np.int32)
    lib().orc_sample_many(lg, lg.size, pos0, n, inv_t, top_p, seed & 0xFFFFFFFF, tok, fr)
    return tok, fr.astype(bool)
