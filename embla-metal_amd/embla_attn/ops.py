"""Torch-facing wrappers over the C ABI: device tensors in, device tensors out, launched on the
current torch stream. Torch supplies device memory and the stream; every computation is the HIP
library's.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch

from . import _lib
from ._lib import BF16, F16, F32, RELU2_SINK, SOFTMAX, call, lib

_DT = {F16: torch.float16, BF16: torch.bfloat16}


_PROBE = None


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def stream_handle(stream=None) -> C.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class Workspace:
    """Split-K partials and counters for decode calls up to max_s keys and n_q heads."""

    def __init__(self, max_s: int, n_q: int = 16, device="cuda"):
        self.nbytes = int(lib().embla_workspace_bytes(max_s, n_q))
        if self.nbytes == 0:
            raise ValueError("invalid workspace shape")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        call("embla_workspace_init", _p(self.buf), self.nbytes, stream_handle())

    @property
    def ptr(self):
        return _p(self.buf)


def decode_int8(q, kc, vc, S, max_s, n_kv, weights=SOFTMAX, scale_dtype=F16, out_dtype=F16,
                chunk=0, ws: Workspace | None = None, scores=None, out=None, stream=None):
    """Split-K decode of fp16 q [n_q][128] over an int8 layer cache (K region kc, V region vc)."""
    n_q = q.shape[0]
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[out_dtype], device=q.device)
    call("embla_decode_int8", _p(q), _p(kc), _p(vc), _p(out), _p(scores), S, max_s, n_q, n_kv,
         weights, scale_dtype, out_dtype, chunk, ws.ptr if ws else None, ws.nbytes if ws else 0,
         stream_handle(stream))
    return out


def decode_int8_noalloc(q, kc, vc, S, max_s, n_kv, weights=SOFTMAX, scale_dtype=F16, out_dtype=F16, chunk=0,
                        scores=None, out=None, stream=None):
    """decode_int8 with its partials in the library's own device array (no workspace argument)."""
    n_q = q.shape[0]
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[out_dtype], device=q.device)
    call("embla_decode_int8_noalloc", _p(q), _p(kc), _p(vc), _p(out), _p(scores), S, max_s, n_q, n_kv,
         weights, scale_dtype, out_dtype, chunk, stream_handle(stream))
    return out


def decode_int8_partials(q, kc, vc, S, max_s, n_kv, ws: Workspace, weights=SOFTMAX, scale_dtype=F16, out_dtype=F16,
                         chunk=0, scores=None, stream=None):
    """The split-K kernel of decode_int8 alone: chunk partials left in ws."""
    call("embla_decode_int8_partials", _p(q), _p(kc), _p(vc), _p(scores), S, max_s, q.shape[0], n_kv, weights,
         scale_dtype, out_dtype, chunk, ws.ptr, ws.nbytes, stream_handle(stream))


def decode_int8_merge(out, S, max_s, n_kv, ws: Workspace, weights=SOFTMAX, out_dtype=F16, chunk=0, stream=None):
    """The merge of decode_int8_partials' chunk partials into out [n_q][128]."""
    call("embla_decode_int8_merge", _p(out), S, max_s, out.shape[0], n_kv, weights, out_dtype, chunk, ws.ptr,
         ws.nbytes, stream_handle(stream))
    return out


def _probe():
    """The bench-only probe library (libembla_probe.so), loaded once."""
    global _PROBE
    if _PROBE is None:
        path = Path(__file__).resolve().parent / "libembla_probe.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built (embla_attn.build.build())")
        _PROBE = C.CDLL(str(path))
        _PROBE.embla_probe_stream_read.restype = C.c_int
        _PROBE.embla_probe_stream_read.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                                   C.c_void_p]
        _PROBE.embla_probe_mfma_rate.restype = C.c_int
        _PROBE.embla_probe_mfma_rate.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    return _PROBE


def stream_read(buf, sink, grid=1024, depth=4, mode=0, stream=None):
    """One streaming read of buf by the bench-only probe library; sink: int32 [grid]; depth 16-byte
    loads in flight a thread (4, 8, 16, 32); mode 0: into registers, grid-strided; 1: into LDS;
    2: into registers, a contiguous slice a workgroup."""
    rc = _probe().embla_probe_stream_read(_p(buf), buf.numel() * buf.element_size(), _p(sink), grid, depth,
                                          int(mode), stream_handle(stream))
    if rc != 0:
        raise RuntimeError(f"embla_probe_stream_read failed ({rc})")


def mfma_rate(grid, iters, sink, stream=None):
    """The bench-only MFMA rate probe: grid workgroups of 4 waves, each wave 4 independent chains
    of iters v_mfma_f32_32x32x16_f16 (32768 flop each); sink float [grid * 4]."""
    rc = _probe().embla_probe_mfma_rate(grid, iters, _p(sink), stream_handle(stream))
    if rc != 0:
        raise RuntimeError(f"embla_probe_mfma_rate failed ({rc})")



def decode_step_int8(qkv, q_off, k_off, v_off, kc, vc, pos, max_s, n_q, n_kv, ws: Workspace, g1=None, g2=None,
                     ng=0, scale_dtype=F16, norm_k=False, out_dtype=BF16, chunk=0, out=None, stream=None):
    """A full layer's decode step with its own append: the new k, v of qkv quantised into the cache
    at pos, the softmax decode over keys 0 .. pos; q raw bf16, head-normed inside."""
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[out_dtype], device=qkv.device)
    call("embla_decode_step_int8", _p(qkv), q_off, k_off, v_off, _p(g1), _p(g2), ng, _p(kc), _p(vc), _p(out), pos,
         max_s, n_q, n_kv, scale_dtype, int(norm_k), out_dtype, chunk, ws.ptr, ws.nbytes, stream_handle(stream))
    return out


def decode_int8_qraw(qraw, kc, vc, S, max_s, n_kv, g1=None, g2=None, ng=0, scale_dtype=F16, out_dtype=BF16,
                     chunk=0, ws: Workspace | None = None, out=None, stream=None):
    """Split-K decode (softmax) of raw bf16 q [n_q][128], head-normed inside the kernel."""
    n_q = qraw.numel() // 128
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[out_dtype], device=qraw.device)
    call("embla_decode_int8_qraw", _p(qraw), _p(g1), _p(g2), ng, _p(kc), _p(vc), _p(out), S, max_s, n_q, n_kv,
         scale_dtype, out_dtype, chunk, ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


def kv_quant_append(k, v, T, p0, n_kv, kc, vc, max_s, in_dtype=BF16, scale_dtype=F16, norm_k=False,
                    stride=None, stream=None):
    stride = stride if stride is not None else n_kv * 128
    call("embla_kv_quant_append", _p(k), _p(v), in_dtype, stride, T, p0, n_kv, _p(kc), _p(vc), max_s,
         scale_dtype, int(norm_k), stream_handle(stream))


def q_prep(qraw, g1, g2, ng, T, n_q, out_dtype=F16, stride=None, out=None, stream=None):
    stride = stride if stride is not None else n_q * 128
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=_DT[out_dtype], device=qraw.device)
    call("embla_q_prep", _p(qraw), _p(g1), _p(g2), ng, stride, T, n_q, _p(out), out_dtype,
         stream_handle(stream))
    return out


def attn_full8(qraw, g1, g2, kc, vc, part, scores, counter, o, S, maxS, ng=2, CH=0, stream=None):
    """Reference-signature full layer (attention.metal:235-363)."""
    p = _lib.AttnParams(S, CH, 0, maxS, S - 1, ng, 0, 0)
    call("embla_attn_full8", _p(qraw), _p(g1), _p(g2), _p(kc), _p(vc), _p(part), _p(scores),
         _p(counter), _p(o), C.byref(p), stream_handle(stream))


def attn_sparse8(qraw, g1, g2, kc, vc, part, idx, counter, o, S, maxS, ng=2, CH=0, stream=None):
    """Reference-signature sparse layer (attention.metal:448-584): idx None = every key 0 .. S-1."""
    p = _lib.AttnParams(S, CH, 0, maxS, S - 1, ng, 0, 0)
    call("embla_attn_sparse8", _p(qraw), _p(g1), _p(g2), _p(kc), _p(vc), _p(part), _p(idx),
         _p(counter), _p(o), C.byref(p), stream_handle(stream))


def attn_full(qraw, g1, g2, kc, vc, part, scores, counter, o, S, maxS, ng=2, CH=0, stream=None):
    """attn_full without KV8 (attention.metal:148-220): bf16 caches in the 16-bit tile layout."""
    p = _lib.AttnParams(S, CH, 0, maxS, S - 1, ng, 0, 0)
    call("embla_attn_full", _p(qraw), _p(g1), _p(g2), _p(kc), _p(vc), _p(part), _p(scores),
         _p(counter), _p(o), C.byref(p), stream_handle(stream))


def attn_sparse(qraw, g1, g2, kc, vc, part, idx, counter, o, S, maxS, ng=2, CH=0, stream=None):
    """attn_sparse without KV8 (attention.metal:370-441): idx None = every key 0 .. S-1."""
    p = _lib.AttnParams(S, CH, 0, maxS, S - 1, ng, 0, 0)
    call("embla_attn_sparse", _p(qraw), _p(g1), _p(g2), _p(kc), _p(vc), _p(part), _p(idx),
         _p(counter), _p(o), C.byref(p), stream_handle(stream))


def kv_append_bf16(qkv, cache, jobs, pm_pos, maxS, T=1, stream=None):
    """kv_append(_b) without KV8: jobs a list of (k, v, kc, vc) element offsets."""
    arr = (_lib.KVJob * len(jobs))(*[_lib.KVJob(*j) for j in jobs])
    call("embla_kv_append_bf16", _p(qkv), _p(cache), arr, len(jobs), pm_pos, maxS, T, stream_handle(stream))


def attn_full_b(qkv, g1, g2, kc, vc, part, counter, o, p0, T, maxS, stream=None):
    """attn_full_b (prefill.metal:214-282) over bf16 caches; o bf16 [T][2048]."""
    p = _lib.AttnB(p0, 0, 0, maxS)
    call("embla_attn_full_b", _p(qkv), _p(g1), _p(g2), _p(kc), _p(vc), _p(part), _p(counter), _p(o),
         C.byref(p), T, stream_handle(stream))


def sliding_decode(q, k_new, v_new, kring, vring, pos, window, ring, n_kv, dtype=F16, chunk=0,
                   ws: Workspace | None = None, out=None, stream=None):
    """One decode step over a 16-bit ring: appends (k_new, v_new) at pos, attends the window."""
    n_q = q.shape[0]
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[dtype], device=q.device)
    call("embla_sliding_decode", _p(q), _p(k_new), _p(v_new), _p(kring), _p(vring), _p(out), pos, window, ring,
         n_q, n_kv, dtype, chunk, ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


def attn_sliding(qkv, qg, kg, kc, vc, o, pos, stream=None):
    """Reference-signature sliding layer (attention.metal:26-102)."""
    call("embla_attn_sliding", _p(qkv), _p(qg), _p(kg), _p(kc), _p(vc), _p(o), pos, stream_handle(stream))


def index_scores(qi, w, ki, n, stream=None):
    scores = torch.empty(n, dtype=torch.float32, device=qi.device)
    call("embla_index_scores", _p(qi), _p(w), _p(ki), _p(scores), n, qi.shape[0], stream_handle(stream))
    return scores


def select_topk(scores, S, n_sets=1, topk=1024, recent=128, score_stride=0, stream=None):
    idx = torch.empty((n_sets, topk + recent), dtype=torch.int32, device=scores.device)
    call("embla_select_topk", _p(scores), score_stride, _p(idx), topk + recent, S, n_sets, topk, recent,
         stream_handle(stream))
    return idx


def select_keys(scores, S, maxS, stream=None):
    """Reference-signature select_keys: 2 sets of [maxS] scores -> idx [2][1152]."""
    idx = torch.empty((2, 1152), dtype=torch.int32, device=scores.device)
    call("embla_select_keys", _p(scores), _p(idx), S, maxS, stream_handle(stream))
    return idx


def sparse_decode(q, kc, vc, idx, nsel, max_s, n_kv, idx_stride=0, dtype=F16, chunk=0, ws=None, out=None,
                  stream=None):
    n_q = q.shape[0]
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[dtype], device=q.device)
    call("embla_sparse_decode", _p(q), _p(kc), _p(vc), _p(idx), idx_stride, nsel, _p(out), max_s, n_q, n_kv, dtype,
         chunk, ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


class SparseWorkspace:
    def __init__(self, max_s: int, n_q: int = 16, device="cuda"):
        self.max_s, self.n_q = max_s, n_q
        self.nbytes = int(lib().embla_sparse_workspace_bytes(max_s, n_q))
        self.buf = torch.zeros(self.nbytes, dtype=torch.uint8, device=device)
        self.recount_off = int(lib().embla_sparse_workspace_recount_offset(max_s, n_q))

    @property
    def ptr(self):
        return _p(self.buf)

    def audit(self, stream=None) -> int:
        """embla_sparse_workspace_audit: EMBLA_ERR_WORKSPACE (-4) if a call since the last audit found
        the workspace not clean, else 0; clears the count."""
        return int(lib().embla_sparse_workspace_audit(self.ptr, self.nbytes, self.max_s, self.n_q, stream_handle(stream)))

    def recounts(self) -> int:
        """Calls that found the select's histogram buffer not clean and recounted it (a device word
        of the workspace; reading it synchronises)."""
        return int(self.buf[self.recount_off:self.recount_off + 4].view(torch.int32).item())

    def selection(self):
        """The last sparse_layer_decode call's selected rows (top 1024 + latest 128), int32 [1152]:
        the workspace region after the scores (embla_sparse_layer_decode's layout)."""
        off = (self.max_s * 4 + 255) // 256 * 256
        return self.buf[off:off + 1152 * 4].view(torch.int32)


def sparse_layer_decode(q, qi, w, ki, kc, vc, S, max_s, n_kv, ws: SparseWorkspace, dtype=F16, out=None,
                        stream=None):
    n_q = q.shape[0]
    if out is None:
        out = torch.empty((n_q, 128), dtype=_DT[dtype], device=q.device)
    call("embla_sparse_layer_decode", _p(q), _p(qi), _p(w), _p(ki), _p(kc), _p(vc), _p(out), S, max_s, n_q, n_kv,
         qi.shape[0], dtype, ws.ptr, ws.nbytes, stream_handle(stream))
    return out


class PrefillWorkspace:
    def __init__(self, T: int, n_q: int = 16, device="cuda", staged_p0=None, n_kv: int = 4):
        """staged_p0: also room for the staged fp16 copy of keys 0 .. staged_p0 + T - 1."""
        if staged_p0 is None:
            self.nbytes = int(lib().embla_prefill_workspace_bytes(T, n_q))
        else:
            self.nbytes = int(lib().embla_prefill_staged_workspace_bytes(T, staged_p0, n_q, n_kv))
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)

    @property
    def ptr(self):
        return _p(self.buf)


def prefill_int8(q, kc, vc, T, p0, max_s, n_kv, weights=SOFTMAX, scale_dtype=F16, window=0, q_dtype=BF16,
                 out_dtype=BF16, q_strides=None, out=None, out_strides=None, ws=None, stream=None):
    """Prefill attention of T query rows over an int8 layer cache holding keys 0 .. p0 + T - 1."""
    n_q = q.shape[1] if q_strides is None else q.shape[0]
    qs = q_strides or (n_q * 128, 128)
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=_DT[out_dtype], device=q.device)
    os_ = out_strides or (n_q * 128, 128)
    call("embla_prefill_int8", _p(q), q_dtype, qs[0], qs[1], _p(kc), _p(vc), _p(out), out_dtype, os_[0], os_[1], T, p0,
         max_s, n_q, n_kv, weights, scale_dtype, window, ws.ptr if ws else None, ws.nbytes if ws else 0,
         stream_handle(stream))
    return out


def prefill_full(q, k, v, kc, vc, T, p0, max_s, n_kv, out=None, ws=None, stream=None):
    n_q = q.shape[1]
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=torch.bfloat16, device=q.device)
    call("embla_prefill_full", _p(q), _p(k), _p(v), _p(kc), _p(vc), _p(out), T, p0, max_s, n_q, n_kv,
         ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


def q_prep_b(qkv, g1, g2, T, out=None, stream=None):
    """Reference-signature q_prep_b: qkv [T][4096] bf16 -> qn [16][T][128] bf16, head-major."""
    if out is None:
        out = torch.empty((16, T, 128), dtype=torch.bfloat16, device=qkv.device)
    call("embla_q_prep_b", _p(qkv), _p(g1), _p(g2), _p(out), T, stream_handle(stream))
    return out


def relu2_prefill(qn, kc, vc, Tq, Tk, maxS, out=None, stream=None):
    """Reference-signature relu2_prefill_nax: qn [16][Tq][128] bf16 -> out [Tq][2048] bf16."""
    if out is None:
        out = torch.empty((Tq, 2048), dtype=torch.bfloat16, device=qn.device)
    call("embla_relu2_prefill", _p(qn), _p(kc), _p(vc), _p(out), Tq, Tk, maxS, stream_handle(stream))
    return out


def ring_append(k, v, T, p0, n_kv, kring, vring, ring, dtype=BF16, kg=None, stride=None, stream=None):
    stride = stride if stride is not None else n_kv * 128
    call("embla_ring_append", _p(k), _p(v), dtype, stride, T, p0, n_kv, _p(kring), _p(vring), ring, _p(kg),
         stream_handle(stream))


def prefill_sliding(q, k, v, kring, vring, T, p0, ring, window, n_kv, out=None, ws=None, stream=None):
    n_q = q.shape[1]
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=torch.bfloat16, device=q.device)
    call("embla_prefill_sliding", _p(q), _p(k), _p(v), _p(kring), _p(vring), _p(out), T, p0, ring, window, n_q, n_kv,
         ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


def attn_sliding8_b(qkv, qg, kg, kc, vc, p0, T, out=None, stream=None):
    """Reference-signature kv_sliding_b + attn_sliding8_b: qkv [T][4096] bf16 -> o [T][2048] bf16."""
    if out is None:
        out = torch.empty((T, 2048), dtype=torch.bfloat16, device=qkv.device)
    call("embla_attn_sliding8_b", _p(qkv), _p(qg), _p(kg), _p(kc), _p(vc), _p(out), p0, T, stream_handle(stream))
    return out


def prefill_ring(q, kring, vring, T, p0, ring, window, n_kv, dtype=BF16, qg=None, out=None, ws=None, stream=None):
    """Windowed prefill over a 16-bit ring already holding the chunk; q [T][n_q][128]."""
    n_q = q.shape[1]
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=q.dtype, device=q.device)
    call("embla_prefill_ring", _p(q), dtype, n_q * 128, 128, _p(kring), _p(vring), ring, _p(out), n_q * 128, 128, T,
         p0, n_q, n_kv, window, _p(qg), ws.ptr if ws else None, ws.nbytes if ws else 0, stream_handle(stream))
    return out


class SparsePrefillWorkspace:
    def __init__(self, T: int, p0: int, device="cuda"):
        self.nbytes = int(lib().embla_sparse_prefill_workspace_bytes(T, p0))
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)

    @property
    def ptr(self):
        return _p(self.buf)


def prefill_sparse(q, k, v, qi, w, ki, kc, vc, T, p0, max_s, n_kv, ws, out=None, idx=None, stream=None):
    """Sparse-layer prefill chunk: append k, v (row-major int8 cache), per-row top-1024 + latest 128
    by the index score, attention. Returns (o [T][n_q][128] bf16, idx [T][1152] int32 or None)."""
    n_q = q.shape[1]
    if out is None:
        out = torch.empty((T, n_q, 128), dtype=torch.bfloat16, device=q.device)
    call("embla_prefill_sparse", _p(q), _p(k), _p(v), _p(qi), _p(w), _p(ki), _p(kc), _p(vc), _p(out), _p(idx), T, p0,
         max_s, n_q, n_kv, ws.ptr, ws.nbytes, stream_handle(stream))
    return out, idx


def kv_block_copy(cache, regions, p0, max_s, n_kv, stored, save, scale_dtype=F16, stream=None):
    """Prefix-cache block of full layers: positions p0 .. p0+127 of each layer's K and V region
    (byte offsets `regions` [[k, v], ...] in `cache`) to `stored` (save) or back."""
    import ctypes as C
    flat = [int(x) for kv in regions for x in kv]
    arr = (C.c_ulonglong * len(flat))(*flat)
    call("embla_kv_block_copy", _p(cache), C.cast(arr, C.c_void_p), len(regions), p0, max_s, n_kv, scale_dtype,
         _p(stored), 1 if save else 0, stream_handle(stream))


def ring_block_copy(cache, regions, p0, ring, n_kv, stored, save, stream=None):
    """Sliding-layer checkpoint: ring slots p0 % ring .. +127 of each layer's K and V ring."""
    import ctypes as C
    flat = [int(x) for kv in regions for x in kv]
    arr = (C.c_ulonglong * len(flat))(*flat)
    call("embla_ring_block_copy", _p(cache), C.cast(arr, C.c_void_p), len(regions), p0, ring, n_kv, _p(stored),
         1 if save else 0, stream_handle(stream))


class EmblaSeg(C.Structure):
    """A stacked segment of embla_gemv_q4 (gemv.metal's Seg)."""
    _fields_ = [("w", C.c_ulonglong), ("s", C.c_ulonglong), ("b", C.c_ulonglong), ("end", C.c_uint),
                ("x", C.c_uint), ("y", C.c_uint), ("pad", C.c_uint)]


EPI_BF16, EPI_RELU2, EPI_ADD, EPI_F32_BF, EPI_F32 = range(5)


def gemv_q4(W, X, Y, segs, K, epi, stream=None):
    """y = W x over stacked 4-bit segments: W a uint8 buffer, X bf16, Y bf16 (epi 0, 1) or fp32;
    segs: (w, s, b, end, x, y) tuples of byte offsets in W, end row, element offsets in X and Y."""
    arr = (EmblaSeg * len(segs))(*[EmblaSeg(*g, 0) for g in segs])
    call("embla_gemv_q4", _p(W), _p(X), _p(Y), C.cast(arr, C.c_void_p), len(segs), K, epi, stream_handle(stream))
    return Y


def gemm_q4(W, wo, X, Y, T, O, K, epi, ldx=None, ldy=None, stream=None):
    """Y = X W^T for T tokens: W a uint8 buffer with the words, scales and biases at byte offsets
    wo = (w, s, b); X bf16 [T][ldx]; Y [T][ldy] bf16 (epi 0, 1) or fp32."""
    arr = (C.c_ulonglong * 3)(*[int(v) for v in wo])
    call("embla_gemm_q4", _p(W), C.cast(arr, C.c_void_p), _p(X), _p(Y), T, O, K, ldx or K, ldy or O, epi,
         stream_handle(stream))
    return Y


class SampleState:
    """The sampling tail's buffers for vocabularies up to V tokens (Engine.swift:261-267): the token
    ids by position, the greedy words (word 0 the polled word, then one a position) and the
    workspace."""

    def __init__(self, V: int, max_pos: int, device="cuda"):
        self.V = V
        self.ws_bytes = int(lib().embla_sample_workspace_bytes(V))
        if self.ws_bytes == 0:
            raise ValueError("vocabulary outside 1 .. 65536")
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)
        self.tokens = torch.zeros(max_pos + 2, dtype=torch.int32, device=device)
        self.greedy = torch.zeros(max_pos + 3, dtype=torch.int32, device=device)

    def _args(self, pos, prompt_len):
        if not 0 <= pos <= self.tokens.numel() - 2:
            raise ValueError("position outside the buffers")
        return _p(self.tokens), self.V, self.greedy.data_ptr() + 4, pos, prompt_len


def argmax(logits, st: SampleState, pos: int, prompt_len: int = 0, stream=None):
    """The greedy token of fp32 logits [V] at position pos (misc.metal:86-128)."""
    tok, V, g, pos, pl = st._args(pos, prompt_len)
    call("embla_argmax", _p(logits), tok, V, g, pos, pl, _p(st.ws), st.ws_bytes, stream_handle(stream))


def sample(logits, st: SampleState, pos: int, inv_t: float, top_p: float, seed: int, prompt_len: int = 0,
           stream=None):
    """The top-p Gumbel draw at position pos (misc.metal:196-298)."""
    tok, V, g, pos, pl = st._args(pos, prompt_len)
    call("embla_sample", _p(logits), tok, V, g, pos, pl, inv_t, top_p, seed & 0xFFFFFFFF, _p(st.ws), st.ws_bytes,
         stream_handle(stream))
