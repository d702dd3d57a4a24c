"""The C ABI library loads, exports every entry point include/embla_attn.h declares, and rejects
invalid arguments on the host (no GPU needed: validation precedes any HIP call)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from embla_attn import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "embla_attn.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(embla_\w+)\s*\(", text)))


def test_header_symbols_exported():
    L = _lib.lib()
    names = declared()
    assert len(names) >= 8
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_workspace():
    L = _lib.lib()
    assert L.embla_version() >= 1
    assert L.embla_workspace_bytes(32768, 16) > 1024 * 16 * 130 * 4
    assert L.embla_workspace_bytes(0, 16) == 0


@pytest.mark.parametrize("S,max_s,n_q,n_kv", [(0, 1024, 16, 4), (2000, 1024, 16, 4), (10, 1000, 16, 4),
                                                (10, 1024, 16, 3)])
def test_decode_rejects_bad_shapes(S, max_s, n_q, n_kv):
    L = _lib.lib()
    d = C.c_void_p(16)
    rc = L.embla_decode_int8(d, d, d, d, None, S, max_s, n_q, n_kv, 0, 0, 0, 0, None, 0, None)
    assert rc == _lib.EMBLA_ERR_INVALID


def test_decode_rejects_missing_workspace_and_nulls():
    L = _lib.lib()
    d = C.c_void_p(16)
    assert L.embla_decode_int8(d, d, d, d, None, 4096, 4096, 16, 4, 0, 0, 0, 128, None, 0, None) == _lib.EMBLA_ERR_WORKSPACE
    assert L.embla_decode_int8(None, d, d, d, None, 64, 64, 16, 4, 0, 0, 0, 0, None, 0, None) == _lib.EMBLA_ERR_INVALID
    # SCORES only with the reference's ReLU² layers
    assert L.embla_decode_int8(d, d, d, d, d, 64, 64, 16, 4, 0, 0, 0, 0, None, 0, None) == _lib.EMBLA_ERR_UNSUPPORTED


def test_kv_append_rejects_out_of_range():
    L = _lib.lib()
    d = C.c_void_p(16)
    assert L.embla_kv_quant_append(d, d, 1, 512, 10, 1020, 4, d, d, 1024, 0, 0, None) == _lib.EMBLA_ERR_INVALID
    assert L.embla_kv_quant_append(d, d, 1, 100, 1, 0, 4, d, d, 1024, 0, 0, None) == _lib.EMBLA_ERR_INVALID


def test_block_copy_rejects_bad_arguments():
    """Block save/restore: p0 not a multiple of 128, a block past max_s, unaligned regions, too
    many layers, a ring not a multiple of 128 (no GPU: validation precedes any HIP call)."""
    L = _lib.lib()
    d = C.c_void_p(256)
    regs = (C.c_ulonglong * 4)(0, 4096, 8192, 12288)
    bad = (C.c_ulonglong * 4)(0, 4100, 8192, 12288)
    ok = L.embla_kv_block_bytes(2, 4, 0)
    assert ok == 2 * 2 * 4 * 128 * 130
    assert L.embla_kv_block_copy(d, regs, 2, 100, 1024, 4, 0, d, 1, None) < 0
    assert L.embla_kv_block_copy(d, regs, 2, 1024, 1024, 4, 0, d, 1, None) < 0
    assert L.embla_kv_block_copy(d, bad, 2, 128, 1024, 4, 0, d, 1, None) < 0
    assert L.embla_kv_block_copy(d, regs, 65, 128, 1024, 4, 0, d, 1, None) < 0
    assert L.embla_ring_block_copy(d, regs, 2, 128, 1000, 4, d, 0, None) < 0
    assert L.embla_ring_block_bytes(2, 4) == 2 * 2 * 4 * 128 * 256


def test_sampling_rejects_bad_arguments():
    """The sampling tail: vocabulary outside 1 .. 65536, unaligned logits, T or top-p out of range,
    a short workspace (no GPU: validation precedes any HIP call)."""
    L = _lib.lib()
    d = C.c_void_p(256)
    g = C.c_void_p(260)
    assert L.embla_sample_workspace_bytes(0) == 0 and L.embla_sample_workspace_bytes(65537) == 0
    ws = L.embla_sample_workspace_bytes(65536)
    assert ws == 65536 * 2 + 2560 + 64 * 4096
    assert L.embla_argmax(d, d, 65537, g, 0, 0, d, ws, None) < 0
    assert L.embla_argmax(C.c_void_p(260), d, 1000, g, 0, 0, d, ws, None) < 0
    assert L.embla_argmax(d, d, 65536, g, 0, 0, d, ws - 1, None) < 0
    assert L.embla_sample(d, d, 65536, g, 0, 0, 0.0, 0.9, 1, d, ws, None) < 0
    assert L.embla_sample(d, d, 65536, g, 0, 0, float("inf"), 0.9, 1, d, ws, None) < 0
    assert L.embla_sample(d, d, 65536, g, 0, 0, 1.0, 0.0, 1, d, ws, None) < 0
    assert L.embla_sample(d, d, 65536, g, 0, 0, 1.0, 1.5, 1, d, ws, None) < 0
    assert L.embla_sample(d, d, 65536, g, -1, 0, 1.0, 0.9, 1, d, ws, None) < 0
    assert L.embla_sample(d, d, 65536, g, 0, 0, 1.0, 0.9, 1, None, ws, None) < 0


def test_decode_split_rejects_single_chunk():
    """The partials/merge pair needs at least two chunks: one chunk writes o itself."""
    L = _lib.lib()
    d = C.c_void_p(256)
    ws = L.embla_workspace_bytes(1024, 16)
    assert L.embla_decode_int8_partials(d, d, d, None, 100, 1024, 16, 4, 0, 0, 0, 0, d, ws, None) < 0
    assert L.embla_decode_int8_merge(d, 100, 1024, 16, 4, 0, 0, 0, d, ws, None) < 0
    assert L.embla_decode_int8_partials(d, d, d, None, 1024, 1024, 16, 4, 0, 0, 0, 256, None, 0, None) < 0


def test_decode_step_rejects_bad_arguments():
    L = _lib.lib()
    d = C.c_void_p(256)
    ws = L.embla_workspace_bytes(1024, 16)

    def step(pos=10, max_s=1024, n_q=16, n_kv=4, scale=0, out=1, chunk=0, ng=0, offs=(0, 2048, 2560), w=d, wb=ws):
        return L.embla_decode_step_int8(d, *offs, None, None, ng, d, d, d, pos, max_s, n_q, n_kv, scale, 0, out, chunk,
                                        w, wb, None)

    assert step(pos=1024) == _lib.EMBLA_ERR_INVALID            # pos past the cache
    assert step(pos=-1) == _lib.EMBLA_ERR_INVALID
    assert step(offs=(0, 2049, 2560)) == _lib.EMBLA_ERR_INVALID  # k not 16-byte aligned
    assert step(offs=(4, 2048, 2560)) == _lib.EMBLA_ERR_INVALID  # q not 16-byte aligned
    assert step(ng=1) == _lib.EMBLA_ERR_INVALID                # a gain count without its gains
    assert step(chunk=48) == _lib.EMBLA_ERR_INVALID
    assert step(w=None, wb=0) == _lib.EMBLA_ERR_WORKSPACE
    assert step(pos=9000, max_s=16384, chunk=32) == _lib.EMBLA_ERR_INVALID  # 282 chunks and the append: over 256
    assert step(scale=2) == _lib.EMBLA_ERR_UNSUPPORTED         # fp32 scales: no instance
    assert step(n_q=32, wb=L.embla_workspace_bytes(1024, 32)) == _lib.EMBLA_ERR_UNSUPPORTED   # 8 q heads a kv head


def test_decode_noalloc_rejects_beyond_its_array():
    """The zero-allocation decode keeps its partials in a fixed device array: a call whose chunks
    would not fit is refused on the host, before any HIP call."""
    L = _lib.lib()
    cap = L.embla_decode_int8_noalloc_max_bytes()
    assert cap == 256 * 32 * 132 * 4
    d = C.c_void_p(16)
    # 256 chunks of 512 keys x 64 query heads x 528 B = 8.6 MB > 4.1 MB
    rc = L.embla_decode_int8_noalloc(d, d, d, d, None, 131072, 131072, 64, 16, 0, 0, 0, 512, None)
    assert rc == _lib.EMBLA_ERR_WORKSPACE
    rc = L.embla_decode_int8_noalloc(d, d, d, d, None, 2000, 1024, 16, 4, 0, 0, 0, 0, None)
    assert rc == _lib.EMBLA_ERR_INVALID
    assert L.embla_decode_int8_noalloc(None, d, d, d, None, 10, 1024, 16, 4, 0, 0, 0, 0, None) == _lib.EMBLA_ERR_INVALID


def test_bf16_cache_entry_points_reject_bad_arguments():
    """The bf16 full-layer cache entry points validate on the host, before any HIP call."""
    L = _lib.lib()
    d = C.c_void_p(16)
    bad = _lib.AttnParams(2000, 0, 0, 1024, 1999, 2, 0, 0)   # S > maxS
    assert L.embla_attn_full(d, d, d, d, d, d, None, d, d, C.byref(bad), None) == _lib.EMBLA_ERR_INVALID
    assert L.embla_attn_sparse(d, d, d, d, d, d, None, d, d, C.byref(bad), None) == _lib.EMBLA_ERR_INVALID
    ok = _lib.AttnParams(100, 48, 0, 1024, 99, 2, 0, 0)      # CH not a multiple of 32
    assert L.embla_attn_full(d, d, d, d, d, d, None, d, d, C.byref(ok), None) == _lib.EMBLA_ERR_INVALID
    jobs = (_lib.KVJob * 1)(_lib.KVJob(2048, 2304, 0, 4096))
    assert L.embla_kv_append_bf16(d, d, jobs, 1, 1000, 1024, 30, None) == _lib.EMBLA_ERR_INVALID   # past maxS
    pb = _lib.AttnB(1000, 0, 0, 1024)
    assert L.embla_attn_full_b(d, d, d, d, d, d, d, d, C.byref(pb), 30, None) == _lib.EMBLA_ERR_INVALID


@pytest.mark.parametrize("n_q,n_kv,n_ih,dtype,rc", [(16, 3, 4, 0, _lib.EMBLA_ERR_INVALID),
                                                     (16, 4, 4, 9, _lib.EMBLA_ERR_INVALID),
                                                     (16, 16, 4, 0, _lib.EMBLA_ERR_UNSUPPORTED),
                                                     (16, 4, 3, 0, _lib.EMBLA_ERR_UNSUPPORTED)])
def test_sparse_layer_rejects_before_any_launch(n_q, n_kv, n_ih, dtype, rc):
    """Every argument of the sparse layer's kernels (scorer, classify, attention) is checked before
    the first launch: a call rejected after its scorer had counted would leave the select's
    histogram stale. (Fake pointers: a launch here, with no GPU, could not return these codes.)"""
    L = _lib.lib()
    d = C.c_void_p(256)
    nb = L.embla_sparse_workspace_bytes(32768, n_q)
    got = L.embla_sparse_layer_decode(d, d, d, d, d, d, d, 32768, 32768, n_q, n_kv, n_ih, dtype, d, nb, None)
    assert got == rc


def test_sparse_workspace_recount_word_inside():
    L = _lib.lib()
    for max_s, n_q in [(32768, 16), (4096, 32), (1153, 8)]:
        nb, off = L.embla_sparse_workspace_bytes(max_s, n_q), L.embla_sparse_workspace_recount_offset(max_s, n_q)
        assert off % 4 == 0 and 0 < off < nb - 4
    assert L.embla_sparse_workspace_recount_offset(0, 16) == 0


def test_prefill_staged_workspace_bytes():
    """The staged workspace holds the split partials and then fp16 K and V for keys 0 .. p0 + T - 1
    (rounded up to 128 positions) of every kv head; invalid sizes give 0."""
    L = _lib.lib()
    base = L.embla_prefill_workspace_bytes(2048, 16)
    st = L.embla_prefill_staged_workspace_bytes(2048, 30720, 16, 4)
    assert st >= base + 2 * 4 * 32768 * 128 * 2
    assert L.embla_prefill_staged_workspace_bytes(100, 5, 16, 4) >= L.embla_prefill_workspace_bytes(100, 16) + 2 * 4 * 128 * 256
    assert L.embla_prefill_staged_workspace_bytes(0, 5, 16, 4) == 0
    assert L.embla_prefill_staged_workspace_bytes(10, -1, 16, 4) == 0


def test_sparse_workspace_audit_rejects_bad_arguments():
    L = _lib.lib()
    d = C.c_void_p(256)
    nb = L.embla_sparse_workspace_bytes(32768, 16)
    assert L.embla_sparse_workspace_audit(None, nb, 32768, 16, None) == _lib.EMBLA_ERR_INVALID
    assert L.embla_sparse_workspace_audit(d, nb - 1, 32768, 16, None) == _lib.EMBLA_ERR_WORKSPACE
    assert L.embla_sparse_workspace_audit(d, nb, 0, 16, None) == _lib.EMBLA_ERR_INVALID
