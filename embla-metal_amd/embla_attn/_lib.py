"""ctypes binding of libembla_attn.so (the C ABI declared in include/embla_attn.h).

The library is the product path; there is no fallback. Loading fails loudly when it is missing.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libembla_attn.so"

EMBLA_OK = 0
EMBLA_ERR_INVALID = -1
EMBLA_ERR_UNSUPPORTED = -2
EMBLA_ERR_HIP = -3
EMBLA_ERR_WORKSPACE = -4
ERRORS = {
    EMBLA_ERR_INVALID: "invalid argument",
    EMBLA_ERR_UNSUPPORTED: "unsupported combination",
    EMBLA_ERR_HIP: "HIP launch error",
    EMBLA_ERR_WORKSPACE: "workspace missing or too small",
}

F16, BF16, F32 = 0, 1, 2
SOFTMAX, RELU2_SINK = 0, 1

vp, sz, i32, u32p, f32p = C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_uint32), C.c_void_p


class AttnParams(C.Structure):
    """Mirrors AttnParams (attention.metal:8-16)."""
    _fields_ = [(n, C.c_int32) for n in ("S", "CH", "C", "maxS", "pos", "ng", "pad0", "pad1")]


class AttnB(C.Structure):
    """Mirrors AttnB (prefill.metal:217)."""
    _fields_ = [(n, C.c_int32) for n in ("p0", "CH", "C", "maxS")]


class KVJob(C.Structure):
    """Mirrors KVJob (attention.metal:108-111)."""
    _fields_ = [(n, C.c_uint32) for n in ("k", "v", "kc", "vc")]


# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "embla_version": (i32, []),
    "embla_workspace_bytes": (sz, [i32, i32]),
    "embla_workspace_init": (i32, [vp, sz, vp]),
    "embla_decode_int8": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_attn_full8": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, C.POINTER(AttnParams), vp]),
    "embla_kv_quant_append": (i32, [vp, vp, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, vp]),
    "embla_kv_append": (i32, [vp, vp, C.POINTER(KVJob), i32, i32, i32, i32, vp]),
    "embla_q_prep": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, i32, vp]),
    "embla_sliding_decode": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_attn_sliding": (i32, [vp, vp, vp, vp, vp, vp, i32, vp]),
    "embla_index_scores": (i32, [vp, vp, vp, vp, i32, i32, vp]),
    "embla_select_topk": (i32, [vp, i32, vp, i32, i32, i32, i32, i32, vp]),
    "embla_select_keys": (i32, [vp, vp, i32, i32, vp]),
    "embla_sparse_decode": (i32, [vp, vp, vp, vp, i32, i32, vp, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_sparse_workspace_bytes": (sz, [i32, i32]),
    "embla_sparse_workspace_recount_offset": (sz, [i32, i32]),
    "embla_sparse_workspace_audit": (i32, [vp, sz, i32, i32, vp]),
    "embla_prefill_int8": (i32, [vp, i32, C.c_long, C.c_long, vp, vp, vp, i32, C.c_long, C.c_long, i32, i32, i32, i32,
                                 i32, i32, i32, i32, vp, sz, vp]),
    "embla_prefill_workspace_bytes": (sz, [i32, i32]),
    "embla_prefill_staged_workspace_bytes": (sz, [i32, i32, i32, i32]),
    "embla_prefill_full": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_relu2_prefill": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "embla_attn_sparse8": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
    "embla_sparse_prefill_workspace_bytes": (sz, [i32, i32]),
    "embla_prefill_sparse": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_ring_append": (i32, [vp, vp, i32, i32, i32, i32, i32, vp, vp, i32, vp, vp]),
    "embla_kv_block_bytes": (sz, [i32, i32, i32]),
    "embla_gemv_q4": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "embla_gemm_q4": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
    "embla_sample_workspace_bytes": (sz, [i32]),
    "embla_q_prep_b": (i32, [vp, vp, vp, vp, i32, vp]),
    "embla_decode_step_int8": (i32, [vp, i32, i32, i32, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32,
                                     vp, sz, vp]),
    "embla_decode_int8_partials": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_decode_int8_merge": (i32, [vp, i32, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_kv_append_bf16": (i32, [vp, vp, C.POINTER(KVJob), i32, i32, i32, i32, vp]),
    "embla_attn_full": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, C.POINTER(AttnParams), vp]),
    "embla_attn_sparse": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, C.POINTER(AttnParams), vp]),
    "embla_attn_full_b": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, C.POINTER(AttnB), i32, vp]),
    "embla_decode_int8_noalloc": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "embla_decode_int8_noalloc_max_bytes": (sz, []),
    "embla_decode_int8_qraw": (i32, [vp, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_argmax": (i32, [vp, vp, i32, vp, i32, i32, vp, sz, vp]),
    "embla_sample": (i32, [vp, vp, i32, vp, i32, i32, C.c_float, C.c_float, C.c_uint32, vp, sz, vp]),
    "embla_kv_block_copy": (i32, [vp, vp, i32, i32, i32, i32, i32, vp, i32, vp]),
    "embla_ring_block_bytes": (sz, [i32, i32]),
    "embla_ring_block_copy": (i32, [vp, vp, i32, i32, i32, i32, vp, i32, vp]),
    "embla_prefill_ring": (i32, [vp, i32, C.c_long, C.c_long, vp, vp, i32, vp, C.c_long, C.c_long, i32, i32, i32, i32,
                                 i32, vp, vp, sz, vp]),
    "embla_prefill_sliding": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
    "embla_attn_sliding8_b": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, vp]),
    "embla_attn_sliding_b": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, vp]),
    "embla_sparse_layer_decode": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, sz, vp]),
}

_lib = None


class EmblaError(RuntimeError):
    def __init__(self, fn: str, rc: int):
        super().__init__(f"{fn} returned {rc} ({ERRORS.get(rc, 'unknown error')})")
        self.rc = rc


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m embla_attn.build` "
                               "(or __graft_entry__.build()); there is no fallback path")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def call(name: str, *args) -> int:
    """Calls an entry point and raises EmblaError on a non-zero return."""
    rc = getattr(lib(), name)(*args)
    if rc != EMBLA_OK:
        raise EmblaError(name, rc)
    return rc
