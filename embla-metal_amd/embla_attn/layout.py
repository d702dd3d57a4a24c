"""Host-side (numpy) packing of logical K/V rows into the device cache layouts of
include/embla_attn.h, and back.

K and V are stored in 32-key tiles in MFMA lane order (one wave's 16-byte loads read each tile as
contiguous 1 KB runs); an int8 region is the tiles of every kv head, then the scales
[n_kv][max_s]. 16-bit rings use the same tile orders with 2-byte elements and no scales.
"""
from __future__ import annotations

import numpy as np


def tile_offsets(kind: str, es: int) -> np.ndarray:
    """[32][128] element offsets inside a tile of key k (row) and dim d (column)."""
    k = np.arange(32)[:, None]
    d = np.arange(128)[None, :]
    t = k >> 4
    if kind == "k":
        m = k & 15
        lane = m + 16 * (d >> 5)
        p = (d & 31) * es
        j = t * 2 * es + (p >> 4)
    else:
        g = (k >> 2) & 3
        i = k & 3
        lane = (d >> 3) + 16 * g
        p = (8 * (d & 7) + 4 * t + i) * es
        j = p >> 4
    off = (j * 64 + lane) * 16 + (p & 15)
    return off // es


def to_tiles(rows: np.ndarray, kind: str) -> np.ndarray:
    """Logical rows [n_kv][max_s][128] (1- or 2-byte elements) -> the tile layout, flat."""
    n_kv, max_s, hd = rows.shape
    assert max_s % 32 == 0 and hd == 128
    es = rows.dtype.itemsize
    off = tile_offsets(kind, es).reshape(-1)
    out = np.empty((n_kv, max_s // 32, 4096), rows.dtype)
    out[:, :, off] = rows.reshape(n_kv, max_s // 32, 4096)
    return out.reshape(-1)


def from_tiles(flat: np.ndarray, n_kv: int, max_s: int, kind: str) -> np.ndarray:
    es = flat.dtype.itemsize
    off = tile_offsets(kind, es).reshape(-1)
    t = flat.reshape(n_kv, max_s // 32, 4096)
    return np.ascontiguousarray(t[:, :, off].reshape(n_kv, max_s, 128))


def region_bytes(n_kv: int, max_s: int, scale_bytes: int) -> int:
    return n_kv * max_s * 128 + n_kv * max_s * scale_bytes


def pack_region(rows: np.ndarray, scales: np.ndarray, max_s: int, kind: str) -> np.ndarray:
    """Logical int8 rows [n_kv][S][128] and scales [n_kv][S] (fp16 bits as uint16, or float32)
    -> the region's bytes (uint8), positions S .. max_s-1 zero."""
    n_kv, S, _ = rows.shape
    full = np.zeros((n_kv, max_s, 128), np.int8)
    full[:, :S] = rows
    sc = np.zeros((n_kv, max_s), scales.dtype)
    sc[:, :S] = scales
    return np.concatenate([to_tiles(full, kind).view(np.uint8), sc.reshape(-1).view(np.uint8)])


def unpack_region(buf: np.ndarray, n_kv: int, max_s: int, kind: str, scale_dtype) -> tuple:
    """The region's bytes -> (logical int8 rows [n_kv][max_s][128], scales [n_kv][max_s])."""
    buf = np.asarray(buf, np.uint8)
    nrow = n_kv * max_s * 128
    rows = from_tiles(buf[:nrow].view(np.int8), n_kv, max_s, kind)
    es = np.dtype(scale_dtype).itemsize
    sc = buf[nrow:nrow + n_kv * max_s * es].view(scale_dtype).reshape(n_kv, max_s)
    return rows, sc


def pack_ring16(rows: np.ndarray, kind: str) -> np.ndarray:
    """16-bit rows [n_kv][ring][128] (uint16 bits) -> the ring's tile layout, flat."""
    return to_tiles(np.ascontiguousarray(rows, np.uint16), kind)
