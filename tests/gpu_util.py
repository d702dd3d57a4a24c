"""Helpers for the GPU parity tests: uploads, region packing, the tolerance of the north star."""
import sys

import numpy as np

from embla_attn import layout, synth

ATOL, RTOL = 2e-3, 1e-2   # max-abs 2e-3 / rel 1e-2, fp32 accumulation


def say(msg):
    """Names the case before a GPU step, flushed, so a fault is attributable."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def f16_host(t):
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16).view(np.float16).astype(np.float32)


def bf16_host(t):
    import torch
    return synth.bf16_val(t.view(torch.int16).cpu().numpy().view(np.uint16))


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tolerance, max abs err {err.max():.3e}"


def upload_int8_case(c, max_s, scale_dtype=np.uint16):
    """Packs a decode_int8_case's K/V into device regions."""
    kreg = layout.pack_region(c["K"], c["ks"].astype(scale_dtype) if scale_dtype != np.uint16 else c["ks"], max_s, "k")
    vreg = layout.pack_region(c["V"], c["vs"].astype(scale_dtype) if scale_dtype != np.uint16 else c["vs"], max_s, "v")
    return dev(kreg), dev(vreg)


def chunk_rows(T=2048, block=32):
    """Rows of a prefill chunk to check at full size: one edge row of every `block`-row tile
    (first rows of even tiles, last rows of odd ones), both edges of the chunk and of its halves:
    at least T / block rows, every tile boundary touched."""
    rows = {0, 1, T // 2 - 1, T // 2, T - 2, T - 1}
    for b in range(T // block):
        rows.add(block * b if b % 2 == 0 else block * b + block - 1)
    return sorted(r for r in rows if r < T)
