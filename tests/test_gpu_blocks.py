"""Prefix-cache block save/restore (Engine.fullSpans / windowSpans / copy, PrefixCache.swift:147-200):
the stored bytes are the spans of positions p0 .. p0+127 in the reference's order (per layer K then
V; per kv head its rows, then each head's scales), decoded here with the layout module's own tile
decoder; a restore into a zeroed cache writes those positions back bit for bit and nothing else."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import dev, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def layers(g, n_layers, n_kv, max_s, scale_dtype):
    """Random K, V regions a layer (rows int8, scales of scale_dtype) packed at 256-byte aligned
    offsets of one buffer with gaps between them; returns (buffer, offsets, logical contents)."""
    sb = np.dtype(scale_dtype).itemsize
    rb = layout.region_bytes(n_kv, max_s, sb)
    stride = (rb + 511) // 256 * 256   # a gap after each region
    buf = np.zeros(2 * n_layers * stride, np.uint8)
    regions, logical = [], []
    for l in range(n_layers):
        offs = []
        for kind_i, kind in enumerate("kv"):
            rows = g.int8(n_kv * max_s * 128).reshape(n_kv, max_s, 128)
            sc = g.uniform(n_kv * max_s).astype(np.float32).reshape(n_kv, max_s)
            sc = synth.f16_bits(sc) if scale_dtype == np.uint16 else sc
            off = (2 * l + kind_i) * stride
            buf[off:off + rb] = layout.pack_region(rows, sc, max_s, kind)
            offs.append(off)
            logical.append((rows, sc))
        regions.append(offs)
    return buf, regions, logical


@pytest.mark.parametrize("n_kv,scale", [(4, "f16"), (2, "f32")])
def test_kv_block_save_restore(torch_gpu, n_kv, scale):
    from embla_attn import ops
    torch = torch_gpu
    n_layers, max_s, p0 = 3, 1024, 384
    sdt, code = (np.uint16, ops.F16) if scale == "f16" else (np.float32, ops.F32)
    g = synth.SplitMix64(77)
    buf, regions, logical = layers(g, n_layers, n_kv, max_s, sdt)
    cache = dev(buf)
    nbytes = ops.lib().embla_kv_block_bytes(n_layers, n_kv, code)
    sb = np.dtype(sdt).itemsize
    assert nbytes == n_layers * 2 * n_kv * 128 * (128 + sb)
    stored = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    say(f"kv block save n_kv={n_kv} scale={scale}")
    ops.kv_block_copy(cache, regions, p0, max_s, n_kv, stored, True, scale_dtype=code)
    st = stored.cpu().numpy()
    # the stored spans, in order: for each layer, k then v: each head's rows (tile order), then
    # each head's scales
    at = 0
    for i, (rows, sc) in enumerate(logical):
        for h in range(n_kv):
            got = layout.from_tiles(st[at:at + 128 * 128].view(np.int8), 1, 128, "kv"[i % 2])[0]
            np.testing.assert_array_equal(got, rows[h, p0:p0 + 128], err_msg=f"region {i} head {h} rows")
            at += 128 * 128
        for h in range(n_kv):
            np.testing.assert_array_equal(st[at:at + 128 * sb].view(sdt), sc[h, p0:p0 + 128],
                                          err_msg=f"region {i} head {h} scales")
            at += 128 * sb
    assert at == nbytes
    # restore into a zeroed cache: exactly the block's positions come back
    say("kv block restore")
    fresh = torch.zeros_like(cache)
    ops.kv_block_copy(fresh, regions, p0, max_s, n_kv, stored, False, scale_dtype=code)
    fb = fresh.cpu().numpy()
    for l, offs in enumerate(regions):
        for kind_i, off in enumerate(offs):
            rows, sc = logical[2 * l + kind_i]
            grows, gsc = layout.unpack_region(fb[off:], n_kv, max_s, "kv"[kind_i], sdt)
            want_r = np.zeros_like(rows)
            want_r[:, p0:p0 + 128] = rows[:, p0:p0 + 128]
            want_s = np.zeros_like(sc)
            want_s[:, p0:p0 + 128] = sc[:, p0:p0 + 128]
            np.testing.assert_array_equal(grows, want_r)
            np.testing.assert_array_equal(gsc, want_s)
    mask = np.zeros(fb.size, bool)
    rb = layout.region_bytes(n_kv, max_s, sb)
    for offs in regions:
        for off in offs:
            mask[off:off + rb] = True
    assert not fb[~mask].any(), "bytes outside the regions were written"


def test_ring_block_save_restore(torch_gpu):
    """Sliding-layer checkpoint: ring slots p0 % ring .. +127 of 16-bit K and V rings."""
    from embla_attn import ops
    torch = torch_gpu
    n_layers, n_kv, ring, p0 = 2, 4, 512, 640   # slots 128 .. 255
    g = synth.SplitMix64(78)
    rb = n_kv * ring * 128 * 2
    stride = rb + 256   # a gap after each ring
    buf = np.zeros(2 * n_layers * stride, np.uint8)
    regions, logical = [], []
    for l in range(n_layers):
        offs = []
        for kind_i, kind in enumerate("kv"):
            rows = (g.uniform(n_kv * ring * 128) * 65535).astype(np.uint16).reshape(n_kv, ring, 128)
            off = (2 * l + kind_i) * stride
            buf[off:off + rb] = layout.pack_ring16(rows, kind).view(np.uint8)
            offs.append(off)
            logical.append(rows)
        regions.append(offs)
    cache = dev(buf)
    nbytes = ops.lib().embla_ring_block_bytes(n_layers, n_kv)
    stored = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    say("ring block save")
    ops.ring_block_copy(cache, regions, p0, ring, n_kv, stored, True)
    st = stored.cpu().numpy()
    slot = p0 % ring
    at = 0
    for i, rows in enumerate(logical):
        for h in range(n_kv):
            got = layout.from_tiles(st[at:at + 128 * 256].view(np.uint16), 1, 128, "kv"[i % 2])[0]
            np.testing.assert_array_equal(got, rows[h, slot:slot + 128], err_msg=f"ring {i} head {h}")
            at += 128 * 256
    assert at == nbytes
    say("ring block restore")
    fresh = torch.zeros_like(cache)
    ops.ring_block_copy(fresh, regions, p0, ring, n_kv, stored, False)
    fb = fresh.cpu().numpy()
    for l, offs in enumerate(regions):
        for kind_i, off in enumerate(offs):
            rows = logical[2 * l + kind_i]
            got = layout.from_tiles(fb[off:off + rb].view(np.uint16), n_kv, ring, "kv"[kind_i])
            want = np.zeros_like(rows)
            want[:, slot:slot + 128] = rows[:, slot:slot + 128]
            np.testing.assert_array_equal(got, want)
    mask = np.zeros(fb.size, bool)
    for offs in regions:
        for off in offs:
            mask[off:off + rb] = True
    assert not fb[~mask].any(), "bytes outside the rings were written"
