"""Cache positions past the keys a call reads may hold anything (memory never written): NaN scales
and arbitrary int8 rows there must not reach the output. The kernels read whole 32-key tiles (and
128-key staged tiles in prefill), so the last tile's keys past the limit are masked; these tests
poison them and compare with the oracle over the valid keys only (int8 caches), or with the same
call over a zero-filled ring (16-bit rings)."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, dev, f16_host, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu

NAN16 = np.uint16(0x7E00)


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def poisoned_regions(K, ks, V, vs, S, max_s, seed):
    """Regions whose positions S .. max_s - 1 hold random int8 rows and NaN fp16 scales."""
    g = synth.SplitMix64(seed)
    n_kv = K.shape[0]
    tail = max_s - S
    Kp = np.concatenate([K[:, :S], g.int8(n_kv * tail * 128).reshape(n_kv, tail, 128)], 1)
    Vp = np.concatenate([V[:, :S], g.int8(n_kv * tail * 128).reshape(n_kv, tail, 128)], 1)
    ksp = np.concatenate([ks[:, :S], np.full((n_kv, tail), NAN16, np.uint16)], 1)
    vsp = np.concatenate([vs[:, :S], np.full((n_kv, tail), NAN16, np.uint16)], 1)
    return dev(layout.pack_region(Kp, ksp, max_s, "k")), dev(layout.pack_region(Vp, vsp, max_s, "v"))


@pytest.mark.parametrize("S,max_s,chunk", [(1000, 1024, 0), (33, 64, 0), (4001, 4096, 0),
                                           # chunks of several tiles a wave: the in-tile reload of
                                           # the next tile meets the partial, poisoned last tile
                                           (4001, 4096, 2048), (4001, 4096, 4096), (30001, 30016, 4096)])
def test_decode_ignores_poisoned_tail(torch_gpu, orc, S, max_s, chunk):
    from embla_attn import ops
    torch = torch_gpu
    say(f"decode poisoned tail S={S} max_s={max_s} chunk={chunk}")
    c = synth.decode_int8_case(seed=31, S=S)
    kc, vc = poisoned_regions(c["K"], c["ks"], c["V"], c["vs"], S, max_s, 5)
    o = ops.decode_int8(dev(c["q"], torch.float16), kc, vc, S, max_s, 4, chunk=chunk, ws=ops.Workspace(max_s, 16))
    ref = orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    assert_close(f16_host(o), ref, what=f"S={S}")


@pytest.mark.parametrize("pos", [1000, 40])
def test_decode_step_ignores_poisoned_tail(torch_gpu, orc, pos):
    """The fused step appends position pos itself; positions past it stay poisoned."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"decode step poisoned tail pos={pos}")
    max_s = 1024
    c = synth.decode_int8_case(seed=32, S=pos)
    kc, vc = poisoned_regions(c["K"], c["ks"], c["V"], c["vs"], pos, max_s, 6)
    g = synth.SplitMix64(33)
    qkv = synth.bf16_bits(g.normal(24 * 128) * 2)
    x = dev(qkv, torch.bfloat16)
    o = ops.decode_step_int8(x, 0, 2048, 2560, kc, vc, pos, max_s, 16, 4, ops.Workspace(max_s, 16))
    torch.cuda.synchronize()
    K, ks = layout.unpack_region(kc.cpu().numpy(), 4, max_s, "k", np.uint16)
    V, vs = layout.unpack_region(vc.cpu().numpy(), 4, max_s, "v", np.uint16)
    n = pos + 1
    qn = np.stack([orc.head_norm(synth.bf16_val(qkv[h * 128:(h + 1) * 128])) for h in range(16)])
    ref = orc.decode_int8(qn, np.ascontiguousarray(K[:, :n]), synth.f16_val(np.ascontiguousarray(ks[:, :n])),
                          np.ascontiguousarray(V[:, :n]), synth.f16_val(np.ascontiguousarray(vs[:, :n])))
    assert_close(bf16_host(o), ref, what=f"pos={pos}")


@pytest.mark.parametrize("p0,T,max_s", [(1000, 20, 1152), (100, 5, 256)])
def test_prefill_ignores_poisoned_tail(torch_gpu, orc, p0, T, max_s):
    from embla_attn import ops
    torch = torch_gpu
    say(f"prefill poisoned tail p0={p0} T={T} max_s={max_s}")
    c = synth.prefill_case(seed=34, p0=p0, T=T)
    kc, vc = poisoned_regions(c["K"], c["ks"], c["V"], c["vs"], p0, max_s, 7)
    o = ops.prefill_full(dev(c["q"], torch.bfloat16), dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16),
                         kc, vc, T, p0, max_s, 4)
    torch.cuda.synchronize()
    K, ks = layout.unpack_region(kc.cpu().numpy(), 4, max_s, "k", np.uint16)
    V, vs = layout.unpack_region(vc.cpu().numpy(), 4, max_s, "v", np.uint16)
    n = p0 + T
    ref = orc.prefill_int8(synth.bf16_val(c["q"]), np.ascontiguousarray(K[:, :n]),
                           synth.f16_val(np.ascontiguousarray(ks[:, :n])), np.ascontiguousarray(V[:, :n]),
                           synth.f16_val(np.ascontiguousarray(vs[:, :n])), p0, weights=0)
    assert_close(bf16_host(o), ref, what=f"p0={p0} T={T}")


def ring_pair(rows_hist, upto, R, kind):
    """A ring after positions 0 .. upto - 1, slots never written zero, and the same ring with NaN
    bits in those slots (16-bit rows)."""
    n_kv = rows_hist.shape[0]
    zero = np.zeros((n_kv, R, 128), np.uint16)
    zero[:, :upto] = rows_hist[:, :upto]
    bad = zero.copy()
    bad[:, upto:] = NAN16
    return layout.pack_ring16(zero, kind), layout.pack_ring16(bad, kind)


@pytest.mark.parametrize("pos", [3, 100, 1000])
def test_ring_decode_ignores_unwritten_slots(torch_gpu, pos):
    """Early in a ring's life its slots past pos were never written: NaN bits there change nothing
    (the zero-filled ring's outputs are checked against the oracle in test_gpu_sliding)."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"ring decode unwritten slots pos={pos}")
    R, W, n_kv = 8192, 1024, 4
    g = synth.SplitMix64(40)
    K = synth.f16_bits(g.normal(n_kv * (pos + 1) * 128)).reshape(n_kv, pos + 1, 128)
    V = synth.f16_bits(g.normal(n_kv * (pos + 1) * 128)).reshape(n_kv, pos + 1, 128)
    q = synth.f16_bits(g.normal(16 * 128)).reshape(16, 128)
    outs = []
    for i in range(2):
        kr = dev(ring_pair(K, pos, R, "k")[i])
        vr = dev(ring_pair(V, pos, R, "v")[i])
        outs.append(ops.sliding_decode(dev(q, torch.float16), dev(K[:, pos].copy(), torch.float16),
                                       dev(V[:, pos].copy(), torch.float16), kr, vr, pos, W, R, n_kv,
                                       ws=ops.Workspace(R, 16)))
    torch.cuda.synchronize()
    a, b = (o.cpu().numpy() for o in outs)
    assert np.isfinite(f16_host(outs[1])).all()
    np.testing.assert_array_equal(b, a)


@pytest.mark.parametrize("p0,T", [(0, 40), (100, 20)])
def test_ring_prefill_ignores_unwritten_slots(torch_gpu, p0, T):
    from embla_attn import ops
    torch = torch_gpu
    say(f"ring prefill unwritten slots p0={p0} T={T}")
    R, W, n_kv = 8192, 1024, 4
    g = synth.SplitMix64(41)
    n = p0 + T
    K = synth.f16_bits(g.normal(n_kv * n * 128)).reshape(n_kv, n, 128)
    V = synth.f16_bits(g.normal(n_kv * n * 128)).reshape(n_kv, n, 128)
    q = synth.f16_bits(g.normal(T * 16 * 128)).reshape(T, 16, 128)
    outs = []
    for i in range(2):
        kr = dev(ring_pair(K, n, R, "k")[i])
        vr = dev(ring_pair(V, n, R, "v")[i])
        outs.append(ops.prefill_ring(dev(q, torch.float16), kr, vr, T, p0, R, W, n_kv, dtype=ops.F16))
    torch.cuda.synchronize()
    a, b = (o.cpu().numpy() for o in outs)
    assert np.isfinite(f16_host(outs[1])).all()
    np.testing.assert_array_equal(b, a)


@pytest.mark.parametrize("S,max_s,relu2", [(1000, 1024, True), (4001, 4096, False)])
def test_bf16_cache_decode_ignores_poisoned_tail(torch_gpu, orc, S, max_s, relu2):
    """The bf16 full-layer cache (no KV8): positions past S hold NaN bit patterns."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"bf16 cache decode poisoned tail S={S} relu2={relu2}")
    g = synth.SplitMix64(35)
    K = synth.bf16_bits(g.normal(2 * max_s * 128)).reshape(2, max_s, 128)
    V = synth.bf16_bits(g.normal(2 * max_s * 128)).reshape(2, max_s, 128)
    K[:, S:], V[:, S:] = 0x7FC1, 0xFFC3
    qraw = synth.bf16_bits(g.normal(16 * 128) * 2).reshape(16, 128)
    part = torch.zeros(ops.lib().embla_workspace_bytes(max_s, 16) // 4, dtype=torch.float32, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    fn = ops.attn_full if relu2 else ops.attn_sparse
    fn(dev(qraw.view(np.int16), torch.bfloat16), None, None, dev(layout.pack_ring16(K, "k").view(np.int16)),
       dev(layout.pack_ring16(V, "v").view(np.int16)), part, None, counter, o, S, max_s, ng=0)
    qn = np.stack([orc.head_norm(synth.bf16_val(qraw[h])) for h in range(16)])
    ref = orc.decode_f32(qn, synth.bf16_val(K[:, :S]), synth.bf16_val(V[:, :S]), weights=int(relu2))
    assert_close(bf16_host(o), ref, what=f"S={S}")
