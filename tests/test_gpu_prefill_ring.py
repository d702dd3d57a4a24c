"""Sliding-window prefill over a 16-bit ring (config C5 sliding, and the reference's kv_sliding_b +
attn_sliding8_b) against the oracle: every checked row is an oracle decode over its window."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, chunk_rows, dev, f16_host, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def ring_rows(hist, upto, R):
    """Slot s holds the latest position p < upto with p % R == s; unwritten slots are zero."""
    rows = np.zeros((hist.shape[0], R, 128), hist.dtype)
    for p in range(max(0, upto - R), upto):
        rows[:, p % R] = hist[:, p]
    return rows


def check_rows(orc, got, Q, Kf, Vf, p0, W, rows, what, atol=2e-3):
    for t in rows:
        p = p0 + t
        ref = orc.decode_rows(Q[t], Kf, Vf, np.arange(max(0, p - W + 1), p + 1, dtype=np.int32))
        assert_close(got[t], ref, atol=atol, what=f"{what} row {t} pos {p}")


@pytest.mark.parametrize("R,W,p0,T,split", [(256, 96, 700, 100, False), (8192, 1024, 0, 70, False),
                                             (8192, 1024, 1500, 131, False), (512, 200, 1000, 33, False),
                                             (8192, 4000, 5000, 64, True), (8192, 1024, 2000, 1, False)])
def test_prefill_sliding_bf16(torch_gpu, orc, R, W, p0, T, split):
    from embla_attn import ops
    torch = torch_gpu
    say(f"prefill_sliding R={R} W={W} p0={p0} T={T} split={split}")
    n_q, n_kv = 16, 4
    total = p0 + T
    g = synth.SplitMix64(40 + T)
    K = synth.bf16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    V = synth.bf16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    Q = synth.bf16_bits(g.normal(T * n_q * 128)).reshape(T, n_q, 128)
    kring = dev(layout.pack_ring16(ring_rows(K, p0, R), "k"))
    vring = dev(layout.pack_ring16(ring_rows(V, p0, R), "v"))
    kn = dev(np.ascontiguousarray(K[:, p0:].transpose(1, 0, 2)), torch.bfloat16)
    vn = dev(np.ascontiguousarray(V[:, p0:].transpose(1, 0, 2)), torch.bfloat16)
    ws = ops.PrefillWorkspace(T, n_q) if split else None
    o = ops.prefill_sliding(dev(Q, torch.bfloat16), kn, vn, kring, vring, T, p0, R, W, n_kv, ws=ws)
    got = bf16_host(o)
    check_rows(orc, got, synth.bf16_val(Q), synth.bf16_val(K), synth.bf16_val(V), p0, W, range(T), "sliding")
    # the append put every chunk row at its slot, bit for bit
    torch.cuda.synchronize()
    got_k = layout.from_tiles(kring.cpu().numpy().view(np.uint16), n_kv, R, "k")
    got_v = layout.from_tiles(vring.cpu().numpy().view(np.uint16), n_kv, R, "v")
    np.testing.assert_array_equal(got_k, ring_rows(K, total, R))
    np.testing.assert_array_equal(got_v, ring_rows(V, total, R))


def test_prefill_ring_f16(torch_gpu, orc):
    """fp16 ring (config C2's storage), rows appended with embla_ring_append, then the ring prefill."""
    from embla_attn import ops
    torch = torch_gpu
    R, W, p0, T, n_q, n_kv = 1024, 300, 2000, 97, 16, 4
    say(f"prefill_ring f16 R={R} W={W} p0={p0} T={T}")
    total = p0 + T
    g = synth.SplitMix64(47)
    K = synth.f16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    V = synth.f16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    Q = synth.f16_bits(g.normal(T * n_q * 128)).reshape(T, n_q, 128)
    kring = dev(layout.pack_ring16(ring_rows(K, p0, R), "k"))
    vring = dev(layout.pack_ring16(ring_rows(V, p0, R), "v"))
    kn = dev(np.ascontiguousarray(K[:, p0:].transpose(1, 0, 2)), torch.float16)
    vn = dev(np.ascontiguousarray(V[:, p0:].transpose(1, 0, 2)), torch.float16)
    ops.ring_append(kn, vn, T, p0, n_kv, kring, vring, R, dtype=ops.F16)
    o = ops.prefill_ring(dev(Q, torch.float16), kring, vring, T, p0, R, W, n_kv, dtype=ops.F16)
    check_rows(orc, f16_host(o), synth.f16_val(Q), synth.f16_val(K), synth.f16_val(V), p0, W, range(T), "f16")


def test_prefill_sliding_c5_size_sampled_rows(torch_gpu, orc):
    """C5 sliding at full size: 2048-token chunk after a 30720-token history, window 1024, bf16 ring
    of 8192; the edge rows of every 32-row tile checked."""
    from embla_attn import ops
    torch = torch_gpu
    R, W, p0, T, n_q, n_kv = 8192, 1024, 30720, 2048, 16, 4
    say("prefill_sliding C5 size")
    g = synth.SplitMix64(4)
    lo = p0 - R   # only the ring's span of history is needed
    K = synth.bf16_bits(g.normal(n_kv * (R + T) * 128)).reshape(n_kv, R + T, 128)
    V = synth.bf16_bits(g.normal(n_kv * (R + T) * 128)).reshape(n_kv, R + T, 128)
    Q = synth.bf16_bits(g.normal(T * n_q * 128)).reshape(T, n_q, 128)
    # history positions lo .. p0-1 sit at slot p % R
    hist = np.zeros((n_kv, R, 128), np.uint16)
    for p in range(lo, p0):
        hist[:, p % R] = K[:, p - lo]
    kring = dev(layout.pack_ring16(hist, "k"))
    for p in range(lo, p0):
        hist[:, p % R] = V[:, p - lo]
    vring = dev(layout.pack_ring16(hist, "v"))
    kn = dev(np.ascontiguousarray(K[:, R:].transpose(1, 0, 2)), torch.bfloat16)
    vn = dev(np.ascontiguousarray(V[:, R:].transpose(1, 0, 2)), torch.bfloat16)
    o = ops.prefill_sliding(dev(Q, torch.bfloat16), kn, vn, kring, vring, T, p0, R, W, n_kv)
    got = bf16_host(o)
    Kf, Vf, Qf = synth.bf16_val(K), synth.bf16_val(V), synth.bf16_val(Q)
    for t in chunk_rows(T):
        p = p0 + t
        rows = np.arange(p - W + 1, p + 1, dtype=np.int32) - lo
        ref = orc.decode_rows(Qf[t], Kf, Vf, rows)
        assert_close(got[t], ref, what=f"C5 sliding row {t}")


def test_attn_sliding8_b_reference_mode(torch_gpu, orc):
    """kv_sliding_b + attn_sliding8_b: qkv [T][4096] bf16, q and k normed with gains and rotated in
    the kernels, ring of 4096, window 128; the chunk crosses the ring's wrap."""
    from embla_attn import ops
    torch = torch_gpu
    R, W, n_kv, p0, T = 4096, 128, 4, 4000, 150
    say(f"attn_sliding8_b p0={p0} T={T}")
    total = p0 + T
    g = synth.SplitMix64(9)
    qg = synth.bf16_bits(g.normal(128) * 0.1)
    kg = synth.bf16_bits(g.normal(128) * 0.1)

    def prep(raw_bits, gain, pos):
        x = orc.head_norm(synth.bf16_val(raw_bits), synth.bf16_val(gain), None, 1, round_bf=False)
        return synth.bf16_val(synth.bf16_bits(orc.rope(x, pos)))

    # history before p0: prepared K rows and raw V rows as the ring holds them
    first = max(0, p0 - R)
    Kp = np.zeros((n_kv, total, 128), np.float32)
    Vb = synth.bf16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    qkv = synth.bf16_bits(g.normal(T * 4096) * 1.5).reshape(T, 4096)
    for t in range(T):
        qkv[t, 20 * 128:24 * 128] = Vb[:, p0 + t].reshape(-1)
    for p in range(first, total):
        raw = qkv[p - p0, 16 * 128:20 * 128] if p >= p0 else synth.bf16_bits(g.normal(512) * 1.5)
        for h in range(n_kv):
            Kp[h, p] = prep(raw[h * 128:(h + 1) * 128], kg, p)
    Kb = synth.bf16_bits(Kp)
    kc = dev(layout.pack_ring16(ring_rows(Kb, p0, R), "k"))
    vc = dev(layout.pack_ring16(ring_rows(Vb, p0, R), "v"))
    o = ops.attn_sliding8_b(dev(qkv, torch.bfloat16), dev(qg, torch.bfloat16), dev(kg, torch.bfloat16), kc, vc, p0, T)
    got = bf16_host(o).reshape(T, 16, 128)
    for t in range(0, T, 7):
        p = p0 + t
        q = np.stack([prep(qkv[t, h * 128:(h + 1) * 128], qg, p) for h in range(16)])
        ref = orc.decode_rows(q, Kp, synth.bf16_val(Vb), np.arange(p - W + 1, p + 1, dtype=np.int32))
        assert_close(got[t], ref, atol=2e-3, what=f"ref row {t}")
    torch.cuda.synchronize()
    got_k = layout.from_tiles(kc.cpu().numpy().view(np.uint16), n_kv, R, "k")
    exp_k = ring_rows(Kb, total, R)
    # the norm's butterfly order and RoPE's rounding are the oracle's: the bytes are equal
    np.testing.assert_array_equal(got_k, exp_k)
    got_v = layout.from_tiles(vc.cpu().numpy().view(np.uint16), n_kv, R, "v")
    np.testing.assert_array_equal(got_v, ring_rows(Vb, total, R))
