"""Sliding-window ring decode (config C2 and the reference's attn_sliding) against the oracle,
step after step, across the ring's wrap-around."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, dev, f16_host, bf16_host, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def ring_rows(hist, upto, R):
    """The ring's logical rows after positions 0 .. upto-1 were written: slot s holds the latest
    position p < upto with p % R == s."""
    n_kv = hist.shape[0]
    rows = np.zeros((n_kv, R, 128), hist.dtype)
    for p in range(max(0, upto - R), upto):
        rows[:, p % R] = hist[:, p]
    return rows


@pytest.mark.parametrize("R,W,p_start,steps,chunk", [(8192, 1024, 8192 + 100, 6, 0), (8192, 1024, 3, 4, 0),
                                                      (8192, 1024, 1000, 40, 0), (256, 96, 700, 30, 64),
                                                      (8192, 1024, 9000, 3, 1024)])
def test_sliding_decode_config(torch_gpu, orc, R, W, p_start, steps, chunk):
    from embla_attn import ops
    torch = torch_gpu
    say(f"sliding decode R={R} W={W} p_start={p_start} steps={steps} chunk={chunk}")
    n_kv, n_q = 4, 16
    total = p_start + steps
    g = synth.SplitMix64(1)
    K = synth.f16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    V = synth.f16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    Q = synth.f16_bits(g.normal(steps * n_q * 128)).reshape(steps, n_q, 128)
    kring = dev(layout.pack_ring16(ring_rows(K, p_start, R), "k"))
    vring = dev(layout.pack_ring16(ring_rows(V, p_start, R), "v"))
    ws = ops.Workspace(R, n_q)
    Kf, Vf = synth.f16_val(K), synth.f16_val(V)
    for s in range(steps):
        pos = p_start + s
        o = ops.sliding_decode(dev(Q[s], torch.float16), dev(K[:, pos].copy(), torch.float16),
                               dev(V[:, pos].copy(), torch.float16), kring, vring, pos, W, R, n_kv, chunk=chunk, ws=ws)
        lo = max(0, pos - W + 1)
        ref = orc.decode_rows(synth.f16_val(Q[s]), Kf, Vf, np.arange(lo, pos + 1, dtype=np.int32))
        assert_close(f16_host(o), ref, what=f"step {s} pos {pos}")
    # the ring now holds every appended row at its slot
    torch.cuda.synchronize()
    got_k = layout.from_tiles(kring.cpu().numpy().view(np.uint16), n_kv, R, "k")
    np.testing.assert_array_equal(got_k, ring_rows(K, total, R))


def test_attn_sliding_reference_mode(torch_gpu, orc):
    """attn_sliding: q, k normed with gains and rotated, bf16 ring of 4096, window 128."""
    from embla_attn import ops
    torch = torch_gpu
    R, W, n_kv = 4096, 128, 4
    g = synth.SplitMix64(8)
    qg = synth.bf16_bits(g.normal(128) * 0.1)
    kg = synth.bf16_bits(g.normal(128) * 0.1)
    p_start, steps = 4090, 12   # crosses the wrap at 4096
    total = p_start + steps

    def prep(raw_bits, gain, pos):
        x = orc.head_norm(synth.bf16_val(raw_bits), synth.bf16_val(gain), None, 1, round_bf=False)
        return synth.bf16_val(synth.bf16_bits(orc.rope(x, pos)))

    # history: prepared k rows as the ring holds them, raw v
    Kp = np.zeros((n_kv, total, 128), np.float32)
    Vb = synth.bf16_bits(g.normal(n_kv * total * 128)).reshape(n_kv, total, 128)
    raws = []
    for p in range(total):
        qkv = synth.bf16_bits(g.normal(4096) * 1.5)
        qkv[20 * 128:24 * 128] = Vb[:, p].reshape(-1)
        raws.append(qkv)
        for h in range(n_kv):
            Kp[h, p] = prep(qkv[16 * 128 + h * 128:16 * 128 + (h + 1) * 128], kg, p)
    Kb = synth.bf16_bits(Kp)
    say(f"attn_sliding reference p_start={p_start}")
    kc = dev(layout.pack_ring16(ring_rows(Kb, p_start, R), "k"))
    vc = dev(layout.pack_ring16(ring_rows(Vb, p_start, R), "v"))
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    for s in range(steps):
        pos = p_start + s
        ops.attn_sliding(dev(raws[pos], torch.bfloat16), dev(qg, torch.bfloat16), dev(kg, torch.bfloat16), kc, vc, o, pos)
        q = np.stack([prep(raws[pos][h * 128:(h + 1) * 128], qg, pos) for h in range(16)])
        lo = max(0, pos - W + 1)
        ref = orc.decode_rows(q, Kp, synth.bf16_val(Vb), np.arange(lo, pos + 1, dtype=np.int32))
        assert_close(bf16_host(o), ref, atol=2e-3, what=f"ref step {s}")
    got_k = layout.from_tiles(kc.cpu().numpy().view(np.uint16), n_kv, R, "k")
    exp_k = ring_rows(Kb, total, R)
    # the norm's butterfly order and RoPE's rounding are the oracle's: the bytes are equal
    np.testing.assert_array_equal(got_k, exp_k)
