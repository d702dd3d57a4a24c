"""The 4-bit decode projections (gemv.metal, MLX's affine 4-bit layout) against the oracle's
double-accumulated product: stacked q/k/v segments with their own inputs and outputs, every
epilogue, the o-projection accumulating into an fp32 residual, and K = 4096."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import dev, say
from embla_attn import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def pack(mats):
    """Segments' (words, scales, biases) into one byte buffer, each part 256-byte aligned; returns
    the buffer and each segment's byte offsets."""
    parts, offs, at = [], [], 0
    for m in mats:
        o = []
        for a in m:
            b = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
            pad = (-at) % 256
            parts.append(np.zeros(pad, np.uint8))
            at += pad
            o.append(at)
            parts.append(b)
            at += b.size
        offs.append(o)
    return np.concatenate(parts), offs


def close_bf16(got, ref, what):
    """Within one bf16 rounding step of the oracle (2^-7 relative; the sums differ in order)."""
    err = np.abs(got - ref)
    tol = np.abs(ref) * 2.0 ** -7 + 1e-3 * np.abs(ref).max()
    assert np.all(err <= tol), f"{what}: max err {err.max()} at {np.argmax(err - tol)}"


@pytest.mark.parametrize("epi", [0, 1, 3, 4])
def test_gemv_qkv_segments(torch_gpu, orc, epi):
    """q (2048 rows), k and v (512 each) of one token in one launch; k and v read a second input
    (offset 2048 in X) and write at their own output offsets."""
    from embla_attn import ops
    torch = torch_gpu
    K = 2048
    g = synth.SplitMix64(21)
    shapes = [2048, 512, 512]
    mats = [synth.q4_weights(g, O, K) for O in shapes]
    x = synth.bf16_bits(g.normal(2 * K).astype(np.float32))
    buf, offs = pack(mats)
    ends = np.cumsum(shapes)
    xo = [0, K, K]
    yo = [0, 2048 + 64, 2048 + 64 + 512 + 8]
    segs = [(offs[i][0], offs[i][1], offs[i][2], int(ends[i]), xo[i], yo[i]) for i in range(3)]
    ny = yo[2] + 512
    Y = torch.zeros(ny, dtype=torch.bfloat16 if epi in (0, 1) else torch.float32, device="cuda")
    say(f"gemv qkv epi={epi}")
    ops.gemv_q4(dev(buf), dev(x, torch.bfloat16), Y, segs, K, epi)
    got = Y.float().cpu().numpy()
    for i, (w, s, b) in enumerate(mats):
        ref = orc.q4_matvec(w, s, b, x[xo[i]:xo[i] + K], epi=epi)
        part = got[yo[i]:yo[i] + shapes[i]]
        if epi == 4:
            np.testing.assert_allclose(part, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
        else:
            close_bf16(part, ref, f"segment {i}")
    # rows between the segments' outputs are untouched
    assert not got[2048:2048 + 64].any() and not got[yo[1] + 512:yo[2]].any()


@pytest.mark.parametrize("K", [2048, 4096])
def test_gemv_oproj_accumulates(torch_gpu, orc, K):
    """The o-projection: x (fp32 residual) += bf16(W o), EPI 2."""
    from embla_attn import ops
    torch = torch_gpu
    O = 2048
    g = synth.SplitMix64(22 + K)
    w, s, b = synth.q4_weights(g, O, K)
    o = synth.bf16_bits(g.normal(K).astype(np.float32))
    y0 = g.normal(O).astype(np.float32) * 4
    buf, offs = pack([(w, s, b)])
    Y = dev(y0.copy())
    say(f"gemv o-proj K={K}")
    ops.gemv_q4(dev(buf), dev(o, torch.bfloat16), Y, [(offs[0][0], offs[0][1], offs[0][2], O, 0, 0)], K, 2)
    got = Y.cpu().numpy()
    ref = orc.q4_matvec(w, s, b, o, epi=2, y=y0)
    # y0 + bf16(acc): the bf16 step of acc, and the fp32 sum's rounding
    acc = orc.q4_matvec(w, s, b, o, epi=4)
    assert np.all(np.abs(got - ref) <= np.abs(acc) * 2.0 ** -7 + np.abs(ref) * 2.0 ** -22 + 1e-4)
