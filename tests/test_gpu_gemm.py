"""The 4-bit prefill projections (gemm.metal, MLX's affine 4-bit layout) against the oracle, row
by row: ragged token and row counts (partial tiles), the epilogues, an fp32 residual accumulated
in place, and sampled rows at config C5's size (2048 tokens, q/k/v 3072 rows).

Tolerance: the kernel stages the dequantised weights as bf16, as MLX's GEMM does (each weight
rounded to nearest: within 2^-8 of itself), so an output is within 2^-8 sum |w x| of the exact
product, plus one bf16 rounding of the output (2^-8 of it) for the bf16 epilogues."""
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


def pack(w, s, b):
    parts, offs, at = [], [], 0
    for a in (w, s, b):
        pad = (-at) % 256
        parts.append(np.zeros(pad, np.uint8))
        at += pad
        offs.append(at)
        a8 = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        parts.append(a8)
        at += a8.size
    return np.concatenate(parts), offs


def dense(w, s, b):
    """The dequantised matrix in fp64 (s * q + b), for the error scale."""
    O, K = w.shape[0], w.shape[1] * 8
    q = np.stack([(w >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], -1).reshape(O, K).astype(np.float64)
    return np.repeat(synth.bf16_val(s), 64, 1) * q + np.repeat(synth.bf16_val(b), 64, 1)


def check(got, orc, w, s, b, X, rows, epi, y0=None):
    Wd = dense(w, s, b)
    for t in rows:
        ref = orc.q4_matvec(w, s, b, X[t], epi=epi, y=None if y0 is None else y0[t])
        xt = synth.bf16_val(X[t]).astype(np.float64)
        acc = np.abs(Wd @ xt)
        d = 2.0 ** -8 * np.abs(Wd * xt).sum(1)     # the weights rounded to bf16
        if epi != 4:
            d += 2.0 ** -8 * (acc + d)             # acc rounded to bf16 (the two sides may differ)
        if epi == 1:
            d = 2 * (acc + d) * d + 2.0 ** -8 * (acc + d) ** 2   # squared, then rounded again
        tol = d + 1e-5 + (0 if y0 is None else np.abs(y0[t]) * 2.0 ** -22)
        err = np.abs(got[t] - ref)
        assert np.all(err <= tol), f"token {t}: max err {err.max()} (tol {tol[np.argmax(err - tol)]})"


@pytest.mark.parametrize("epi", [0, 1, 3, 4])
def test_gemm_ragged(torch_gpu, orc, epi):
    from embla_attn import ops
    torch = torch_gpu
    T, O, K = 300, 520, 2048
    g = synth.SplitMix64(31 + epi)
    w, s, b = synth.q4_weights(g, O, K)
    X = synth.bf16_bits(g.normal(T * K).astype(np.float32)).reshape(T, K)
    buf, offs = pack(w, s, b)
    Y = torch.zeros((T, O), dtype=torch.bfloat16 if epi in (0, 1) else torch.float32, device="cuda")
    say(f"gemm ragged epi={epi}")
    ops.gemm_q4(dev(buf), offs, dev(X, torch.bfloat16), Y, T, O, K, epi)
    got = Y.float().cpu().numpy()
    check(got, orc, w, s, b, X, [0, 1, 127, 128, 255, 256, 299], epi)


def test_gemm_residual_strided(torch_gpu, orc):
    """The o-projection at prefill: an fp32 residual [T][ldy] += bf16(X W^T), X rows at a stride."""
    from embla_attn import ops
    torch = torch_gpu
    T, O, K, ldx, ldy = 200, 384, 2048, 2048 + 64, 400
    g = synth.SplitMix64(37)
    w, s, b = synth.q4_weights(g, O, K)
    Xs = synth.bf16_bits(g.normal(T * ldx).astype(np.float32)).reshape(T, ldx)
    y0 = (g.normal(T * ldy).astype(np.float32) * 3).reshape(T, ldy)
    buf, offs = pack(w, s, b)
    Y = dev(y0.copy())
    say("gemm residual strided")
    ops.gemm_q4(dev(buf), offs, dev(Xs, torch.bfloat16), Y, T, O, K, 2, ldx=ldx, ldy=ldy)
    got = Y.cpu().numpy()
    check(got[:, :O], orc, w, s, b, Xs[:, :K], [0, 63, 64, 150, 199], 2, y0=y0[:, :O])
    np.testing.assert_array_equal(got[:, O:], y0[:, O:])   # columns past O untouched


def test_gemm_c5_qkv_sampled(torch_gpu, orc):
    """C5's chunk: 2048 tokens through the q/k/v projection (3072 rows, K 2048), bf16 out."""
    from embla_attn import ops
    torch = torch_gpu
    T, O, K = 2048, 3072, 2048
    g = synth.SplitMix64(39)
    w, s, b = synth.q4_weights(g, O, K)
    X = synth.bf16_bits(g.normal(T * K).astype(np.float32)).reshape(T, K)
    buf, offs = pack(w, s, b)
    Y = torch.empty((T, O), dtype=torch.bfloat16, device="cuda")
    say("gemm C5 qkv")
    ops.gemm_q4(dev(buf), offs, dev(X, torch.bfloat16), Y, T, O, K, 0)
    got = Y.float().cpu().numpy()
    check(got, orc, w, s, b, X, [0, 777, 2047], 0)
