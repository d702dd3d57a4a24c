"""Batched prefill over the int8 cache (config C5 full layer; the reference's relu2_prefill_nax)
against the oracle: whole small chunks, and sampled rows of the full-size chunk (prefill row i
equals decode at position p0 + i, Prefill.swift:10-13)."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, chunk_rows, dev, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def quant_rows(orc, x):   # [n][128] float -> int8, fp32 scale
    q = np.empty(x.shape, np.int8)
    s = np.empty(x.shape[0], np.float32)
    for i in range(x.shape[0]):
        q[i], s[i] = orc.quant_row(x[i], round_bf=True)
    return q, s


def cache_after_chunk(orc, c):
    """The logical int8 cache after the chunk's quantise-and-append (fp16 scales), as the oracle
    defines it."""
    n_kv, p0, T = c["n_kv"], c["p0"], c["T"]
    K = np.concatenate([c["K"], np.zeros((n_kv, T, 128), np.int8)], 1)
    V = np.concatenate([c["V"], np.zeros((n_kv, T, 128), np.int8)], 1)
    ks = np.concatenate([synth.f16_val(c["ks"]), np.zeros((n_kv, T), np.float32)], 1)
    vs = np.concatenate([synth.f16_val(c["vs"]), np.zeros((n_kv, T), np.float32)], 1)
    for h in range(n_kv):
        qk, sk = quant_rows(orc, synth.bf16_val(c["kn"][:, h]))
        qv, sv = quant_rows(orc, synth.bf16_val(c["vn"][:, h]))
        K[h, p0:], V[h, p0:] = qk, qv
        ks[h, p0:] = synth.f16_val(synth.f16_bits(sk))
        vs[h, p0:] = synth.f16_val(synth.f16_bits(sv))
    return K, ks, V, vs


def upload_prefix(c, max_s):
    kc = dev(layout.pack_region(c["K"], c["ks"], max_s, "k"))
    vc = dev(layout.pack_region(c["V"], c["vs"], max_s, "v"))
    return kc, vc


@pytest.mark.parametrize("p0,T,window,split", [(1000, 96, 0, False), (0, 64, 0, False), (517, 70, 0, False),
                                                (300, 100, 40, False), (40, 33, 0, False), (3000, 70, 0, True),
                                                (2100, 64, 0, True), (2500, 40, 600, True),
                                                (777, 1, 0, False), (2500, 1, 0, True)])   # one token: a decode
def test_prefill_full_small(torch_gpu, orc, p0, T, window, split):
    """Fused quantise-and-append + causal softmax prefill vs the oracle on every row."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"prefill small p0={p0} T={T} window={window} split={split}")
    c = synth.prefill_case(seed=4, p0=p0, T=T)
    max_s = ((p0 + T + 31) // 32) * 32
    kc, vc = upload_prefix(c, max_s)
    q = dev(c["q"], torch.bfloat16)
    ws = ops.PrefillWorkspace(T, 16) if split else None
    if window == 0:
        o = ops.prefill_full(q, dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16), kc, vc, T, p0, max_s, 4, ws=ws)
    else:
        ops.kv_quant_append(dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16), T, p0, 4, kc, vc, max_s)
        o = ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, window=window, ws=ws)
    K, ks, V, vs = cache_after_chunk(orc, c)
    ref = orc.prefill_int8(synth.bf16_val(c["q"]), K, ks, V, vs, p0, weights=0, window=window)
    assert_close(bf16_host(o), ref, what=f"p0={p0} T={T} w={window}")


@pytest.mark.parametrize("tok_pad,head_stride,split", [(4, 128, False), (0, 136, False), (4, 128, True),
                                                       (0, 136, True)])
def test_prefill_output_strides(torch_gpu, orc, tok_pad, head_stride, split):
    """Output rows at general strides: a token stride that breaks 16-byte alignment (the kernel
    then stores one row a lane) and heads that are not contiguous (coalesced runs of one row)."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"prefill output strides pad={tok_pad} head_stride={head_stride} split={split}")
    p0, T = 1000, 96
    c = synth.prefill_case(seed=4, p0=p0, T=T)
    max_s = ((p0 + T + 31) // 32) * 32
    kc, vc = upload_prefix(c, max_s)
    q = dev(c["q"], torch.bfloat16)
    ops.kv_quant_append(dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16), T, p0, 4, kc, vc, max_s)
    ts = 15 * head_stride + 128 + tok_pad
    buf = torch.full((T * ts,), float("nan"), dtype=torch.bfloat16, device="cuda")
    ws = ops.PrefillWorkspace(T, 16) if split else None
    ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, out=buf, out_strides=(ts, head_stride), ws=ws)
    got = torch.as_strided(buf, (T, 16, 128), (ts, head_stride, 1))
    K, ks, V, vs = cache_after_chunk(orc, c)
    ref = orc.prefill_int8(synth.bf16_val(c["q"]), K, ks, V, vs, p0, weights=0)
    assert_close(bf16_host(got.contiguous()), ref, what=f"strides ({ts}, {head_stride})")
    # nothing written between the rows
    mask = torch.ones(T * ts, dtype=torch.bool, device="cuda")
    torch.as_strided(mask, (T, 16, 128), (ts, head_stride, 1)).fill_(False)
    assert torch.isnan(buf[mask].float()).all(), "stores outside the output rows"


def test_prefill_c5_full_size_sampled_rows(torch_gpu, orc):
    """Config C5 at full size (T = 2048 after 30720 cached): the edge rows of every 32-row tile
    checked against decode-at-position."""
    from embla_attn import ops
    torch = torch_gpu
    p0, T, max_s = 30720, 2048, 32768
    say("prefill C5 full size")
    c = synth.prefill_case(seed=4, p0=p0, T=T)
    kc, vc = upload_prefix(c, max_s)
    o = ops.prefill_full(dev(c["q"], torch.bfloat16), dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16),
                         kc, vc, T, p0, max_s, 4, ws=ops.PrefillWorkspace(T, 16))
    got = bf16_host(o)
    K, ks, V, vs = cache_after_chunk(orc, c)
    # the chunk's int8 bytes are bit-exact with the oracle's quantisation
    Kr, Ks = layout.unpack_region(kc.cpu().numpy(), 4, max_s, "k", np.uint16)
    np.testing.assert_array_equal(Kr[:, p0:], K[:, p0:])
    for i in chunk_rows(T):
        pos = p0 + i
        ref = orc.decode_int8(synth.bf16_val(c["q"][i]), K[:, :pos + 1], ks[:, :pos + 1], V[:, :pos + 1], vs[:, :pos + 1])
        assert_close(got[i], ref, what=f"row {i}")


def test_relu2_prefill_reference_mode(torch_gpu, orc):
    """relu2_prefill_nax: q [16][Tq][128] head-major, 2 kv heads, fp32 scales, ReLU² with sink."""
    from embla_attn import ops
    torch = torch_gpu
    Tq, Tk, maxS = 80, 600, 640
    say("relu2 prefill reference")
    g = synth.SplitMix64(44)
    K = g.int8(2 * Tk * 128).reshape(2, Tk, 128)
    V = g.int8(2 * Tk * 128).reshape(2, Tk, 128)
    ks = (0.02 + 0.02 * g.uniform(2 * Tk)).astype(np.float32).reshape(2, Tk)
    vs = (0.02 + 0.02 * g.uniform(2 * Tk)).astype(np.float32).reshape(2, Tk)
    qn = synth.bf16_bits((g.normal(16 * Tq * 128) * 2).astype(np.float32)).reshape(16, Tq, 128)
    kc = dev(layout.pack_region(K, ks, maxS, "k"))
    vc = dev(layout.pack_region(V, vs, maxS, "v"))
    o = ops.relu2_prefill(dev(qn, torch.bfloat16), kc, vc, Tq, Tk, maxS)
    got = bf16_host(o).reshape(Tq, 16, 128)
    ref = orc.prefill_int8(synth.bf16_val(qn).transpose(1, 0, 2), K, ks, V, vs, Tk - Tq, weights=1)
    assert_close(got, ref, what="relu2 prefill")


def test_q_prep_b_head_major(torch_gpu, orc):
    """q_prep_b: qkv [T][4096] bf16 -> qn [16][T][128], normed with both gains, rounded to bf16:
    the same bytes as the oracle's head_norm (the sum of squares in the oracle's butterfly order)."""
    from embla_attn import ops
    torch = torch_gpu
    T = 37
    g = synth.SplitMix64(55)
    qkv = synth.bf16_bits(g.normal(T * 4096) * 2).reshape(T, 4096)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    qn = ops.q_prep_b(dev(qkv, torch.bfloat16), dev(g1, torch.bfloat16), dev(g2, torch.bfloat16), T)
    torch.cuda.synchronize()
    got = bf16_host(qn)
    assert got.shape == (16, T, 128)
    for t in range(T):
        for h in range(16):
            want = orc.head_norm(synth.bf16_val(qkv[t, h * 128:(h + 1) * 128]), synth.bf16_val(g1), synth.bf16_val(g2), 2)
            np.testing.assert_array_equal(got[h, t], want, err_msg=f"t={t} h={h}")


@pytest.mark.parametrize("p0,T,tight", [(0, 100, False), (1000, 96, False), (2100, 64, False), (2500, 1, False),
                                         (100, 100, True), (30720, 2048, False)])
def test_prefill_staged_copy_bit_identical(torch_gpu, orc, p0, T, tight):
    """With a workspace that holds the staged fp16 copy, the region is converted once
    (prestage_kernel) and attended through the 16-bit tile path: the products are the ones each
    workgroup's own staging forms, so the output is bit for bit the unstaged path's; positions
    past p0 + T (never written: NaN scales) stay out of it."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"prefill staged copy p0={p0} T={T} tight={tight}")
    c = synth.prefill_case(seed=5, p0=p0, T=T)
    # tight: max_s the chunk's end rounded to 32 only, below the staged copy's 128-position rounding
    max_s = ((p0 + T + 31) // 32) * 32 if tight else ((p0 + T + 127) // 128) * 128 + 32
    kc, vc = upload_prefix(c, max_s)
    nrow = 4 * max_s * 128
    for t in (kc, vc):   # the positions after the chunk: random bytes, NaN scales
        t.view(torch.uint8)[nrow:].view(torch.float16)[torch.arange(4, device="cuda")[:, None] * max_s +
                                                         torch.arange(p0 + T, max_s, device="cuda")] = float("nan")
    q = dev(c["q"], torch.bfloat16)
    ops.kv_quant_append(dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16), T, p0, 4, kc, vc, max_s)
    plain = ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, ws=ops.PrefillWorkspace(T, 16))
    wss = ops.PrefillWorkspace(T, 16, staged_p0=p0)
    wss.buf.fill_(0xFF)   # NaN fp16 everywhere the staging does not write
    staged = ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, ws=wss)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(staged.view(torch.int16).cpu().numpy(), plain.view(torch.int16).cpu().numpy())
    if T <= 100:
        K, ks, V, vs = cache_after_chunk(orc, c)
        ref = orc.prefill_int8(synth.bf16_val(c["q"]), K, ks, V, vs, p0, weights=0)
        assert_close(bf16_host(staged), ref, what=f"staged p0={p0} T={T}")
