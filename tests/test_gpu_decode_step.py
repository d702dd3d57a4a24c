"""embla_decode_step_int8: a full layer's decode step with its own append (the reference's kv_append
then attn_full8 softmax, Engine.swift:782-818) in one split-K launch. The cache bytes it writes are
compared bit for bit with embla_kv_quant_append's; its output with the oracle's decode over the
appended cache (keys 0 .. pos) and with the two-call path (append, then embla_decode_int8_qraw)."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, dev, say, upload_int8_case
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


N_Q, N_KV = 16, 4
Q_OFF, K_OFF, V_OFF = 0, N_Q * 128, N_Q * 128 + N_KV * 128


def step_case(seed, max_s):
    c = synth.decode_int8_case(seed=seed, S=max_s)
    g = synth.SplitMix64(700 + seed)
    qkv = synth.bf16_bits(g.normal((N_Q + 2 * N_KV) * 128) * 2)
    qkv[K_OFF + 128:K_OFF + 256] = 0      # kv head 1's new key is all zeros: int8 zeros, scale 0
    g1 = synth.bf16_bits(1 + g.normal(128) * 0.2)
    g2 = synth.bf16_bits(1 + g.normal(128) * 0.2)
    return c, qkv, g1, g2


# (pos, max_s, chunk): the first token (no cached key: the appended key only), a few keys in one
# chunk, the chunk boundary, and long contexts
CASES = [(0, 1024, 0), (1, 1024, 0), (31, 1024, 0), (32, 1024, 0), (100, 1024, 64), (3000, 4096, 0),
         (32767, 32768, 0), (20000, 32768, 128)]


@pytest.mark.parametrize("pos,max_s,chunk", CASES)
@pytest.mark.parametrize("norm_k", [True, False])
def test_decode_step_matches_append_then_decode(torch_gpu, orc, pos, max_s, chunk, norm_k):
    from embla_attn import ops
    torch = torch_gpu
    say(f"decode step pos={pos} max_s={max_s} chunk={chunk} norm_k={norm_k}")
    c, qkv, g1, g2 = step_case(pos % 97 + 3, max_s)
    kc, vc = upload_int8_case(c, max_s)
    kc2, vc2 = kc.clone(), vc.clone()
    x = dev(qkv, torch.bfloat16)
    dg1, dg2 = dev(g1, torch.bfloat16), dev(g2, torch.bfloat16)
    ws = ops.Workspace(max_s, N_Q)
    o = ops.decode_step_int8(x, Q_OFF, K_OFF, V_OFF, kc, vc, pos, max_s, N_Q, N_KV, ws, g1=dg1, g2=dg2, ng=2,
                             norm_k=norm_k, chunk=chunk)
    # the two-call path
    kv = x[K_OFF:].view(2, N_KV, 128)
    ops.kv_quant_append(kv[0], kv[1], 1, pos, N_KV, kc2, vc2, max_s, norm_k=norm_k)
    o2 = ops.decode_int8_qraw(x[:N_Q * 128], kc2, vc2, pos + 1, max_s, N_KV, g1=dg1, g2=dg2, ng=2, ws=ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy(), kc2.cpu().numpy())
    np.testing.assert_array_equal(vc.cpu().numpy(), vc2.cpu().numpy())
    K, ks = layout.unpack_region(kc.cpu().numpy(), N_KV, max_s, "k", np.uint16)
    V, vs = layout.unpack_region(vc.cpu().numpy(), N_KV, max_s, "v", np.uint16)
    qr = synth.bf16_val(qkv[:N_Q * 128].reshape(N_Q, 128))
    qn = np.stack([orc.head_norm(qr[h], synth.bf16_val(g1), synth.bf16_val(g2), 2) for h in range(N_Q)])
    n = pos + 1
    ref = orc.decode_int8(qn, np.ascontiguousarray(K[:, :n]), synth.f16_val(np.ascontiguousarray(ks[:, :n])),
                          np.ascontiguousarray(V[:, :n]), synth.f16_val(np.ascontiguousarray(vs[:, :n])))
    got = bf16_host(o)
    assert_close(got, ref, what=f"pos={pos}")
    assert_close(got, bf16_host(o2), what=f"pos={pos} against the two-call path")


def test_decode_step_successive_positions(torch_gpu, orc):
    """Steps at positions 0 .. 40 in turn, each appending its own token: the cache after them is
    the one-call appends', and each step's output is the oracle's over the keys so far."""
    from embla_attn import ops
    torch = torch_gpu
    say("decode step, successive positions")
    max_s = 256
    ws = ops.Workspace(max_s, N_Q)
    c, _, g1, g2 = step_case(1, max_s)
    kc, vc = upload_int8_case(c, max_s)
    kc2, vc2 = kc.clone(), vc.clone()
    dg1, dg2 = dev(g1, torch.bfloat16), dev(g2, torch.bfloat16)
    g = synth.SplitMix64(99)
    for pos in range(41):
        qkv = synth.bf16_bits(g.normal((N_Q + 2 * N_KV) * 128) * 2)
        x = dev(qkv, torch.bfloat16)
        o = ops.decode_step_int8(x, Q_OFF, K_OFF, V_OFF, kc, vc, pos, max_s, N_Q, N_KV, ws, g1=dg1, g2=dg2, ng=2,
                                 norm_k=True)
        kv = x[K_OFF:].view(2, N_KV, 128)
        ops.kv_quant_append(kv[0], kv[1], 1, pos, N_KV, kc2, vc2, max_s, norm_k=True)
        if pos in (0, 7, 40):
            torch.cuda.synchronize()
            K, ks = layout.unpack_region(kc2.cpu().numpy(), N_KV, max_s, "k", np.uint16)
            V, vs = layout.unpack_region(vc2.cpu().numpy(), N_KV, max_s, "v", np.uint16)
            qr = synth.bf16_val(qkv[:N_Q * 128].reshape(N_Q, 128))
            qn = np.stack([orc.head_norm(qr[h], synth.bf16_val(g1), synth.bf16_val(g2), 2) for h in range(N_Q)])
            n = pos + 1
            ref = orc.decode_int8(qn, np.ascontiguousarray(K[:, :n]), synth.f16_val(np.ascontiguousarray(ks[:, :n])),
                                  np.ascontiguousarray(V[:, :n]), synth.f16_val(np.ascontiguousarray(vs[:, :n])))
            assert_close(bf16_host(o), ref, what=f"step at pos={pos}")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy(), kc2.cpu().numpy())
    np.testing.assert_array_equal(vc.cpu().numpy(), vc2.cpu().numpy())
    assert not ws.buf[:256].cpu().numpy().any(), "counters left nonzero"
