"""The reference's full and sparse layers over bf16 caches (EMBLA_KV8=0): kv_append / kv_append_b,
attn_full (ReLU², scores), attn_sparse (softmax, every key or the SEL rows) and attn_full_b, through
the C ABI against the oracle (orc_decode_f32, pinned on the CPU) on the same seeded inputs. Cache
bytes bit-exact; outputs within max-abs 2e-3 / rel 1e-2; scores to fp32 sums of exact products."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, dev, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def case(seed, S, maxS):
    g = synth.SplitMix64(seed)
    K = synth.bf16_bits(g.normal(2 * S * 128)).reshape(2, S, 128)
    V = synth.bf16_bits(g.normal(2 * S * 128)).reshape(2, S, 128)
    qraw = synth.bf16_bits(g.normal(16 * 128) * 2.0).reshape(16, 128)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    Kf = np.zeros((2, maxS, 128), np.uint16)
    Vf = np.zeros((2, maxS, 128), np.uint16)
    Kf[:, :S], Vf[:, :S] = K, V
    return K, V, qraw, g1, g2, layout.pack_ring16(Kf, "k").view(np.int16), layout.pack_ring16(Vf, "v").view(np.int16)


def prep_q(orc, qraw, g1, g2, ng=2):
    return np.stack([orc.head_norm(synth.bf16_val(qraw[h]), synth.bf16_val(g1), synth.bf16_val(g2), ng)
                     for h in range(qraw.shape[0])])


def buffers(torch, maxS):
    from embla_attn import ops
    part = torch.zeros(ops.lib().embla_workspace_bytes(maxS, 16) // 4, dtype=torch.float32, device="cuda")
    counter = torch.zeros(4, dtype=torch.int32, device="cuda")
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    return part, counter, o


@pytest.mark.parametrize("S,maxS", [(1, 32), (33, 64), (1000, 1024), (5000, 5024), (32768, 32768)])
def test_attn_full_bf16_relu2_scores(torch_gpu, orc, S, maxS):
    from embla_attn import ops
    torch = torch_gpu
    say(f"attn_full bf16 S={S}")
    K, V, qraw, g1, g2, kt, vt = case(11, S, maxS)
    part, counter, o = buffers(torch, maxS)
    scores = torch.full((2, maxS), -1.0, dtype=torch.float32, device="cuda")
    ops.attn_full(dev(qraw.view(np.int16), torch.bfloat16), dev(g1.view(np.int16), torch.bfloat16), dev(g2.view(np.int16), torch.bfloat16), dev(kt), dev(vt),
                  part, scores, counter, o, S, maxS)
    ref, rsc = orc.decode_f32(prep_q(orc, qraw, g1, g2), synth.bf16_val(K), synth.bf16_val(V), weights=1,
                              want_scores=True)
    assert_close(bf16_host(o), ref, what=f"attn_full S={S}")
    got = scores.cpu().numpy()[:, :S]
    # bf16 products are exact in fp32: the scores are fp32 sums, within 2^-16 of sum_d |q_d k_d|
    # (128 roundings of 2^-24 with a 2x margin), the max over the kv head's query heads
    qn = np.abs(prep_q(orc, qraw, g1, g2).astype(np.float64))
    Kf = np.abs(synth.bf16_val(K).astype(np.float64))
    bound = np.stack([(qn[8 * h:8 * h + 8] @ Kf[h].T).max(0) for h in range(2)])
    assert (np.abs(got - rsc) <= bound * 2.0 ** -16).all(), f"scores off by {np.abs(got - rsc).max()}"


@pytest.mark.parametrize("S,maxS", [(7, 32), (1000, 1024), (20000, 20000)])
def test_attn_sparse_bf16_all_keys(torch_gpu, orc, S, maxS):
    from embla_attn import ops
    torch = torch_gpu
    say(f"attn_sparse bf16 all keys S={S}")
    K, V, qraw, g1, g2, kt, vt = case(12, S, maxS)
    part, counter, o = buffers(torch, maxS)
    ops.attn_sparse(dev(qraw.view(np.int16), torch.bfloat16), dev(g1.view(np.int16), torch.bfloat16), dev(g2.view(np.int16), torch.bfloat16), dev(kt), dev(vt),
                    part, None, counter, o, S, maxS)
    ref = orc.decode_f32(prep_q(orc, qraw, g1, g2), synth.bf16_val(K), synth.bf16_val(V), weights=0)
    assert_close(bf16_host(o), ref, what=f"attn_sparse S={S}")


@pytest.mark.parametrize("nsel,S", [(1152, 5000), (70, 300), (1152, 32768)])
def test_attn_sparse_bf16_selected_rows(torch_gpu, orc, nsel, S):
    from embla_attn import ops
    torch = torch_gpu
    say(f"attn_sparse bf16 SEL nsel={nsel} S={S}")
    maxS = (S + 31) // 32 * 32
    K, V, qraw, g1, g2, kt, vt = case(13, S, maxS)
    rng = np.random.default_rng(nsel)
    idx = np.stack([rng.permutation(S)[:nsel] for _ in range(2)]).astype(np.uint32)
    part, counter, o = buffers(torch, maxS)
    ops.attn_sparse(dev(qraw.view(np.int16), torch.bfloat16), dev(g1.view(np.int16), torch.bfloat16), dev(g2.view(np.int16), torch.bfloat16), dev(kt), dev(vt),
                    part, dev(idx.view(np.int32)), counter, o, nsel, maxS)
    ref = orc.decode_f32(prep_q(orc, qraw, g1, g2), synth.bf16_val(K), synth.bf16_val(V), weights=0, rows=idx)
    assert_close(bf16_host(o), ref, what=f"attn_sparse SEL nsel={nsel}")


@pytest.mark.parametrize("p0,T,maxS", [(0, 1, 64), (100, 40, 256), (3000, 130, 4096)])
def test_kv_append_bf16_then_attn_full_b(torch_gpu, orc, p0, T, maxS):
    """The prefill flow without KV8: kv_append_b of the chunk, then attn_full_b over keys 0 .. p0 + t."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"kv_append_bf16 + attn_full_b p0={p0} T={T}")
    g = synth.SplitMix64(14)
    hist = synth.bf16_bits(g.normal(2 * 2 * maxS * 128)).reshape(2, 2, maxS, 128)   # K, V history
    hist[:, :, p0:] = 0
    qkv = synth.bf16_bits(g.normal(T * 4096) * 1.5).reshape(T, 4096)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    # one cache buffer: the layer's K region then its V region (element offsets in the jobs)
    region = 2 * maxS * 128
    cache = np.concatenate([layout.pack_ring16(hist[0], "k"), layout.pack_ring16(hist[1], "v")]).view(np.int16)
    cdev = dev(cache)
    kq, vq = 16 * 128, 18 * 128   # the k and v rows of the 2 kv heads in qkv
    ops.kv_append_bf16(dev(qkv.view(np.int16), torch.bfloat16), cdev, [(kq, vq, 0, region)], p0, maxS, T)
    torch.cuda.synchronize()
    got = cdev.cpu().numpy().view(np.uint16)
    Kc = layout.from_tiles(got[:region], 2, maxS, "k")
    Vc = layout.from_tiles(got[region:], 2, maxS, "v")
    for t in range(T):
        for h in range(2):
            k = orc.head_norm(synth.bf16_val(qkv[t, kq + 128 * h:kq + 128 * (h + 1)]), ng=0, round_bf=True)
            np.testing.assert_array_equal(Kc[h, p0 + t], synth.bf16_bits(k), err_msg=f"K row t={t} h={h}")
            np.testing.assert_array_equal(Vc[h, p0 + t], qkv[t, vq + 128 * h:vq + 128 * (h + 1)])
    np.testing.assert_array_equal(Kc[:, :p0], hist[0][:, :p0])
    part = torch.zeros(T * 16 * 129, dtype=torch.float32, device="cuda")
    counter = torch.zeros(2 * T, dtype=torch.int32, device="cuda")
    o = torch.empty((T, 2048), dtype=torch.bfloat16, device="cuda")
    kreg, vreg = cdev[:region], cdev[region:]
    ops.attn_full_b(dev(qkv.view(np.int16), torch.bfloat16), dev(g1.view(np.int16), torch.bfloat16), dev(g2.view(np.int16), torch.bfloat16), kreg, vreg, part,
                    counter, o, p0, T, maxS)
    out = bf16_host(o).reshape(T, 16, 128)
    Kf, Vf = synth.bf16_val(Kc), synth.bf16_val(Vc)
    for t in sorted({0, min(1, T - 1), T // 2, T - 1}):
        q = prep_q(orc, qkv[t, :2048].reshape(16, 128), g1, g2)
        ref = orc.decode_f32(q, Kf[:, :p0 + t + 1], Vf[:, :p0 + t + 1], weights=1)
        assert_close(out[t], ref, what=f"attn_full_b row {t}")
