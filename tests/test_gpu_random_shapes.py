"""Seeded random shapes against the oracle: decode over int8 caches at random lengths, capacities
and chunkings; prefill at random prefix lengths and chunk sizes, staged and unstaged (bit-equal to
each other); the sparse-layer decode at random lengths, its selection bit for bit. The cases are
drawn once from fixed seeds, so a failure names a reproducible shape."""
import random

import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, dev, f16_host, say, upload_int8_case
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


def _decode_cases():
    rng = random.Random(1234)
    out = []
    for i in range(8):
        S = rng.randint(1, 20000)
        max_s = (S + 31) // 32 * 32 + 32 * rng.randint(0, 3)
        chunk = rng.choice([0, 0, 32, 96, 128, 512])
        if chunk and (S + chunk - 1) // chunk > 256:
            chunk = 0
        out.append((300 + i, S, max_s, chunk))
    return out


def _prefill_cases():
    rng = random.Random(5678)
    out = []
    for i in range(5):
        p0, T = rng.randint(0, 5000), rng.randint(1, 300)
        out.append((400 + i, p0, T, (p0 + T + 31) // 32 * 32 + 32 * rng.randint(0, 2)))
    return out


def _sparse_cases():
    rng = random.Random(9012)
    return [rng.randint(1, 32768) for _ in range(5)] + [1152, 1153]


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


@pytest.mark.parametrize("seed,S,max_s,chunk", _decode_cases())
def test_decode_random_shape(torch_gpu, orc, seed, S, max_s, chunk):
    from embla_attn import ops
    torch = torch_gpu
    say(f"random decode seed={seed} S={S} max_s={max_s} chunk={chunk}")
    c = synth.decode_int8_case(seed=seed, S=S)
    kc, vc = upload_int8_case(c, max_s)
    o = ops.decode_int8(dev(c["q"], torch.float16), kc, vc, S, max_s, 4, chunk=chunk, ws=ops.Workspace(max_s, 16))
    ref = orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    assert_close(f16_host(o), ref, what=f"decode S={S} chunk={chunk}")


@pytest.mark.parametrize("seed,p0,T,max_s", _prefill_cases())
def test_prefill_random_shape(torch_gpu, orc, seed, p0, T, max_s):
    from embla_attn import ops
    torch = torch_gpu
    say(f"random prefill seed={seed} p0={p0} T={T} max_s={max_s}")
    c = synth.prefill_case(seed=seed, p0=p0, T=T)
    kc = dev(layout.pack_region(c["K"], c["ks"], max_s, "k"))
    vc = dev(layout.pack_region(c["V"], c["vs"], max_s, "v"))
    q = dev(c["q"], torch.bfloat16)
    ops.kv_quant_append(dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16), T, p0, 4, kc, vc, max_s)
    a = ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, ws=ops.PrefillWorkspace(T, 16))
    b = ops.prefill_int8(q, kc, vc, T, p0, max_s, 4, ws=ops.PrefillWorkspace(T, 16, staged_p0=p0))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.view(torch.int16).cpu().numpy(), b.view(torch.int16).cpu().numpy())
    Kr, Ks = layout.unpack_region(kc.cpu().numpy(), 4, max_s, "k", np.uint16)
    Vr, Vs = layout.unpack_region(vc.cpu().numpy(), 4, max_s, "v", np.uint16)
    n = p0 + T
    ref = orc.prefill_int8(synth.bf16_val(c["q"]), Kr[:, :n], synth.f16_val(Ks[:, :n]), Vr[:, :n],
                           synth.f16_val(Vs[:, :n]), p0)
    assert_close(bf16_host(b), ref, what=f"prefill p0={p0} T={T}")


@pytest.fixture(scope="module")
def sparse_setup(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    c = synth.sparse_case(seed=3, ctx=32768)
    ws = ops.SparseWorkspace(32768, 16)
    args = [dev(c["q"], torch.float16), dev(c["qi"], torch.float16), dev(c["w"]), dev(c["ki"], torch.float16),
            dev(c["K"], torch.float16), dev(c["V"], torch.float16)]
    return c, ws, args


@pytest.mark.parametrize("S", _sparse_cases())
def test_sparse_layer_random_length(torch_gpu, orc, sparse_setup, S):
    from embla_attn import ops
    c, ws, args = sparse_setup
    say(f"random sparse layer S={S}")
    o = ops.sparse_layer_decode(*args, S, 32768, 4, ws)
    if S > 1152:
        sc = orc.index_scores(c["qi"], c["w"], c["ki"][:S - 128])
        sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
        np.testing.assert_array_equal(ws.selection().cpu().numpy().astype(np.uint32), sel)
        sel = sel.astype(np.int32)
    else:
        sel = np.arange(S, dtype=np.int32)
    ref = orc.decode_rows(synth.f16_val(c["q"]), synth.f16_val(c["K"]), synth.f16_val(c["V"]), sel)
    assert_close(f16_host(o), ref, what=f"sparse S={S}")
