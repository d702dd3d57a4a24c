"""The HIP path on the golden fixtures' inputs against their stored outputs (bit-exact for the
selection and the int8 bytes, max-abs 2e-3 + rel 1e-2 for attention outputs)."""
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, dev, f16_host, say, upload_int8_case
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def test_golden_c1_decode(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    say("golden c1 decode")
    c = synth.decode_int8_case(seed=0, S=1024)
    kc, vc = upload_int8_case(c, 1024)
    o = ops.decode_int8(dev(c["q"], torch.float16), kc, vc, 1024, 1024, 4, ws=ops.Workspace(1024, 16))
    assert_close(f16_host(o), load("c1_decode")["out"], what="c1")


def test_golden_c4_select(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    say("golden c4 select 4k")
    c = synth.sparse_case(seed=3, ctx=4096)
    g = load("c4_select_4k")
    sc = ops.index_scores(dev(c["qi"], torch.float16), dev(c["w"]), dev(c["ki"], torch.float16), 4096 - 128)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), g["scores"].view(np.uint32))
    idx = ops.select_topk(sc, 4096)
    np.testing.assert_array_equal(idx.cpu().numpy()[0].astype(np.uint32), g["sel"])


def test_golden_quant_rows(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    say("golden quant rows")
    g = load("quant_rows")
    max_s = 64
    x = g["x"].reshape(64, 1, 128)
    kc = torch.zeros(max_s * 128 + max_s * 4, dtype=torch.uint8, device="cuda")
    vc = torch.zeros_like(kc)
    ops.kv_quant_append(dev(x, torch.bfloat16), dev(x, torch.bfloat16), 64, 0, 1, kc, vc, max_s, scale_dtype=ops.F32)
    torch.cuda.synchronize()
    K, ks = layout.unpack_region(kc.cpu().numpy(), 1, max_s, "k", np.float32)
    np.testing.assert_array_equal(K[0], g["q"])
    np.testing.assert_array_equal(ks[0], g["scale"])


def test_golden_c5_prefill_small(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    say("golden c5 prefill small")
    c = synth.prefill_case(seed=4, p0=300, T=40)
    max_s = 352
    kc = dev(layout.pack_region(c["K"], c["ks"], max_s, "k"))
    vc = dev(layout.pack_region(c["V"], c["vs"], max_s, "v"))
    o = ops.prefill_full(dev(c["q"], torch.bfloat16), dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16),
                         kc, vc, 40, 300, max_s, 4)
    assert_close(bf16_host(o), load("c5_prefill_small")["out"], what="c5 small")


def test_golden_c2_window(torch_gpu):
    from embla_attn import ops
    torch = torch_gpu
    say("golden c2 window")
    g = synth.SplitMix64(1)
    K = synth.f16_bits(g.normal(4 * 300 * 128)).reshape(4, 300, 128)
    V = synth.f16_bits(g.normal(4 * 300 * 128)).reshape(4, 300, 128)
    q = synth.f16_bits(g.normal(16 * 128)).reshape(16, 128)
    R, W = 512, 96
    rows = np.zeros((4, R, 128), np.uint16)
    rows[:, :299] = K[:, :299]
    kring = dev(layout.pack_ring16(rows, "k"))
    rows[:, :299] = V[:, :299]
    vring = dev(layout.pack_ring16(rows, "v"))
    o = ops.sliding_decode(dev(q, torch.float16), dev(K[:, 299].copy(), torch.float16), dev(V[:, 299].copy(), torch.float16),
                           kring, vring, 299, W, R, 4, ws=ops.Workspace(R, 16))
    assert_close(f16_host(o), load("c2_window_small")["out"], what="c2 window")
