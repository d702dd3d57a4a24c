"""embla_decode_int8_noalloc (partials in the library's own device array, nothing allocated)
against embla_decode_int8 with a caller workspace: the same kernels, so the outputs are equal bit
for bit; two calls in a row, the second smaller, and both against the oracle."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, dev, f16_host, say, upload_int8_case
from embla_attn import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def test_noalloc_matches_workspace_decode(torch_gpu, orc):
    from embla_attn import ops
    torch = torch_gpu
    for S, seed, chunk in [(32768, 2, 0), (5000, 11, 0), (1000, 5, 128), (40, 7, 0)]:
        say(f"decode noalloc S={S} seed={seed} chunk={chunk}")
        c = synth.decode_int8_case(seed=seed, S=S)
        max_s = (S + 31) // 32 * 32
        kc, vc = upload_int8_case(c, max_s)
        q = dev(c["q"], torch.float16)
        ws = ops.Workspace(max_s, c["n_q"])
        want = ops.decode_int8(q, kc, vc, S, max_s, c["n_kv"], chunk=chunk, ws=ws)
        got = ops.decode_int8_noalloc(q, kc, vc, S, max_s, c["n_kv"], chunk=chunk)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())
        ref = orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
        assert_close(f16_host(got), ref, what=f"noalloc S={S}")


def test_noalloc_under_graph_capture(torch_gpu, orc):
    """The callers it is for: a decode captured in a HIP graph with no allocation inside. Replayed
    three times with eager calls (on the same device array) and a new q between replays; every
    replay equals the eager call on the same inputs bit for bit."""
    from embla_attn import ops
    torch = torch_gpu
    S = 20000
    say(f"decode noalloc graph S={S}")
    c = synth.decode_int8_case(seed=12, S=S)
    max_s = (S + 31) // 32 * 32
    kc, vc = upload_int8_case(c, max_s)
    q = dev(c["q"], torch.float16)
    out = torch.empty((16, 128), dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        ops.decode_int8_noalloc(q, kc, vc, S, max_s, 4, out=out)   # first call on the device: outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.decode_int8_noalloc(q, kc, vc, S, max_s, 4, out=out)
    gen = torch.Generator(device="cuda").manual_seed(5)
    for r in range(3):
        q.copy_(torch.randn(16, 128, generator=gen, device="cuda").half())
        ops.decode_int8_noalloc(q, kc, vc, 5000, max_s, 4)   # eager work on the same array between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = ops.decode_int8_noalloc(q, kc, vc, S, max_s, 4)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy(),
                                      err_msg=f"replay {r}")
    ref = orc.decode_int8(f16_host(q), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    assert_close(f16_host(out), ref, what="noalloc graph replay")
