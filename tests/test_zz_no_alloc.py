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
