"""int8 quantise-and-append is bit-exact with the oracle (write_row8 / kv_append semantics)."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import dev, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def quant_ref(orc, x_rows, norm, round_bf):
    q = np.empty(x_rows.shape, np.int8)
    s = np.empty(x_rows.shape[:-1], np.float32)
    for idx in np.ndindex(*x_rows.shape[:-1]):
        q[idx], s[idx] = orc.quant_row(x_rows[idx], norm=norm, round_bf=round_bf)
    return q, s


@pytest.mark.parametrize("T,p0", [(2048, 30720), (1, 100), (13, 5), (8, 16), (37, 1003)])
@pytest.mark.parametrize("mode", ["config", "reference"])
def test_kv_quant_append_bit_exact(torch_gpu, orc, T, p0, mode):
    from embla_attn import ops
    torch = torch_gpu
    say(f"kv quant append mode={mode} T={T} p0={p0}")
    n_kv = 4 if mode == "config" else 2
    max_s = 32768
    g = synth.SplitMix64(4 + T)
    k = synth.bf16_bits(g.normal(T * n_kv * 128) * 1.5).reshape(T, n_kv, 128)
    v = synth.bf16_bits(g.normal(T * n_kv * 128)).reshape(T, n_kv, 128)
    if T > 3:
        k[2] = 0  # an all-zero row: zeros and scale 0
    sdt = np.uint16 if mode == "config" else np.float32
    # pre-fill the regions with a pattern: positions outside [p0, p0+T) must keep it
    fill = (np.arange(n_kv * max_s * 128) % 251 - 125).astype(np.int8).reshape(n_kv, max_s, 128)
    sfill = np.full((n_kv, max_s), 7, sdt)
    kc = dev(layout.pack_region(fill, sfill, max_s, "k"))
    vc = dev(layout.pack_region(fill, sfill, max_s, "v"))
    ops.kv_quant_append(dev(k, torch.bfloat16), dev(v, torch.bfloat16), T, p0, n_kv, kc, vc, max_s,
                        scale_dtype=0 if mode == "config" else 2, norm_k=mode == "reference")
    torch.cuda.synchronize()
    Kr, Ks = layout.unpack_region(kc.cpu().numpy(), n_kv, max_s, "k", sdt)
    Vr, Vs = layout.unpack_region(vc.cpu().numpy(), n_kv, max_s, "v", sdt)
    kf = synth.bf16_val(k).transpose(1, 0, 2)
    vf = synth.bf16_val(v).transpose(1, 0, 2)
    qk, sk = quant_ref(orc, kf, norm=mode == "reference", round_bf=True)
    qv, sv = quant_ref(orc, vf, norm=False, round_bf=True)
    sl = slice(p0, p0 + T)
    np.testing.assert_array_equal(Kr[:, sl], qk)
    np.testing.assert_array_equal(Vr[:, sl], qv)
    if mode == "config":
        np.testing.assert_array_equal(Ks[:, sl], synth.f16_bits(sk))
        np.testing.assert_array_equal(Vs[:, sl], synth.f16_bits(sv))
    else:
        np.testing.assert_array_equal(Ks[:, sl], sk)
        np.testing.assert_array_equal(Vs[:, sl], sv)
    # untouched neighbours
    for a, b in ((Kr, fill), (Vr, fill)):
        np.testing.assert_array_equal(a[:, max(0, p0 - 9):p0], b[:, max(0, p0 - 9):p0])
        np.testing.assert_array_equal(a[:, p0 + T:p0 + T + 9], b[:, p0 + T:p0 + T + 9])
