"""Sparse-layer batched prefill (config C5 sparse): per-row ReLU² index scores, the exact top-1024 +
latest 128 (checked bit for bit against the oracle's select_keys of the oracle's spec scores), and
the attention over those rows of the row-major int8 cache (against the oracle's prefill)."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, bf16_host, chunk_rows, dev, say
from embla_attn import synth
from test_gpu_prefill import quant_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def pack_rows(rows, scales_bits, max_s):
    """Row-major int8 region: rows [n_kv][max_s][128] int8, then fp16 scales [n_kv][max_s]."""
    n_kv, p0, _ = rows.shape
    r = np.zeros((n_kv, max_s, 128), np.int8)
    r[:, :p0] = rows
    s = np.zeros((n_kv, max_s), np.uint16)
    s[:, :p0] = scales_bits
    return np.concatenate([r.reshape(-1).view(np.uint8), s.reshape(-1).view(np.uint8)])


def oracle_cache(orc, c):
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


def run(torch, c):
    from embla_attn import ops
    p0, T = c["p0"], c["T"]
    max_s = ((p0 + T + 31) // 32) * 32
    kc = dev(pack_rows(c["K"], c["ks"], max_s))
    vc = dev(pack_rows(c["V"], c["vs"], max_s))
    idx = torch.zeros((T, 1152), dtype=torch.int32, device="cuda")
    ws = ops.SparsePrefillWorkspace(T, p0)
    o, _ = ops.prefill_sparse(dev(c["q"], torch.bfloat16), dev(c["kn"], torch.bfloat16), dev(c["vn"], torch.bfloat16),
                              dev(c["qi"], torch.float16), dev(c["w"]), dev(c["ki"], torch.float16), kc, vc, T, p0,
                              max_s, c["n_kv"], ws, idx=idx)
    return bf16_host(o), idx.cpu().numpy().astype(np.uint32), kc, max_s


def check_rows(orc, c, got, idx, rows, cache):
    K, ks, V, vs = cache
    p0 = c["p0"]
    for t in rows:
        S = p0 + t + 1
        if S > 1152:
            sc = orc.index_scores(c["qi"][t], c["w"][t], c["ki"][:S - 128])
            sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
            np.testing.assert_array_equal(idx[t], sel, err_msg=f"row {t}: selection")
        else:
            sel = np.arange(S, dtype=np.uint32)
        ref = orc.prefill_int8(synth.bf16_val(c["q"][t:t + 1]), K, ks, V, vs, S - 1, rows_sel=sel[None])
        assert_close(got[t], ref[0], what=f"row {t}")


@pytest.mark.parametrize("p0,T", [(1500, 64), (1100, 100), (3000, 40), (1300, 1), (1300, 2)])
def test_prefill_sparse_small(torch_gpu, orc, p0, T):
    say(f"prefill sparse p0={p0} T={T}")
    c = synth.sparse_prefill_case(seed=4, p0=p0, T=T)
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_gq8(torch_gpu, orc):
    """8 query heads a kv head (32 over 4): the gather kernel's GQ = 8 variant."""
    p0, T = 1400, 48
    say("prefill sparse GQ 8")
    c = synth.sparse_prefill_case(seed=8, p0=p0, T=T, n_q=32, n_kv=4)
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_ties(torch_gpu, orc):
    """Duplicated index keys give equal spec scores around the threshold: ties by lower index."""
    p0, T = 2000, 24
    c = synth.sparse_prefill_case(seed=5, p0=p0, T=T)
    ki = c["ki"]
    ki[700:1400] = ki[0:700]            # every key of [0, 700) appears twice
    ki[1400:1900:5] = ki[3]
    say("prefill sparse ties")
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_all_equal_band_overflow(torch_gpu, orc):
    """Identical index keys: every score is equal, the band holds every key (the unlisted path)."""
    p0, T = 1600, 3
    c = synth.sparse_prefill_case(seed=6, p0=p0, T=T)
    c["ki"][:] = c["ki"][0]
    say("prefill sparse all equal")
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_zero_ties_band_overflow(torch_gpu, orc):
    """Most index keys zero: their scores are exactly 0 and fewer than 1024 keys score above 0, so
    the 1024th score is a tie at 0 among ~3800 keys (a band too large to list: the overflow kernel),
    taken by lower index."""
    p0, T = 4000, 6
    c = synth.sparse_prefill_case(seed=9, p0=p0, T=T)
    c["ki"][150:3950] = 0
    say("prefill sparse zero ties")
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_small_scores_band_overflow(torch_gpu, orc):
    """Most index keys 1000x smaller than the rest: their distinct scores all lie within the error
    bound of the 1024th (set by the largest key norm), so the band overflows and is ranked exactly
    by the overflow kernel; a few mid-sized keys make the selection mix both kinds."""
    p0, T = 3000, 5
    c = synth.sparse_prefill_case(seed=10, p0=p0, T=T)
    ki = synth.f16_val(c["ki"])
    ki[:p0 - 200] *= 1e-3
    ki[500:p0 - 200:40] *= 30.0
    c["ki"] = synth.f16_bits(ki)
    say("prefill sparse small scores")
    got, idx, _, _ = run(torch_gpu, c)
    check_rows(orc, c, got, idx, range(T), oracle_cache(orc, c))


def test_prefill_sparse_c5_size_all_rows(torch_gpu, orc):
    """C5 sparse at full size: 2048 rows after 30720 cached positions. Every row's selection
    against the SHA-256 of the oracle's (tests/golden/c5_sparse_selection.npz, same seeded
    inputs); attention outputs and selections re-derived on the edge rows of every 32-row tile."""
    import hashlib
    from pathlib import Path
    p0, T = 30720, 2048
    say("prefill sparse C5 size")
    c = synth.sparse_prefill_case(seed=4, p0=p0, T=T)
    got, idx, _, _ = run(torch_gpu, c)
    want = np.load(Path(__file__).resolve().parent / "golden" / "c5_sparse_selection.npz", allow_pickle=False)
    gotsha = np.stack([np.frombuffer(hashlib.sha256(idx[t].astype(np.uint32).tobytes()).digest(), np.uint8)
                       for t in range(T)])
    bad = np.nonzero((gotsha != want["row_sha256"]).any(1))[0]
    assert bad.size == 0, f"{bad.size} of {T} rows select differently, first rows {bad[:8].tolist()}"
    check_rows(orc, c, got, idx, chunk_rows(T), oracle_cache(orc, c))
