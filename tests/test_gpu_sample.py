"""The sampling tail on the GPU (embla_argmax, embla_sample; misc.metal:86-128, 196-298) against the
oracle: the softcap bit for bit over every finite bf16 logit, the greedy token and the reference's
outputs (greedy[pos], token[pos + 1] past the prompt, the polled word), the draw token for token on
the cases whose decisions are not within floating-point error of a boundary (the oracle flags
those), and the draw's frequencies against the nucleus distribution (SampleTests.swift:7-58)."""
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


def test_softcap_every_bf16(torch_gpu, orc):
    """The draw's first kernel writes the capped row as bf16 at the workspace's start."""
    from embla_attn import ops
    torch = torch_gpu
    say("sample softcap, every bf16")
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = synth.bf16_val(bits)
    v = np.where(np.isnan(v), np.float32(0), v).astype(np.float32)
    st = ops.SampleState(65536, 8)
    ops.sample(dev(v), st, 0, 1.0, 1.0, 1)
    torch.cuda.synchronize()
    got = st.ws[:2 * 65536].cpu().numpy().view(np.uint16)
    want = synth.bf16_bits(orc.softcap(v))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} inputs differ, first bf16 input {bits[bad[0]]:#06x}"


@pytest.mark.parametrize("V", [65536, 1000, 65533, 1])
def test_argmax_outputs(torch_gpu, orc, V):
    from embla_attn import ops
    torch = torch_gpu
    say(f"argmax V={V}")
    g = np.random.default_rng(V)
    st = ops.SampleState(V, 64)
    for pos, prompt in [(5, 10), (9, 10), (40, 10)]:
        lg = (g.standard_normal(V) * 5).astype(np.float32)
        if V > 2000:   # a tie after the softcap in two blocks: the first index wins
            lg[1500] = 250.0
            lg[V - 3] = 900.0
        st.tokens.fill_(-1)
        ops.argmax(dev(lg), st, pos, prompt)
        torch.cuda.synchronize()
        want = orc.argmax(lg)
        gr = st.greedy.cpu().numpy().view(np.uint32)
        tk = st.tokens.cpu().numpy()
        assert gr[1 + pos] == want
        assert gr[0] == ((pos + 1) << 16) | want
        if pos + 1 >= prompt:
            assert tk[pos + 1] == want
        else:
            assert (tk == -1).all(), "a token written inside the prompt"


def logits_row(seed, V, kind, a):
    """'normal': N(0, a^2) logits (flat or saturated: the bisection over all tokens); 'hot': a
    tokens U(2, 8) over an N(-6, 1) background (peaked: few candidates)."""
    g = np.random.default_rng(seed)
    if kind == "normal":
        return (g.standard_normal(V) * a).astype(np.float32)
    lg = (g.standard_normal(V) - 6).astype(np.float32)
    hot = g.choice(V, int(a), replace=False)
    lg[hot] = g.uniform(2, 8, int(a)).astype(np.float32)
    return lg


CASES = [  # (seed, V, kind, a, T, top_p)
    (1, 65536, "normal", 4.0, 1.0, 0.9), (2, 65536, "normal", 6.0, 0.7, 0.95),
    (3, 65536, "normal", 1.0, 1.0, 0.9), (4, 65536, "normal", 0.5, 2.0, 0.8),
    (5, 65536, "normal", 3.0, 1.0, 1.0), (6, 50000, "normal", 5.0, 0.8, 0.5),
    (7, 65536, "normal", 20.0, 1.0, 0.9), (8, 4096, "normal", 2.0, 1.5, 0.7),
    (9, 65536, "normal", 8.0, 0.3, 0.9),
    (10, 65536, "hot", 300, 1.0, 0.9),     # 316 candidates
    (11, 65536, "hot", 1500, 0.8, 0.95),   # 1500 candidates
    (12, 65536, "hot", 40, 1.2, 0.6),      # 6817 candidates: all tokens
    (10, 65536, "hot", 300, 1.0, 0.999),   # candidates short of top-p's mass: all tokens
]


@pytest.mark.parametrize("seed,V,kind,a,T,top_p", CASES)
def test_sample_matches_oracle(torch_gpu, orc, seed, V, kind, a, T, top_p):
    from embla_attn import ops
    torch = torch_gpu
    say(f"sample seed={seed} V={V} {kind} {a} T={T} top_p={top_p}")
    lg = logits_row(seed, V, kind, a)
    n = 40
    want, fragile = orc.sample_many(lg, 0, n, 1.0 / T, top_p, 4242 + seed)
    st = ops.SampleState(V, n + 2)
    x = dev(lg)
    for pos in range(n):
        ops.sample(x, st, pos, 1.0 / T, top_p, 4242 + seed)
    torch.cuda.synchronize()
    got = st.greedy.cpu().numpy().view(np.uint32)[1:1 + n]
    ok = ~fragile
    assert ok.sum() >= n // 2, "too few decisive cases to compare"
    np.testing.assert_array_equal(got[ok], want[ok])


def test_sample_distribution(torch_gpu):
    """SampleTests.swift:7-58: ten likely tokens over a flat tail, 6000 positions a setting."""
    from embla_attn import ops
    torch = torch_gpu
    V, n = 65536, 6000
    capped = np.array([3.0 - 0.3 * i if i < 10 else -10.0 for i in range(V)], np.float32)
    raw = (15 * np.arctanh(capped.astype(np.float64) / 15)).astype(np.float32)
    x = dev(raw)
    st = ops.SampleState(V, n + 2)
    for T, top_p in [(1.0, 1.0), (0.6, 0.9), (1.0, 0.95), (3.0, 0.9)]:
        say(f"sample distribution T={T} top_p={top_p}")
        for pos in range(n):
            ops.sample(x, st, pos, 1.0 / T, top_p, 1234)
        torch.cuda.synchronize()
        got = st.greedy.cpu().numpy().view(np.uint32)[1:1 + n]
        counts = np.bincount(np.minimum(got, 10), minlength=11)
        w = np.exp((capped.astype(np.float64) - 3.0) / T)
        z = w.sum()
        keep, mass = 0, 0.0
        while mass < top_p * z and keep < V:
            mass += w[keep]
            keep += 1
        for i in range(10):
            q = w[i] / mass if i < keep else 0.0
            f = counts[i] / n
            sd = np.sqrt(q * (1 - q) / n)
            assert abs(f - q) < 5 * sd + 1e-9, (T, top_p, i, f, q)
        if keep <= 10:
            assert counts[keep:].sum() == 0, "draws outside the nucleus"


def test_sample_vanishing_top_p_is_argmax(torch_gpu, orc):
    from embla_attn import ops
    torch = torch_gpu
    g = np.random.default_rng(11)
    lg = (g.standard_normal(65536) * 3).astype(np.float32)
    st = ops.SampleState(65536, 8)
    for pos in range(4):
        ops.sample(dev(lg), st, pos, 1.0, 1e-7, pos)
    torch.cuda.synchronize()
    assert (st.greedy.cpu().numpy().view(np.uint32)[1:5] == orc.argmax(lg)).all()
