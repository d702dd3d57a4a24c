"""The oracle's sampling tail (misc.metal:83-128 argmax, 164-298 sample), pinned by what the
mathematics fixes and by the reference's own statistical test (SampleTests.swift:7-58): the softcap
over every finite bf16 input against an independent numpy evaluation and its symmetry, monotony and
saturation; the greedy token against numpy's first argmax; the draw's frequencies against the
analytic top-p nucleus distribution within 5 sigma, and its limits (a vanishing top-p is the argmax,
a draw is a function of seed and position)."""
import numpy as np
import pytest

from embla_attn import synth


def all_finite_bf16():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = synth.bf16_val(bits)
    return bits[np.isfinite(vals)], vals[np.isfinite(vals)]


def np_bf(x):
    return synth.bf16_val(synth.bf16_bits(np.asarray(x, np.float32)))


def np_softcap(l):
    """bf(bf(tanh(bf(bf(l) / 15))) * 15), tanh in fp64 rounded once, vectorised."""
    y = np_bf(np_bf(l) / np.float32(15))
    t = np.tanh(y.astype(np.float64)).astype(np.float32)
    return np_bf(np_bf(t) * np.float32(15))


def test_softcap_every_bf16(orc):
    _, v = all_finite_bf16()
    got = orc.softcap(v)
    np.testing.assert_array_equal(got, np_softcap(v))
    # odd, non-decreasing, bounded by 15, saturating, the identity near 0 (to a bf16 step)
    np.testing.assert_array_equal(orc.softcap(-v), -got)
    order = np.argsort(v, kind="stable")
    assert (np.diff(got[order]) >= 0).all()
    assert np.abs(got).max() == 15.0
    assert (orc.softcap(np.array([200.0, 1e4, 3e38], np.float32)) == 15.0).all()
    small = v[(np.abs(v) < 0.5) & (v != 0)]
    c = orc.softcap(small)
    assert (np.abs(c - small) <= np.abs(small) * 2.0 ** -7 + 1e-30).all()
    assert orc.softcap(np.zeros(1, np.float32))[0] == 0.0


def test_argmax_first_of_largest(orc):
    g = np.random.default_rng(3)
    for V in (1, 7, 1000, 65536):
        lg = (g.standard_normal(V) * 4).astype(np.float32)
        assert orc.argmax(lg) == int(np.argmax(np_softcap(lg)))
    # ties after the softcap: distinct raw logits that cap to the same bf16 -> the first index
    lg = np.zeros(5000, np.float32)
    lg[1234] = 300.0
    lg[77] = 200.0   # both cap to 15
    assert orc.argmax(lg) == 77


def nucleus(capped, T, top_p):
    w = np.exp((capped.astype(np.float64) - capped.max()) / T)
    z = w.sum()
    keep, mass = 0, 0.0
    while mass < top_p * z and keep < len(w):
        mass += w[keep]
        keep += 1
    return w, keep, mass


@pytest.mark.parametrize("T,top_p", [(1.0, 1.0), (0.6, 0.9), (1.0, 0.95), (3.0, 0.9)])
def test_sample_distribution(orc, T, top_p):
    """SampleTests.swift:7-58 on the oracle: ten likely tokens over a flat tail."""
    V, n = 65536, 1500
    capped = np.array([3.0 - 0.3 * i if i < 10 else -10.0 for i in range(V)], np.float32)
    raw = (15 * np.arctanh(capped.astype(np.float64) / 15)).astype(np.float32)
    tok, _ = orc.sample_many(raw, 0, n, 1.0 / T, top_p, 1234)
    counts = np.bincount(np.minimum(tok, 10), minlength=11)
    w, keep, mass = nucleus(capped, T, top_p)
    for i in range(10):
        q = w[i] / mass if i < keep else 0.0
        f = counts[i] / n
        sd = np.sqrt(q * (1 - q) / n)
        assert abs(f - q) < 5 * sd + 1e-9, (i, f, q)
    if keep <= 10:
        assert counts[keep:].sum() == 0, "draws outside the nucleus"


def test_sample_limits(orc):
    g = np.random.default_rng(5)
    lg = (g.standard_normal(20000) * 3).astype(np.float32)
    want = orc.argmax(lg)
    # a vanishing top-p keeps only the largest
    tok, _ = orc.sample_many(lg, 0, 30, 1.0, 1e-7, 9)
    assert (tok == want).all()
    # a draw is a function of (logits, T, top-p, seed, position)
    a, _ = orc.sample_many(lg, 100, 20, 0.8, 0.9, 11)
    b = np.array([orc.sample(lg, 100 + k, 0.8, 0.9, 11)[0] for k in range(20)])
    np.testing.assert_array_equal(a, b)
    c, _ = orc.sample_many(lg, 100, 20, 0.8, 0.9, 12)
    assert (a != c).any()


def test_mix32_bijective_on_sample(orc):
    """The hash is a bijection on 32-bit words (xorshifts and odd multiplies); 0 is fixed."""
    f = orc.lib().orc_mix32
    assert f(0) == 0
    xs = np.random.default_rng(1).integers(0, 2**32, 20000, dtype=np.uint64)
    ys = {f(int(x)) for x in xs}
    assert len(ys) == len(set(int(x) for x in xs))


def _lowbias32_inverse(y):
    """The inverse of Wellons' lowbias32 (hash-prospector, 2018), written from its published
    inverse: undo the xorshifts (x ^= x >> 16 is an involution; x ^= x >> 15 is undone by
    x ^= x >> 15 ^ x >> 30) and multiply by the published inverses of the two odd constants
    (0x43021123 = 0x846ca68b^-1, 0x1d69e2a5 = 0x7feb352d^-1 mod 2^32)."""
    M = 0xFFFFFFFF
    y ^= y >> 16
    y = (y * 0x43021123) & M
    y ^= (y >> 15) ^ (y >> 30)
    y = (y * 0x1d69e2a5) & M
    y ^= y >> 16
    return y


def test_mix32_is_lowbias32(orc):
    """The sampler's hash (misc.metal:186-191) is Wellons' lowbias32; the oracle's restatement
    inverts exactly under that hash's published inverse, which pins both multipliers (a changed
    or transposed constant fails) independently of the oracle's own text."""
    f = orc.lib().orc_mix32
    xs = np.random.default_rng(2).integers(0, 2**32, 5000, dtype=np.uint64)
    for x in [0, 1, 2, 0x80000000, 0xFFFFFFFF] + [int(v) for v in xs]:
        assert _lowbias32_inverse(f(x)) == x, hex(x)
