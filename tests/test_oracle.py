"""Pins the C oracle (oracle/oracle.c) without the reference, which cannot run here (Swift +
Metal) and ships no attention golden vectors: against independent numpy fp64 brute force, closed
forms, invariants and special cases chosen so a dropped term, wrong index or sign fails."""
import numpy as np
import pytest

from embla_attn import synth

pytestmark = []


def np_decode(q, K, ks, V, vs, weights=0):
    """fp64 brute force of decode attention over dequantised rows."""
    n_q = q.shape[0]
    n_kv = K.shape[0]
    gq = n_q // n_kv
    out = np.zeros((n_q, 128))
    for h in range(n_q):
        kv = h // gq
        Kd = K[kv].astype(np.float64) * ks[kv][:, None]
        Vd = V[kv].astype(np.float64) * vs[kv][:, None]
        s = Kd @ q[h].astype(np.float64) / np.sqrt(128.0)
        if weights == 0:
            p = np.exp(s - s.max())
            out[h] = p @ Vd / p.sum()
        else:
            w = np.maximum(s, 0) ** 2
            out[h] = w @ Vd / (np.sqrt(128.0) + w.sum())
    return out


# ------------------------------------------------------------------ element conversions
def test_f16_bf16_conversions(orc):
    g = synth.SplitMix64(11)
    x = (g.normal(4000) * np.exp(g.normal(4000) * 4)).astype(np.float32)
    for v in x[:2000]:
        assert orc.lib().orc_f32_to_f16(float(v)) == synth.f16_bits(np.float32(v))
        assert orc.lib().orc_f32_to_bf16(float(v)) == synth.bf16_bits(np.float32(v))
    bits = np.arange(0, 65536, 37, dtype=np.uint16)
    finite = np.isfinite(bits.view(np.float16))
    got = np.array([orc.lib().orc_f16_to_f32(int(b)) for b in bits[finite]], np.float32)
    np.testing.assert_array_equal(got, bits[finite].view(np.float16).astype(np.float32))


# ------------------------------------------------------------------ int8 quantisation
def np_quant(x, round_bf):
    x = np.asarray(x, np.float32)
    if round_bf:
        x = synth.bf16_val(synth.bf16_bits(x))
    a = np.float32(np.max(np.abs(x)))
    inv = np.float32(127.0) / a if a > 0 else np.float32(0)
    return np.rint(x * inv).astype(np.int8), np.float32(a / np.float32(127.0))


def test_quant_row_definition(orc):
    g = synth.SplitMix64(5)
    for i in range(200):
        x = (g.normal(128) * (0.01 + 10 * g.uniform(1)[0])).astype(np.float32)
        for rb in (False, True):
            q, s = orc.quant_row(x, round_bf=rb)
            q2, s2 = np_quant(x, rb)
            np.testing.assert_array_equal(q, q2)
            assert np.float32(s) == s2


def test_quant_row_special_cases(orc):
    q, s = orc.quant_row(np.zeros(128))
    assert not q.any() and s == 0.0
    x = np.linspace(-3, 1, 128).astype(np.float32)
    q, s = orc.quant_row(x)
    assert q[0] == -127 and q.max() < 127 and np.float32(s) == np.float32(3.0) / np.float32(127)
    # exact halves round to even: a = 127 makes q = x
    x = np.zeros(128, np.float32)
    x[0] = 127.0
    x[1:6] = [0.5, 1.5, 2.5, -0.5, -1.5]
    q, _ = orc.quant_row(x)
    assert list(q[:6]) == [127, 0, 2, 2, 0, -2]


def test_quant_row_norm_matches_fp64(orc):
    """RMS-normed K rows (kv_append): bytes agree with an fp64 norm except at rounding
    boundaries, where they differ by one."""
    g = synth.SplitMix64(6)
    diffs = 0
    for i in range(100):
        x = synth.bf16_val(synth.bf16_bits(g.normal(128) * 3)).astype(np.float32)
        q, s = orc.quant_row(x, norm=True, round_bf=True)
        r = 1.0 / np.sqrt((x.astype(np.float64) ** 2).sum() / 128 + 1.1920929e-07)
        y = synth.bf16_val(synth.bf16_bits((x * r).astype(np.float32))).astype(np.float64)
        a = np.abs(y).max()
        q64 = np.rint(y * 127 / a)
        assert np.abs(q.astype(np.int64) - q64).max() <= 1
        diffs += int((q != q64).sum())
        assert abs(s - a / 127) <= 1e-6 * a
    assert diffs < 100 * 128 * 0.01


# ------------------------------------------------------------------ decode
@pytest.mark.parametrize("weights", [0, 1])
@pytest.mark.parametrize("n_kv", [4, 2])
def test_decode_int8_vs_fp64(orc, weights, n_kv):
    c = synth.decode_int8_case(seed=7, S=300, n_kv=n_kv)
    q = synth.f16_val(c["q"])
    ks, vs = synth.f16_val(c["ks"]), synth.f16_val(c["vs"])
    if weights == 1:
        q = q * 8  # ReLU² needs positive scores of some size to be non-trivial
    got = orc.decode_int8(q, c["K"], ks, c["V"], vs, weights=weights)
    ref = np_decode(q, c["K"], ks, c["V"], vs, weights)
    np.testing.assert_allclose(got, ref, atol=2e-6, rtol=1e-5)


def test_decode_int8_closed_forms(orc):
    rng = np.random.default_rng(0)
    n_kv, S = 4, 64
    q = rng.standard_normal((16, 128)).astype(np.float32)
    V = rng.integers(-127, 128, (n_kv, S, 128)).astype(np.int8)
    vs = rng.uniform(0.005, 0.02, (n_kv, S)).astype(np.float32)
    # identical keys: softmax is uniform, the output is the mean of the dequantised values
    K = np.repeat(rng.integers(-127, 128, (n_kv, 1, 128)).astype(np.int8), S, axis=1)
    ks = np.full((n_kv, S), 0.01, np.float32)
    out = orc.decode_int8(q, K, ks, V, vs)
    mean = (V.astype(np.float64) * vs[..., None]).mean(axis=1)
    np.testing.assert_allclose(out, np.repeat(mean, 4, axis=0), atol=1e-6)
    # ReLU² with every score negative: all weights zero, output exactly zero
    K2 = np.full((n_kv, S, 128), -100, np.int8)
    out2 = orc.decode_int8(np.abs(q), K2, ks, V, vs, weights=1)
    assert not out2.any()
    # GQA 1:1 equals MHA: query head h reads kv head h
    c = synth.decode_int8_case(seed=9, S=50, n_q=4, n_kv=4)
    o = orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    for h in range(4):
        oh = orc.decode_int8(synth.f16_val(c["q"])[h:h + 1], c["K"][h:h + 1], synth.f16_val(c["ks"])[h:h + 1],
                             c["V"][h:h + 1], synth.f16_val(c["vs"])[h:h + 1])
        np.testing.assert_allclose(o[h], oh[0], atol=1e-7)


def test_decode_scores_and_selected_rows(orc):
    c = synth.decode_int8_case(seed=3, S=200, n_q=16, n_kv=2)
    q = synth.f16_val(c["q"])
    ks, vs = synth.f16_val(c["ks"]), synth.f16_val(c["vs"])
    out, sc = orc.decode_int8(q, c["K"], ks, c["V"], vs, weights=1, want_scores=True)
    for kv in range(2):
        dots = c["K"][kv].astype(np.float64) @ q[kv * 8:(kv + 1) * 8].T.astype(np.float64)
        np.testing.assert_allclose(sc[kv], (dots * ks[kv][:, None]).max(1), rtol=1e-5, atol=1e-5)
    # SEL: attending a subset equals attending the gathered rows as a cache of their own
    rows = np.stack([np.sort(np.random.default_rng(kv).choice(200, 37, replace=False)) for kv in range(2)])
    got = orc.decode_int8(q, c["K"], ks, c["V"], vs, weights=0, rows=rows.astype(np.uint32), n_sel=37)
    Kg = np.stack([c["K"][kv][rows[kv]] for kv in range(2)])
    Vg = np.stack([c["V"][kv][rows[kv]] for kv in range(2)])
    ksg = np.stack([ks[kv][rows[kv]] for kv in range(2)])
    vsg = np.stack([vs[kv][rows[kv]] for kv in range(2)])
    np.testing.assert_allclose(got, np_decode(q, Kg, ksg, Vg, vsg, 0), atol=2e-6, rtol=1e-5)


@pytest.mark.parametrize("weights", [0, 1])
def test_decode_f32_vs_fp64_and_int8(orc, weights):
    """The bf16-cache decode (attn_full / attn_sparse without KV8): fp64 brute force on bf16 rows;
    bit for bit the int8 decode's arithmetic on integer-valued rows with unit scales; scores the
    raw q·k maximum; SEL equals the gathered rows."""
    g = synth.SplitMix64(21)
    n_kv, S = 2, 260
    K = synth.bf16_val(synth.bf16_bits(g.normal(n_kv * S * 128))).reshape(n_kv, S, 128)
    V = synth.bf16_val(synth.bf16_bits(g.normal(n_kv * S * 128))).reshape(n_kv, S, 128)
    q = synth.bf16_val(synth.bf16_bits(g.normal(16 * 128) * (3.0 if weights else 1.0))).reshape(16, 128)
    ones = np.ones((n_kv, S), np.float32)
    got, sc = orc.decode_f32(q, K, V, weights=weights, want_scores=True)
    np.testing.assert_allclose(got, np_decode(q, K, ones, V, ones, weights), atol=2e-6, rtol=1e-5)
    for kv in range(n_kv):
        dots = K[kv].astype(np.float64) @ q[kv * 8:(kv + 1) * 8].T.astype(np.float64)
        np.testing.assert_allclose(sc[kv], dots.max(1), rtol=1e-5, atol=1e-4)
    Ki = g.int8(n_kv * S * 128).reshape(n_kv, S, 128)
    Vi = g.int8(n_kv * S * 128).reshape(n_kv, S, 128)
    qi = q / 16
    np.testing.assert_array_equal(orc.decode_f32(qi, Ki.astype(np.float32), Vi.astype(np.float32), weights=weights),
                                  orc.decode_int8(qi, Ki, ones, Vi, ones, weights=weights))
    rows = np.stack([np.sort(np.random.default_rng(kv).choice(S, 41, replace=False)) for kv in range(n_kv)])
    gs = orc.decode_f32(q, K, V, weights=weights, rows=rows.astype(np.uint32))
    Kg = np.stack([K[kv][rows[kv]] for kv in range(n_kv)])
    Vg = np.stack([V[kv][rows[kv]] for kv in range(n_kv)])
    np.testing.assert_array_equal(gs, orc.decode_f32(q, Kg, Vg, weights=weights))


# ------------------------------------------------------------------ selection
def np_select(sc, S, topk=1024, recent=128):
    n = S - recent
    order = np.lexsort((np.arange(n), -sc[:n].astype(np.float64)))
    return set(order[:topk].tolist())


def verify_selection(idx, sc, S, topk=1024, recent=128):
    """Engine.verifySelection (Engine.swift:1115-1131)."""
    n = S - recent
    row = [int(x) for x in idx]
    assert len(set(row)) == topk + recent
    assert row[topk:] == list(range(n, S))
    s = sc[:n]
    kth = np.sort(s)[::-1][topk - 1]
    assert all(r < n and s[r] >= kth for r in row[:topk])
    assert (s > kth).sum() <= topk


@pytest.mark.parametrize("case", ["random", "ties", "all_equal", "negative"])
def test_select_keys(orc, case):
    S = 5000
    g = synth.SplitMix64(21)
    sc = g.normal(S).astype(np.float32)
    if case == "ties":
        sc = np.round(sc * 4) / 4  # heavy ties at the boundary
    elif case == "all_equal":
        sc = np.full(S, 0.5, np.float32)
    elif case == "negative":
        sc = -np.abs(sc) - 1
    idx = orc.select_keys(sc, S)
    verify_selection(idx, sc, S)
    assert set(idx[:1024].tolist()) == np_select(sc, S)
    kth_bits = sorted((orc.order_bits(v) for v in sc[:S - 128]), reverse=True)[1023]
    bits = np.array([orc.order_bits(v) for v in sc[:S - 128]])
    ngt = int((bits > kth_bits).sum())
    # greater keys first in index order, then the tied ones in index order
    assert list(idx[:ngt]) == sorted(idx[:ngt])
    assert list(idx[ngt:1024]) == sorted(idx[ngt:1024])
    assert all(bits[i] > kth_bits for i in idx[:ngt]) and all(bits[i] == kth_bits for i in idx[ngt:1024])
    if case == "all_equal":
        assert list(idx[:1024]) == list(range(1024))


def test_order_bits_monotone(orc):
    v = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf], np.float32)
    b = [orc.order_bits(x) for x in v]
    assert b == sorted(b) and b[3] < b[4]


# ------------------------------------------------------------------ index scorer
def test_index_scores(orc):
    g = synth.SplitMix64(31)
    qi = synth.f16_bits(g.normal(4 * 64)).reshape(4, 64)
    ki = synth.f16_bits(g.normal(700 * 64)).reshape(700, 64)
    w = g.uniform(4).astype(np.float32)
    got = orc.index_scores(qi, w, ki)
    dots = synth.f16_val(ki).astype(np.float64) @ synth.f16_val(qi).astype(np.float64).T
    ref = (np.maximum(dots, 0) ** 2 * w.astype(np.float64)).sum(1)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6)
    assert (got >= 0).all() and (got == 0).any() == ((dots <= 0).all(1)).any()
    # a key with every dot negative scores exactly 0; a one-hot q reads one coordinate
    q1 = np.zeros((4, 64), np.float64)
    q1[:, 5] = [1, 2, 0.5, 0.25]
    k1 = np.zeros((3, 64))
    k1[0, 5], k1[1, 5], k1[2, 5] = 2.0, -1.0, 0.5
    s1 = orc.index_scores(synth.f16_bits(q1), np.ones(4, np.float32), synth.f16_bits(k1))
    np.testing.assert_array_equal(s1, np.array([4 * (1 + 4 + 0.25 + 0.0625), 0.0, 0.25 * (1 + 4 + 0.25 + 0.0625)], np.float32))


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("weights,window", [(0, 0), (1, 0), (0, 16)])
def test_prefill_equals_decode_per_row(orc, weights, window):
    """Row i of prefill equals decode at position p0 + i over the same keys (Prefill.swift:10-13)."""
    c = synth.decode_int8_case(seed=12, S=96, n_kv=4)
    ks, vs = synth.f16_val(c["ks"]), synth.f16_val(c["vs"])
    T, p0 = 8, 88
    g = synth.SplitMix64(13)
    q = g.normal(T * 16 * 128).astype(np.float32).reshape(T, 16, 128)
    out = orc.prefill_int8(q, c["K"], ks, c["V"], vs, p0, weights=weights, window=window)
    for i in range(T):
        pos = p0 + i
        lo = max(0, pos - window + 1) if window else 0
        ref = np_decode(q[i], c["K"][:, lo:pos + 1], ks[:, lo:pos + 1], c["V"][:, lo:pos + 1], vs[:, lo:pos + 1], weights)
        np.testing.assert_allclose(out[i], ref, atol=2e-6, rtol=1e-5)


def test_decode_rows_window(orc):
    g = synth.SplitMix64(17)
    K = g.normal(4 * 64 * 128).astype(np.float32).reshape(4, 64, 128)
    V = g.normal(4 * 64 * 128).astype(np.float32).reshape(4, 64, 128)
    q = g.normal(16 * 128).astype(np.float32).reshape(16, 128)
    pos = np.arange(40, 60, dtype=np.int32)
    got = orc.decode_rows(q, K, V, pos)
    ones = np.ones((4, 64), np.float32)
    # the same math as int8 decode with unit scales on integer-valued K/V
    Ki = np.clip(np.rint(K * 20), -127, 127).astype(np.int8)
    Vi = np.clip(np.rint(V * 20), -127, 127).astype(np.int8)
    got2 = orc.decode_rows(q, Ki.astype(np.float32), Vi.astype(np.float32), pos)
    ref2 = np_decode(q, Ki[:, 40:60], ones[:, 40:60], Vi[:, 40:60], ones[:, 40:60])
    np.testing.assert_allclose(got2, ref2, rtol=1e-5, atol=1e-4)
    assert np.isfinite(got).all()


def test_rope_rotation(orc):
    x = np.arange(128, dtype=np.float32) / 7
    y = orc.rope(x, 0)
    np.testing.assert_array_equal(y, x)
    y = orc.rope(x, 1000)
    np.testing.assert_array_equal(y[64:], x[64:])
    n0 = np.hypot(x[:32], x[32:64])
    np.testing.assert_allclose(np.hypot(y[:32], y[32:64]), n0, rtol=1e-6)
    th = (np.float32(-1000) * np.array([orc.lib().orc_rope_freq(d) for d in range(32)], np.float32)).astype(np.float64)
    np.testing.assert_allclose(y[:32], x[:32] * np.cos(th) - x[32:64] * np.sin(th), atol=1e-5)


# ------------------------------------------------------------------ cache layouts
def test_tile_layout_is_a_permutation_matching_the_kernels_formula():
    from embla_attn import layout
    for kind in ("k", "v"):
        for es in (1, 2):
            off = layout.tile_offsets(kind, es)
            assert sorted(off.reshape(-1).tolist()) == list(range(4096))
    # the K formula written out for one element: key 21 (half 1, row 5), dim 70 (lane group 2)
    assert layout.tile_offsets("k", 1)[21, 70] == ((2 * 1 + (6 // 16)) * 64 + 5 + 32) * 16 + 6
    # V: key 21 = 16*1 + 4*1 + 1, dim 70 = 8*8 + 6: lane 8 + 16, byte 8*6 + 4 + 1
    assert layout.tile_offsets("v", 1)[21, 70] == ((53 // 16) * 64 + 24) * 16 + 53 % 16
    rng = np.random.default_rng(1)
    rows = rng.integers(-127, 128, (2, 64, 128)).astype(np.int8)
    for kind in ("k", "v"):
        np.testing.assert_array_equal(layout.from_tiles(layout.to_tiles(rows, kind), 2, 64, kind), rows)


def test_head_norm_vs_fp64(orc):
    """head_norm (common.metal:13-26): x * (1 + g1) * (1 + g2) / sqrt(mean(x²) + 2^-23)."""
    g = synth.SplitMix64(23)
    for ng in (0, 1, 2):
        x = synth.bf16_val(synth.bf16_bits(g.normal(128) * 4)).astype(np.float32)
        g1 = synth.bf16_val(synth.bf16_bits(g.normal(128) * 0.3))
        g2 = synth.bf16_val(synth.bf16_bits(g.normal(128) * 0.3))
        got = orc.head_norm(x, g1, g2, ng, round_bf=False)
        ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1.1920929e-07)
        if ng >= 1:
            ref = ref * (1 + g1.astype(np.float64))
        if ng >= 2:
            ref = ref * (1 + g2.astype(np.float64))
        np.testing.assert_allclose(got, ref, rtol=3e-6, atol=1e-6)
        # rounding to bf16 is the RNE of the unrounded value
        np.testing.assert_array_equal(orc.head_norm(x, g1, g2, ng, round_bf=True), synth.bf16_val(synth.bf16_bits(got)))
    # a zero row stays zero (eps keeps the factor finite)
    assert not orc.head_norm(np.zeros(128), None, None, 0).any()


# ---------------------------------------------------------------- 4-bit projections (gemv/gemm)
def _bf(v):
    return synth.bf16_bits(np.asarray(v, np.float32))


def test_q4_matvec_nibble_order_known_answers(orc):
    """gemm.metal's dequant: nibble q of word c (bits 4q..) is column 8c + q; group g of 64
    columns has one scale and bias. Hand-built words with known nibbles, closed-form sums."""
    O, K = 3, 2048
    w = np.zeros((O, K // 8), np.uint32)
    w[0, 0] = 0x76543210            # columns 0..7 hold 0..7
    w[1, 9] = 0xF0000000            # column 8 * 9 + 7 = 79 holds 15
    w[2, :] = 0xFFFFFFFF            # every column 15
    s = np.full((O, K // 64), _bf(1.0)[()], np.uint16)
    b = np.zeros((O, K // 64), np.uint16)
    s[1, 1] = _bf(0.5)              # column 79 is in group 1
    s[2, :] = _bf(2.0)
    b[2, :] = _bf(-3.0)             # w = 2 * 15 - 3 = 27
    # x = 1 on columns 0..7 and 79, 0 elsewhere
    x = np.zeros(K, np.float32)
    x[:8] = 1.0
    x[79] = 1.0
    y = orc.q4_matvec(w, s, b, _bf(x), epi=4)
    assert y[0] == 28.0                  # 0 + 1 + ... + 7
    assert y[1] == 7.5                   # 15 * 0.5 at column 79
    assert y[2] == 27.0 * 9              # nine columns of 27
    # one-hot columns read back each column's weight
    g = synth.SplitMix64(5)
    wr = (g.uniform(O * K // 8) * 2 ** 32).astype(np.uint64).astype(np.uint32).reshape(O, K // 8)
    sr = _bf(g.uniform(O * K // 64) + 0.5).reshape(O, K // 64)
    br = _bf(g.uniform(O * K // 64) - 0.5).reshape(O, K // 64)
    for c in [0, 1, 7, 8, 63, 64, 65, 1000, 2047]:
        e = np.zeros(K, np.float32)
        e[c] = 1.0
        y = orc.q4_matvec(wr, sr, br, _bf(e), epi=4)
        q = np.array([(int(wr[r, c // 8]) >> (4 * (c % 8))) & 15 for r in range(O)], np.float64)
        want = synth.bf16_val(sr[:, c // 64]).astype(np.float64) * q + synth.bf16_val(br[:, c // 64])
        np.testing.assert_array_equal(y, want.astype(np.float32))


def test_q4_matvec_epilogues(orc):
    """gemv.metal:77-88. Column 0's weight is 1 * 1 + 2^-9 (scale 1, bias 2^-9: both exact in
    bf16), every other weight 0, so acc = (1 + 2^-9) x0 and each epilogue's rounding shows."""
    K = 2048
    w = np.zeros((1, K // 8), np.uint32)
    w[0, 0] = 1
    s = np.full((1, K // 64), _bf(1.0)[()], np.uint16)
    b = np.zeros((1, K // 64), np.uint16)
    b[0, 0] = _bf(2.0 ** -9)
    for x0, epi, y0, want in [(1.0, 0, None, 1.0),                          # bf16(1 + 2^-9) = 1
                              (-2.0, 1, None, 0.0),                         # relu of a negative
                              (3.0, 1, None, 9.0),                          # bf16(3.006) = 3, squared
                              (1.0, 2, 10.0, 11.0),                         # y += bf16(acc)
                              (1.0, 3, None, 1.0),
                              (1.0, 4, None, 1.0 + 2.0 ** -9)]:             # unrounded
        x = np.zeros(K, np.float32)
        x[0] = x0
        y = orc.q4_matvec(w, s, b, _bf(x), epi=epi, y=None if y0 is None else np.float32([y0]))
        assert y[0] == np.float32(want), (x0, epi, y[0])


def test_q4_matvec_mlx_quantised_round_trip(orc):
    """An independent affine quantiser (MLX's published one: per group of 64, scale = (max -
    min) / 15, bias = min, q = round((w - bias) / scale)) packed into words: the oracle's product
    matches the dense product of the dequantised matrix, and the original within the bound."""
    O, K = 8, 2048
    g = synth.SplitMix64(11)
    Wd = g.normal(O * K).astype(np.float32).reshape(O, K)
    x = synth.bf16_val(_bf(g.normal(K)))
    G = Wd.reshape(O, K // 64, 64)
    lo, hi = G.min(-1), G.max(-1)
    sc = synth.bf16_val(_bf((hi - lo) / 15))
    bi = synth.bf16_val(_bf(lo))
    q = np.clip(np.rint((G - bi[..., None]) / sc[..., None]), 0, 15).astype(np.uint32).reshape(O, K)
    words = np.zeros((O, K // 8), np.uint32)
    for j in range(8):
        words |= q[:, j::8] << np.uint32(4 * j)
    y = orc.q4_matvec(words, _bf(sc), _bf(bi), _bf(x), epi=4)
    deq = (sc[..., None] * q.reshape(O, K // 64, 64) + bi[..., None]).reshape(O, K).astype(np.float64)
    np.testing.assert_allclose(y, deq @ x.astype(np.float64), rtol=1e-6, atol=1e-4)
    bound = (np.repeat(sc, 64, axis=1) * 0.51 + 0.02) @ np.abs(x)
    assert np.all(np.abs(y - Wd.astype(np.float64) @ x) <= bound)
