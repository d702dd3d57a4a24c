"""Parity of the int8 split-K decode (configs C1 and C3; the reference's attn_full8 / attn_sparse8
math) against the C oracle on the same seeded inputs."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, dev, f16_host, bf16_host, say, upload_int8_case
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def run_cfg_decode(torch, c, max_s, chunk=0, ws=None):
    from embla_attn import ops
    kc, vc = upload_int8_case(c, max_s)
    q = dev(c["q"], torch.float16)
    ws = ws or ops.Workspace(max_s, c["n_q"])
    o = ops.decode_int8(q, kc, vc, c["S"], max_s, c["n_kv"], chunk=chunk, ws=ws)
    torch.cuda.synchronize()
    return f16_host(o)


def oracle_cfg(orc, c, weights=0):
    return orc.decode_int8(synth.f16_val(c["q"]), c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]),
                           weights=weights)


@pytest.mark.parametrize("S,max_s,seed", [(1024, 1024, 0), (1000, 1024, 5), (33, 64, 6), (1, 32, 7), (4096, 4096, 2),
                                          (16384, 16384, 2), (32768, 32768, 2),
                                          (131072, 131072, 9)])   # beyond the configs: a 128k context
def test_decode_softmax_int8_matches_oracle(torch_gpu, orc, S, max_s, seed):
    say(f"decode softmax int8 S={S} max_s={max_s} seed={seed}")
    c = synth.decode_int8_case(seed=seed, S=S)
    got = run_cfg_decode(torch_gpu, c, max_s)
    assert_close(got, oracle_cfg(orc, c), what=f"S={S}")


@pytest.mark.parametrize("S,chunk", [(4000, 128), (4000, 256), (4000, 512), (4000, 2048), (4000, 4096),
                                     (12000, 128), (20000, 128), (32768, 128), (8000, 96)])   # 65 .. 256 chunks
def test_decode_independent_of_split(torch_gpu, orc, S, chunk):
    say(f"decode split S={S} chunk={chunk}")
    c = synth.decode_int8_case(seed=0, S=S)
    ref = oracle_cfg(orc, c)
    got = run_cfg_decode(torch_gpu, c, (S + 31) // 32 * 32, chunk=chunk)
    assert_close(got, ref, what=f"S={S} chunk={chunk}")


@pytest.mark.parametrize("S", [40, 5000])
def test_decode_f16_scales_bf16_out(torch_gpu, orc, S):
    """The sub-layer step's decode: fp16 scales, bf16 output for the o-projection's input."""
    from embla_attn import ops
    say(f"decode f16 scales bf16 out S={S}")
    c = synth.decode_int8_case(seed=11, S=S)
    kc, vc = upload_int8_case(c, 8192)
    o = ops.decode_int8(dev(c["q"], torch_gpu.float16), kc, vc, S, 8192, c["n_kv"], out_dtype=ops.BF16,
                        ws=ops.Workspace(8192, c["n_q"]))
    torch_gpu.cuda.synchronize()
    assert_close(bf16_host(o), oracle_cfg(orc, c), what=f"S={S}")


@pytest.mark.parametrize("ng,S", [(0, 3000), (2, 32768), (1, 77)])
def test_decode_qraw_matches_oracle(torch_gpu, orc, ng, S):
    """embla_decode_int8_qraw: raw bf16 q, head-normed (with ng gains) inside the decode kernel."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"decode raw q ng={ng} S={S}")
    c = synth.decode_int8_case(seed=13 + ng, S=S)
    g = synth.SplitMix64(50 + ng)
    qraw = synth.bf16_bits(g.normal(16 * 128) * 3)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    ms = (S + 31) // 32 * 32
    kc, vc = upload_int8_case(c, ms)
    o = ops.decode_int8_qraw(dev(qraw, torch.bfloat16), kc, vc, S, ms, 4, g1=dev(g1, torch.bfloat16),
                             g2=dev(g2, torch.bfloat16), ng=ng, ws=ops.Workspace(ms, 16))
    torch.cuda.synchronize()
    qn = np.stack([orc.head_norm(synth.bf16_val(qraw.reshape(16, 128)[h]), synth.bf16_val(g1), synth.bf16_val(g2), ng)
                   for h in range(16)])
    ref = orc.decode_int8(qn, c["K"], synth.f16_val(c["ks"]), c["V"], synth.f16_val(c["vs"]))
    assert_close(bf16_host(o), ref, what=f"ng={ng} S={S}")


@pytest.mark.parametrize("S", [32768, 3000])
def test_decode_partials_then_merge_equals_one_call(torch_gpu, S):
    """embla_decode_int8_partials + embla_decode_int8_merge run the one-call decode's two kernels."""
    from embla_attn import ops
    torch = torch_gpu
    say(f"decode partials + merge S={S}")
    c = synth.decode_int8_case(seed=21, S=S)
    ms = (S + 31) // 32 * 32
    kc, vc = upload_int8_case(c, ms)
    q = dev(c["q"], torch.float16)
    ws = ops.Workspace(ms, 16)
    one = ops.decode_int8(q, kc, vc, S, ms, 4, ws=ws)
    ops.decode_int8_partials(q, kc, vc, S, ms, 4, ws)
    two = ops.decode_int8_merge(torch.empty_like(one), S, ms, 4, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(two.cpu().numpy(), one.cpu().numpy())


def test_decode_repeated_calls_leave_counters_zero(torch_gpu, orc):
    from embla_attn import ops
    say("decode repeated calls, one workspace")
    ws = ops.Workspace(8192, 16)
    for seed, S in [(1, 8192), (2, 3000), (3, 8000)]:
        c = synth.decode_int8_case(seed=seed, S=S)
        got = run_cfg_decode(torch_gpu, c, 8192, ws=ws)
        assert_close(got, oracle_cfg(orc, c), what=f"call S={S}")
    torch_gpu.cuda.synchronize()
    assert not ws.buf[:256].cpu().numpy().any()


def test_full8_reference_mode(torch_gpu, orc):
    """attn_full8: raw bf16 q with two gains, 2 kv heads, ReLU² + sink, fp32 scales, SCORES."""
    import torch
    from embla_attn import ops
    say("attn_full8 reference mode")
    S, max_s = 3000, 4096
    g = synth.SplitMix64(40)
    qraw = synth.bf16_bits(g.normal(16 * 128) * 2)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    # a cache as kv_append writes it: normed rows, int8, fp32 scales
    K = g.int8(2 * S * 128).reshape(2, S, 128)
    V = g.int8(2 * S * 128).reshape(2, S, 128)
    ks = (0.02 + 0.01 * g.uniform(2 * S)).astype(np.float32).reshape(2, S)
    vs = (0.02 + 0.01 * g.uniform(2 * S)).astype(np.float32).reshape(2, S)
    kc = dev(layout.pack_region(K, ks, max_s, "k"))
    vc = dev(layout.pack_region(V, vs, max_s, "v"))
    from embla_attn import _lib
    part = torch.zeros(_lib.lib().embla_workspace_bytes(max_s, 16), dtype=torch.uint8, device="cuda")
    counter = torch.zeros(2, dtype=torch.int32, device="cuda")
    scores = torch.full((2, max_s), -1.0, dtype=torch.float32, device="cuda")
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    ops.attn_full8(dev(qraw, torch.bfloat16), dev(g1, torch.bfloat16), dev(g2, torch.bfloat16), kc, vc, part, scores,
                   counter, o, S, max_s, ng=2)
    torch.cuda.synchronize()
    qn = np.stack([orc.head_norm(synth.bf16_val(qraw.reshape(16, 128)[h]), synth.bf16_val(g1), synth.bf16_val(g2), 2)
                   for h in range(16)])
    ref, ref_sc = orc.decode_int8(qn, K, ks, V, vs, weights=1, want_scores=True)
    assert_close(bf16_host(o), ref, what="full8 o")
    # scores are fp32 sums of exact products: within 2^-16 of sum_d |q_d k_d| ks (128 roundings of
    # 2^-24 each, with a 2x margin), the max over the kv head's query heads
    got_sc = scores.cpu().numpy()[:, :S]
    bound = np.stack([(np.abs(qn[8 * h:8 * h + 8]) @ np.abs(K[h].astype(np.float64)).T).max(0) * ks[h]
                      for h in range(2)])
    assert (np.abs(got_sc - ref_sc) <= bound * 2.0 ** -16).all(), np.abs(got_sc - ref_sc).max()
    assert not counter.cpu().numpy().any()


def test_full8_scores_select_sparse8_chain_near_ties(torch_gpu, orc):
    """The reference's full -> select_keys -> sparse chain (Engine.swift:796-827): attn_full8's
    SCORES feed embla_select_keys, whose rows feed attn_sparse8 (SEL). The scales put 1000 keys a kv
    head clearly above the threshold and 60 in a cluster around it whose scores are 2e-6 apart
    (~30 fp32 steps): the selection must be the oracle's bit for bit, which a q rounded to a
    16-bit fixed point (relative error ~1e-4) cannot give."""
    import torch
    from embla_attn import ops, _lib
    say("full8 -> select_keys -> sparse8 near ties")
    S, max_s = 3000, 4096
    g = synth.SplitMix64(43)
    qraw = synth.bf16_bits(g.normal(16 * 128) * 2)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    K = g.int8(2 * S * 128).reshape(2, S, 128)
    V = g.int8(2 * S * 128).reshape(2, S, 128)
    vs = (0.02 + 0.01 * g.uniform(2 * S)).astype(np.float32).reshape(2, S)
    qn = np.stack([orc.head_norm(synth.bf16_val(qraw.reshape(16, 128)[h]), synth.bf16_val(g1), synth.bf16_val(g2), 2)
                   for h in range(16)])
    ks = (0.02 + 0.01 * g.uniform(2 * S)).astype(np.float32).reshape(2, S)
    near_sets = []
    for h in range(2):
        d = (qn[8 * h:8 * h + 8].astype(np.float64) @ K[h].astype(np.float64).T).max(0)   # [S]
        T = 1.25 * np.abs(d).max() * 0.03   # above every other key's score
        order = np.argsort(-d[:S - 128], kind="stable")   # the largest dots (all > 0)
        top, near = order[:1000], order[1000:1060]
        assert d[near].min() > 0.2 * d[order[0]]
        ks[h, top] = (1.5 * T / d[top]).astype(np.float32)
        r = np.argsort(g.uniform(60)) - 30   # a shuffled cluster: index order is not score order
        near_sets.append(near)
        ks[h, near] = (T * (1.0 + 2e-6 * r) / d[near]).astype(np.float32)
    kc = dev(layout.pack_region(K, ks, max_s, "k"))
    vc = dev(layout.pack_region(V, vs, max_s, "v"))
    part = torch.zeros(_lib.lib().embla_workspace_bytes(max_s, 16), dtype=torch.uint8, device="cuda")
    counter = torch.zeros(2, dtype=torch.int32, device="cuda")
    scores = torch.full((2, max_s), -1.0, dtype=torch.float32, device="cuda")
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    qd, g1d, g2d = dev(qraw, torch.bfloat16), dev(g1, torch.bfloat16), dev(g2, torch.bfloat16)
    ops.attn_full8(qd, g1d, g2d, kc, vc, part, scores, counter, o, S, max_s, ng=2)
    idx = ops.select_keys(scores, S, max_s)
    o2 = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    ops.attn_sparse8(qd, g1d, g2d, kc, vc, part, idx, counter, o2, 1152, max_s)
    torch.cuda.synchronize()
    ref_o, ref_sc = orc.decode_int8(qn, K, ks, V, vs, weights=1, want_scores=True)
    assert_close(bf16_host(o), ref_o, what="chain full8 o")
    ref_rows = np.stack([orc.select_keys(np.ascontiguousarray(ref_sc[h]), S) for h in range(2)])
    got_rows = idx.cpu().numpy().astype(np.uint32).reshape(2, 1152)
    for h in range(2):   # the cluster straddles the threshold: 24 of its 60 keys are in
        assert np.isin(near_sets[h], ref_rows[h, :1024]).sum() == 24
    np.testing.assert_array_equal(got_rows, ref_rows)
    ref2 = orc.decode_int8(qn, K, ks, V, vs, weights=0, rows=ref_rows, n_sel=1152)
    assert_close(bf16_host(o2), ref2, what="chain sparse8 o")


@pytest.mark.parametrize("sel", [True, False])
def test_sparse8_reference_mode(torch_gpu, orc, sel):
    """attn_sparse8: raw bf16 q with two gains, 2 kv heads of the full layer's tile cache (fp32
    scales), softmax over the selected rows idx[kv head][0 .. 1152) (SEL) or every key."""
    import torch
    from embla_attn import ops, _lib
    say(f"attn_sparse8 reference mode sel={sel}")
    S_cache, max_s = 5000, 5024
    g = synth.SplitMix64(41)
    qraw = synth.bf16_bits(g.normal(16 * 128) * 2)
    g1 = synth.bf16_bits(g.normal(128) * 0.2)
    g2 = synth.bf16_bits(g.normal(128) * 0.2)
    K = g.int8(2 * S_cache * 128).reshape(2, S_cache, 128)
    V = g.int8(2 * S_cache * 128).reshape(2, S_cache, 128)
    ks = (0.02 + 0.01 * g.uniform(2 * S_cache)).astype(np.float32).reshape(2, S_cache)
    vs = (0.02 + 0.01 * g.uniform(2 * S_cache)).astype(np.float32).reshape(2, S_cache)
    kc = dev(layout.pack_region(K, ks, max_s, "k"))
    vc = dev(layout.pack_region(V, vs, max_s, "v"))
    part = torch.zeros(_lib.lib().embla_workspace_bytes(max_s, 16), dtype=torch.uint8, device="cuda")
    counter = torch.zeros(2, dtype=torch.int32, device="cuda")
    o = torch.empty((16, 128), dtype=torch.bfloat16, device="cuda")
    qn = np.stack([orc.head_norm(synth.bf16_val(qraw.reshape(16, 128)[h]), synth.bf16_val(g1), synth.bf16_val(g2), 2)
                   for h in range(16)])
    if sel:
        # per kv head: 1024 distinct rows in shuffled order (every tile position, both halves), then
        # the latest 128; the order of the list is irrelevant to the result
        rows = np.zeros((2, 1152), np.uint32)
        for h in range(2):
            r = (g.next(S_cache - 128) % np.uint64(1 << 62)).astype(np.float64)
            rows[h, :1024] = np.argsort(r)[:1024].astype(np.uint32)
            rows[h, 1024:] = np.arange(S_cache - 128, S_cache, dtype=np.uint32)
        ops.attn_sparse8(dev(qraw, torch.bfloat16), dev(g1, torch.bfloat16), dev(g2, torch.bfloat16), kc, vc, part,
                         dev(rows.view(np.int32)), counter, o, 1152, max_s)
        ref = orc.decode_int8(qn, K, ks, V, vs, weights=0, rows=rows, n_sel=1152)
    else:
        ops.attn_sparse8(dev(qraw, torch.bfloat16), dev(g1, torch.bfloat16), dev(g2, torch.bfloat16), kc, vc, part,
                         None, counter, o, S_cache, max_s)
        ref = orc.decode_int8(qn, K, ks, V, vs, weights=0)
    torch.cuda.synchronize()
    assert_close(bf16_host(o), ref, what=f"sparse8 sel={sel}")
