"""Sparse layers (config C4): the index scorer and the radix top-k are bit-exact with the oracle;
attention over the selected rows matches within tolerance; the whole layer end to end."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, dev, f16_host, say
from embla_attn import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


@pytest.fixture(scope="module")
def c4():
    return synth.sparse_case(seed=3, ctx=32768)


def test_index_scores_bit_exact(torch_gpu, orc, c4):
    from embla_attn import ops
    torch = torch_gpu
    n = 32768 - 128
    say("index scores n=32640")
    got = ops.index_scores(dev(c4["qi"], torch.float16), dev(c4["w"]), dev(c4["ki"], torch.float16), n)
    ref = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:n])
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("case", ["c4", "ties", "all_equal", "negative", "small"])
def test_select_topk_bit_exact(torch_gpu, orc, c4, case):
    from embla_attn import ops
    torch = torch_gpu
    S = 32768 if case != "small" else 1153
    if case == "c4":
        sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:S - 128])
    else:
        g = synth.SplitMix64(99)
        sc = g.normal(S - 128).astype(np.float32)
        if case == "ties":
            sc = np.round(sc * 3) / 3
        elif case == "all_equal":
            sc = np.full(S - 128, 1.25, np.float32)
        elif case == "negative":
            sc = -np.abs(sc) - 1
    sc = sc.astype(np.float32)
    say(f"select topk case={case}")
    idx = ops.select_topk(dev(sc), S)
    ref = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
    np.testing.assert_array_equal(idx.cpu().numpy()[0].astype(np.uint32), ref)


def test_select_keys_reference_two_sets(torch_gpu, orc):
    from embla_attn import ops
    torch = torch_gpu
    maxS, S = 8192, 5000
    g = synth.SplitMix64(5)
    sc = (np.round(g.normal(2 * maxS) * 8) / 8).astype(np.float32).reshape(2, maxS)
    say("select_keys reference two sets")
    idx = ops.select_keys(dev(sc), S, maxS)
    for h in range(2):
        np.testing.assert_array_equal(idx.cpu().numpy()[h].astype(np.uint32), orc.select_keys(sc[h], S))


@pytest.mark.parametrize("nsel,chunk", [(1152, 0), (1152, 1152), (37, 0), (300, 64)])
def test_sparse_decode_gathered(torch_gpu, orc, c4, nsel, chunk):
    from embla_attn import ops
    torch = torch_gpu
    say(f"sparse decode gathered nsel={nsel} chunk={chunk}")
    rng = np.random.default_rng(nsel)
    idx = np.sort(rng.choice(32768, nsel, replace=False)).astype(np.uint32)
    rng.shuffle(idx)
    ws = ops.Workspace(32 * ((nsel + 31) // 32) + 4096, 16)
    o = ops.sparse_decode(dev(c4["q"], torch.float16), dev(c4["K"], torch.float16), dev(c4["V"], torch.float16),
                          dev(idx.view(np.int32)), nsel, 32768, 4, chunk=chunk, ws=ws)
    ref = orc.decode_rows(synth.f16_val(c4["q"]), synth.f16_val(c4["K"]), synth.f16_val(c4["V"]), idx.astype(np.int32))
    assert_close(f16_host(o), ref, what=f"nsel={nsel}")


@pytest.mark.parametrize("S", [32768, 1000, 1151, 1152, 1153, 1154, 32767])
def test_sparse_layer_end_to_end(torch_gpu, orc, c4, S):
    from embla_attn import ops
    torch = torch_gpu
    say(f"sparse layer end to end S={S}")
    ws = ops.SparseWorkspace(32768, 16)
    K = dev(c4["K"], torch.float16)
    V = dev(c4["V"], torch.float16)
    o = ops.sparse_layer_decode(dev(c4["q"], torch.float16), dev(c4["qi"], torch.float16), dev(c4["w"]),
                                dev(c4["ki"], torch.float16), K, V, S, 32768, 4, ws)
    if S > 1152:
        sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:S - 128])
        sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S).astype(np.int32)
    else:
        sel = np.arange(S, dtype=np.int32)
    ref = orc.decode_rows(synth.f16_val(c4["q"]), synth.f16_val(c4["K"]), synth.f16_val(c4["V"]), sel)
    assert_close(f16_host(o), ref, what=f"S={S}")


def test_sparse_layer_gq8_bf16(torch_gpu, orc, c4):
    """16 query heads over 2 kv heads (GQ = 8) and bf16 activations and caches: the attention's
    own select in its GQ = 8, bf16 instance."""
    from embla_attn import ops
    torch = torch_gpu
    S = 30001
    say("sparse layer GQ 8 bf16")
    K = synth.bf16_bits(synth.f16_val(c4["K"][:2]))
    V = synth.bf16_bits(synth.f16_val(c4["V"][:2]))
    q = synth.bf16_bits(synth.f16_val(c4["q"]))
    ws = ops.SparseWorkspace(32768, 16)
    o = ops.sparse_layer_decode(dev(q.view(np.int16), torch.bfloat16), dev(c4["qi"], torch.float16), dev(c4["w"]),
                                dev(c4["ki"], torch.float16), dev(K.view(np.int16), torch.bfloat16),
                                dev(V.view(np.int16), torch.bfloat16), S, 32768, 2, ws, dtype=ops.BF16)
    got = ws.selection().cpu().numpy().astype(np.uint32)
    sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:S - 128])
    sel = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
    np.testing.assert_array_equal(got, sel)
    ref = orc.decode_rows(synth.bf16_val(q), synth.bf16_val(K), synth.bf16_val(V), sel.astype(np.int32))
    assert_close(o.float().cpu().numpy(), ref, what="GQ 8 bf16")


def test_sparse_layer_selection_bit_exact(torch_gpu, orc, c4):
    """The layer's selection (scorer histogram, wide classify, final select on the candidates) is
    select_keys' output bit for bit, over consecutive calls of one workspace at different S (each
    call leaves the select's counters zero for the next)."""
    from embla_attn import ops
    torch = torch_gpu
    ws = ops.SparseWorkspace(32768, 16)
    args = [dev(c4["q"], torch.float16), dev(c4["qi"], torch.float16), dev(c4["w"]), dev(c4["ki"], torch.float16),
            dev(c4["K"], torch.float16), dev(c4["V"], torch.float16)]
    for S in [32768, 5000, 1153, 32768, 20011]:
        say(f"sparse layer selection S={S}")
        ops.sparse_layer_decode(*args, S, 32768, 4, ws)
        got = ws.selection().cpu().numpy().astype(np.uint32)
        sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:S - 128])
        ref = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
        np.testing.assert_array_equal(got, ref, err_msg=f"S={S}")


def test_sparse_layer_selection_ties(torch_gpu, orc, c4):
    """Index keys repeated 16 times: every score occurs 16 times, so the threshold value is tied
    and the first of its keys by index are taken."""
    from embla_attn import ops
    torch = torch_gpu
    S = 30000
    ki = np.repeat(c4["ki"][:2048], 16, axis=0)
    ws = ops.SparseWorkspace(32768, 16)
    say("sparse layer selection ties")
    ops.sparse_layer_decode(dev(c4["q"], torch.float16), dev(c4["qi"], torch.float16), dev(c4["w"]),
                            dev(ki, torch.float16), dev(c4["K"], torch.float16), dev(c4["V"], torch.float16),
                            S, 32768, 4, ws)
    got = ws.selection().cpu().numpy().astype(np.uint32)
    sc = orc.index_scores(c4["qi"], c4["w"], ki[:S - 128])
    ref = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
    np.testing.assert_array_equal(got, ref)


def test_sparse_layer_selection_many_candidates(torch_gpu, orc, c4):
    """600 copies of one index key whose score ranks ~900th: the topk-th value is a tie among
    them, so the first digit's candidates (> 256, > 32 in one classify region) take the
    workgroup-wide ranking path of the attention's select."""
    from embla_attn import ops
    torch = torch_gpu
    S = 32768
    ki = c4["ki"].copy()
    sc = orc.index_scores(c4["qi"], c4["w"], ki[:S - 128])
    x = int(np.argsort(-sc.astype(np.float64), kind="stable")[900])
    ki[:600] = ki[x]
    ws = ops.SparseWorkspace(32768, 16)
    say("sparse layer selection many candidates")
    o = ops.sparse_layer_decode(dev(c4["q"], torch.float16), dev(c4["qi"], torch.float16), dev(c4["w"]),
                                dev(ki, torch.float16), dev(c4["K"], torch.float16), dev(c4["V"], torch.float16),
                                S, 32768, 4, ws)
    got = ws.selection().cpu().numpy().astype(np.uint32)
    sc = orc.index_scores(c4["qi"], c4["w"], ki[:S - 128])
    ref = orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)
    np.testing.assert_array_equal(got, ref)
    assert len(np.nonzero(ref[:1024] < 600)[0]) > 0   # some of the copies are taken
    out = orc.decode_rows(synth.f16_val(c4["q"]), synth.f16_val(c4["K"]), synth.f16_val(c4["V"]), ref.astype(np.int32))
    assert_close(f16_host(o), out, what="many candidates")


def test_select_topk_many_sets_unaligned(torch_gpu, orc):
    """Several sets at an odd stride (rows not 16-byte aligned), ragged n, a small topk."""
    from embla_attn import ops
    torch = torch_gpu
    S, stride, n_sets, topk, recent = 5003, 5007, 5, 300, 17
    g = synth.SplitMix64(123)
    sc = (g.normal(n_sets * stride).astype(np.float32) * 10).round().reshape(n_sets, stride)
    say("select topk many sets unaligned")
    idx = ops.select_topk(dev(sc.reshape(-1)), S, n_sets=n_sets, topk=topk, recent=recent, score_stride=stride)
    got = idx.cpu().numpy().astype(np.uint32)
    for s in range(n_sets):
        row = np.concatenate([sc[s, :S - recent], np.zeros(recent, np.float32)])
        ref = orc.select_keys(row, S, topk=topk, recent=recent)
        np.testing.assert_array_equal(got[s], ref, err_msg=f"set {s}")


def _c4_args(torch, c4):
    return [dev(c4["q"], torch.float16), dev(c4["qi"], torch.float16), dev(c4["w"]), dev(c4["ki"], torch.float16),
            dev(c4["K"], torch.float16), dev(c4["V"], torch.float16)]


def _c4_ref_selection(orc, c4, S):
    sc = orc.index_scores(c4["qi"], c4["w"], c4["ki"][:S - 128])
    return orc.select_keys(np.concatenate([sc, np.zeros(128, np.float32)]), S)


def test_sparse_layer_dirty_workspace_recounts(torch_gpu, orc, c4):
    """A workspace full of random bytes (never zeroed) still gives select_keys' selection bit for
    bit: the select finds that its histogram does not count exactly this call's keys and recounts
    them (the workspace's recount word says so once); the next call finds a clean buffer."""
    from embla_attn import ops
    torch = torch_gpu
    ws = ops.SparseWorkspace(32768, 16)
    gen = torch.Generator(device="cpu").manual_seed(7)
    ws.buf.copy_(torch.randint(0, 256, (ws.nbytes,), dtype=torch.uint8, generator=gen))
    ws.buf[ws.recount_off:ws.recount_off + 4].zero_()
    args = _c4_args(torch, c4)
    for i, S in enumerate([32768, 20011, 32768]):
        say(f"sparse layer dirty workspace call {i} S={S}")
        o = ops.sparse_layer_decode(*args, S, 32768, 4, ws)
        got = ws.selection().cpu().numpy().astype(np.uint32)
        ref = _c4_ref_selection(orc, c4, S)
        np.testing.assert_array_equal(got, ref, err_msg=f"call {i} S={S}")
        assert ws.recounts() == 1, f"call {i}: recounts {ws.recounts()}"
    assert ws.audit() == -4   # EMBLA_ERR_WORKSPACE: a call found it not clean; the count is cleared
    assert ws.recounts() == 0 and ws.audit() == 0
    out = orc.decode_rows(synth.f16_val(c4["q"]), synth.f16_val(c4["K"]), synth.f16_val(c4["V"]), ref.astype(np.int32))
    assert_close(f16_host(o), out, what="dirty workspace")


def test_sparse_layer_rejected_call_leaves_no_state(torch_gpu, orc, c4):
    """A call the library rejects (bad n_q / n_kv ratio, bad dtype) launches nothing, so the next
    valid call's selection is select_keys' bit for bit with no recount; an overwritten histogram
    buffer between calls is recounted."""
    from embla_attn import ops
    from embla_attn._lib import EmblaError, lib
    from embla_attn.ops import _p
    torch = torch_gpu
    ws = ops.SparseWorkspace(32768, 16)
    args = _c4_args(torch, c4)
    S = 32768
    ops.sparse_layer_decode(*args, S, 32768, 4, ws)
    out = torch.empty((16, 128), dtype=torch.float16, device="cuda")
    ptrs = [_p(a) for a in args]
    say("sparse layer rejected calls")
    # n_q 16 over n_kv 2 (GQ 8) with fp16 is fine, n_kv 3 is not a divisor; dtype 9 is no dtype
    rc1 = lib().embla_sparse_layer_decode(*ptrs, _p(out), S, 32768, 16, 3, 4, 0, ws.ptr, ws.nbytes, None)
    rc2 = lib().embla_sparse_layer_decode(*ptrs, _p(out), S, 32768, 16, 4, 4, 9, ws.ptr, ws.nbytes, None)
    assert rc1 != 0 and rc2 != 0
    torch.cuda.synchronize()
    for S2 in [32768, 9001]:
        ops.sparse_layer_decode(*args, S2, 32768, 4, ws)
        np.testing.assert_array_equal(ws.selection().cpu().numpy().astype(np.uint32), _c4_ref_selection(orc, c4, S2))
    assert ws.recounts() == 0 and ws.audit() == 0
    # stale counts in both histogram buffers (as if a call had stopped after its scorer)
    # the select's region starts with the two histogram buffers [2][16 copies][256] and then its
    # meta words, the recount word being meta[4]
    base = ws.recount_off - (2 * 16 * 256 + 4) * 4
    ws.buf[base:base + 2 * 16 * 256 * 4].view(torch.int32).add_(3)
    ops.sparse_layer_decode(*args, S, 32768, 4, ws)
    np.testing.assert_array_equal(ws.selection().cpu().numpy().astype(np.uint32), _c4_ref_selection(orc, c4, S))
    assert ws.recounts() == 1
    with pytest.raises(EmblaError):
        ops.sparse_layer_decode(*args, S, 32768, 3, ws)
