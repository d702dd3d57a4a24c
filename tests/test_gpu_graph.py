"""A whole attention sub-layer decode step captured as one HIP graph (the event-chained step of
Engine.swift:71-88 as a graph): per layer the q/k/v projection, the int8 append of the new k, v,
the q preparation and split-K decode (layer 0 as two calls, layer 1 as the decode with the head
norm inside, layer 2 as the decode step that appends its own token) and the o-projection into an
fp32 residual.
The graph is replayed several times with eager work between the replays, and every replay's
outputs (the decode outputs, the residual, the appended cache bytes) equal the eager step's bit
for bit: every kernel here reduces in a fixed order."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import assert_close, dev, say
from embla_attn import layout, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch


def pack(mats):
    parts, offs, at = [], [], 0
    for m in mats:
        o = []
        for a in m:
            b = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
            pad = (-at) % 256
            parts.append(np.zeros(pad, np.uint8))
            at += pad
            o.append(at)
            parts.append(b)
            at += b.size
        offs.append(o)
    return np.concatenate(parts), offs


def test_graph_decode_step_replays(torch_gpu, orc):
    from embla_attn import ops
    torch = torch_gpu
    n_layers, D, n_q, n_kv, max_s, pos = 3, 2048, 16, 4, 1024, 700
    g = synth.SplitMix64(91)
    layers = []
    for l in range(n_layers):
        buf, offs = pack([synth.q4_weights(g, 3072, D), synth.q4_weights(g, D, D)])
        W = dev(buf)
        segs = [(offs[0][0], offs[0][1], offs[0][2], 3072, 0, 0)]
        osegs = [(offs[1][0], offs[1][1], offs[1][2], D, 0, 0)]
        hist = synth.decode_int8_case(seed=92 + l, S=pos, n_kv=n_kv)
        kc = dev(layout.pack_region(hist["K"], hist["ks"], max_s, "k"))
        vc = dev(layout.pack_region(hist["V"], hist["vs"], max_s, "v"))
        layers.append(dict(W=W, segs=segs, osegs=osegs, kc=kc, vc=vc, ws=ops.Workspace(max_s, n_q),
                           o=torch.empty(n_q, 128, dtype=torch.bfloat16, device="cuda"),
                           qf=torch.empty(1, n_q, 128, dtype=torch.float16, device="cuda"),
                           qr=torch.empty(2048, dtype=torch.bfloat16, device="cuda"), mode=l % 3))
    x = dev(synth.bf16_bits(g.normal(D).astype(np.float32)), torch.bfloat16)
    qkv = torch.empty(3072, dtype=torch.bfloat16, device="cuda")
    resid = torch.empty(D, dtype=torch.float32, device="cuda")

    def step():
        resid.zero_()   # a fill kernel, not a memset node
        for L in layers:
            ops.gemv_q4(L["W"], x, qkv, L["segs"], D, ops.EPI_BF16)
            if L["mode"] == 2:   # the append inside the decode launch
                L["qr"].copy_(qkv[:2048])
                ops.decode_step_int8(qkv, 0, 2048, 2560, L["kc"], L["vc"], pos, max_s, n_q, n_kv, L["ws"], out=L["o"])
                ops.gemv_q4(L["W"], L["o"], resid, L["osegs"], D, ops.EPI_ADD)
                continue
            ops.kv_quant_append(qkv[2048:2560], qkv[2560:3072], 1, pos, n_kv, L["kc"], L["vc"], max_s)
            if L["mode"] == 1:   # the head norm inside the decode kernel
                L["qr"].copy_(qkv[:2048])
                ops.decode_int8_qraw(qkv[:2048], L["kc"], L["vc"], pos + 1, max_s, n_kv, ws=L["ws"], out=L["o"])
            else:
                ops.q_prep(qkv[:2048], None, None, 0, 1, n_q, out=L["qf"])
                ops.decode_int8(L["qf"][0], L["kc"], L["vc"], pos + 1, max_s, n_kv, out_dtype=ops.BF16,
                                ws=L["ws"], out=L["o"])
            ops.gemv_q4(L["W"], L["o"], resid, L["osegs"], D, ops.EPI_ADD)

    def snapshot():
        torch.cuda.synchronize()
        return [L["o"].float().cpu().numpy().copy() for L in layers] + [resid.cpu().numpy().copy()] + \
               [torch.cat([L["kc"], L["vc"]]).cpu().numpy().copy() for L in layers]

    say("graph decode step: eager")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step()
    want = snapshot()
    assert np.isfinite(want[n_layers]).all() and np.abs(want[n_layers]).max() > 0
    # the eager step itself: each layer's decode output against the oracle over the q and the
    # cache (history plus the appended position) it read
    for l, L in enumerate(layers):
        cache = want[n_layers + 1 + l].view(np.uint8)
        rb = L["kc"].numel()
        K, ks = layout.unpack_region(cache[:rb], n_kv, max_s, "k", np.uint16)
        V, vs = layout.unpack_region(cache[rb:], n_kv, max_s, "v", np.uint16)
        n = pos + 1
        if L["mode"]:   # the raw q the layer read
            qb = L["qr"].view(torch.int16).cpu().numpy().view(np.uint16).reshape(n_q, 128)
            q = np.stack([orc.head_norm(synth.bf16_val(qb[h])) for h in range(n_q)])
        else:
            q = L["qf"].float().cpu().numpy()[0]
        ref = orc.decode_int8(q, K[:, :n], synth.f16_val(ks[:, :n]), V[:, :n], synth.f16_val(vs[:, :n]))
        assert_close(want[l], ref, what=f"layer {l} decode")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        say(f"graph decode step: replay {rep}")
        # eager work between the replays, on the outputs' buffers too
        resid.fill_(float(rep + 1))
        for L in layers:
            L["o"].fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        got = snapshot()
        for i, (a, b) in enumerate(zip(got, want)):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {rep}: output {i}")
