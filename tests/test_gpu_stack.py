"""GPU parity of the 42-layer stacked decode configuration: T=8 per layer, 42 layers each with its own 288 EXL3 4-bit
experts (hidden 4096, intermediate 1024; 76 GB of experts in all) and its own router, Zipf(1.2)-skewed expert
popularity produced by the router GEMM itself, each layer's routed output added to the residual stream that feeds
the next layer, the whole forward captured as one HIP graph.

Checks: every graph replay (with eager work and host synchronisation between replays) equals the eager forward bit
for bit; and for two sampled layers, the router picks of the layer's actual input are bit-exact against the oracle
router, and two sampled tokens' routed outputs match the float64 oracle (rel_l2 <= 5e-3), the reference's default
decode numerics (the oracle's tf_parity mode, TF_PARITY=1) within the reference's own build-vs-production bar E.1
(rel_l2 <= 2e-3 and per token row <= 1e-2, code/fork/docs/DESIGN.md:520-523), and, elementwise within rtol 2e-2 /
atol 1e-3 on the bf16 output, the oracle at the decode kernels' rounding points. Elementwise against float64 and
against tf_parity the layer-41 outputs (RMS ~1.7; the fp16 intermediates of either numerics move outputs near zero by
more than 1e-3) do not hold that bar everywhere; the share of elements outside it and the worst element are printed.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe, routing

pytestmark = pytest.mark.gpu

K, N, E, TOPK, LAYERS, T = 4096, 1024, 288, 8, 42, 8


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def test_stacked_decode_graph(cuda):
    from mi355moe import ops, synthetic
    _say(f"stacked decode: {LAYERS} layers x {E} experts, T={T}, building weights")
    layers, routers = [], []
    for l in range(LAYERS):
        layers.append(synthetic.exl3_layer(E, K, N, seed=700 + l, device=cuda))
        routers.append(synthetic.zipf_router(E, K, seed=800 + l, rank_seed=900 + l, device=cuda))
    xs = [synthetic.zipf_activations(T, K, seed=950, device=cuda)] + [
        torch.empty(T, K, dtype=torch.bfloat16, device=cuda) for _ in range(LAYERS)]
    outs = [torch.empty(T, K, dtype=torch.bfloat16, device=cuda) for _ in range(LAYERS)]
    ids = [torch.empty(T, TOPK, dtype=torch.int32, device=cuda) for _ in range(LAYERS)]
    wts = [torch.empty(T, TOPK, dtype=torch.float32, device=cuda) for _ in range(LAYERS)]

    def forward():
        for l in range(LAYERS):
            w, b = routers[l]
            ops.moe_layer(layers[l], xs[l], router_w=w, topk=TOPK, bias=b, routed_scale=2.5, limit=10.0,
                          out=outs[l], picks_out=(ids[l], wts[l]))
            torch.add(xs[l], outs[l], out=xs[l + 1])

    forward()
    torch.cuda.synchronize()
    ref = [x.clone() for x in xs]
    ref_ids = [i.clone() for i in ids]
    distinct = [int(torch.unique(i).numel()) for i in ids]
    _say(f"  distinct experts per layer: mean {sum(distinct) / LAYERS:.1f}, min {min(distinct)}, max {max(distinct)}")
    assert sum(distinct) / LAYERS < 50          # the Zipf skew concentrates the picks (uniform routing gives ~58)

    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        forward()
    torch.cuda.current_stream(cuda).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward()
    scratch = synthetic.activations(300, K, seed=3, device=cuda)
    sids = synthetic.random_ids(300, E, TOPK, seed=4, device=cuda)
    sw = synthetic.softmax_weights(300, TOPK, seed=5, device=cuda)
    for rep in range(3):
        for x in xs[1:]:
            x.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for l in range(LAYERS):
            assert torch.equal(ids[l], ref_ids[l]), (rep, l)
        assert all(torch.equal(a, b) for a, b in zip(xs, ref)), rep
        ops.moe_forward_ids(layers[0], scratch, sids, sw)          # eager work between replays
        torch.cuda.synchronize()
    _say("  graph replays equal the eager forward")

    for l in (0, LAYERS - 1):
        w, b = routers[l]
        x_l = ref[l]
        lg = routing.router_logits(x_l.float().cpu().numpy(), w.float().cpu().numpy())
        rid, rw = routing.topk_sigmoid_bias(lg, b.cpu().numpy(), TOPK, 2.5)
        assert np.array_equal(ids[l].cpu().numpy(), rid), l
        assert np.array_equal(wts[l].cpu().numpy(), rw), l
        sample = np.array([0, T - 1])
        ids_s = rid[sample]
        used = np.unique(ids_s)
        remap = {int(e): i for i, e in enumerate(used)}
        local = np.vectorize(remap.get)(ids_s)
        sel = torch.as_tensor(used, dtype=torch.long, device=cuda)
        lay = {k: getattr(layers[l], k).index_select(0, sel).cpu().numpy() for k in
               ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
        tok, exx, w16 = moe.pairs_from_routing(local, rw[sample], len(used), TOPK)
        x16 = x_l[torch.from_numpy(sample).to(cuda)].to(torch.float16).cpu().numpy()
        ref64 = moe.forward(lay, x16, tok, exx, w16, 10.0, "f64")
        ref_k = moe.forward(lay, x16, tok, exx, w16, 10.0, "decode_x")
        ref_tf = moe.forward(lay, x16, tok, exx, w16, 10.0, "tf_parity")
        got = outs[l][torch.from_numpy(sample).to(cuda)].float().cpu().numpy()
        r, rk, rt = _rel(got, ref64), _rel(got, ref_k), _rel(got, ref_tf)
        rows = max(_rel(got[i], ref_tf[i]) for i in range(sample.size))
        _say(f"  layer {l}: tokens {sample.tolist()} rel_l2 vs float64 {r:.3e}, vs the kernels' rounding {rk:.3e}, "
             f"vs the reference's default numerics {rt:.3e} (worst row {rows:.3e})")
        assert r <= 5e-3, (l, r)
        assert rt <= 2e-3 and rows <= 1e-2, (l, rt, rows)
        assert np.allclose(got, ref_k, rtol=2e-2, atol=1e-3), l
        for name, rv in (("float64", ref64), ("tf_parity", ref_tf)):
            bad = ~np.isclose(got, rv, rtol=2e-2, atol=1e-3)
            i = int(np.argmax(np.abs(got - rv) - 2e-2 * np.abs(rv)))
            _say(f"    elementwise vs {name}: {bad.mean():.4%} outside rtol 2e-2 / atol 1e-3; worst: token "
                 f"{sample[i // K]} column {i % K} got {got.flat[i]:.5f} ref {rv.flat[i]:.5f}")
    del graph, layers, routers, xs, outs, ref
    torch.cuda.empty_cache()
