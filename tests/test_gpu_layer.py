"""GPU parity of the whole-layer entry (mi355moe_moe_layer): router logits, top-k, permutation, expert GEMMs and
combine in one call, against the separate entry points chained (each of which is pinned against the oracle
elsewhere) and, for the routing, against the oracle directly. The outputs must equal the chained entries bit for
bit, on repeated calls, under graph replay, and with other calls sharing the workspace in between.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import routing

pytestmark = pytest.mark.gpu

K, N, E = 4096, 1024, 288


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def model(cuda):
    from mi355moe import synthetic
    ex = synthetic.exl3_layer(E, K, N, seed=41, device=cuda)
    w, b = synthetic.router(E, K, seed=42, device=cuda)
    return ex, w, b


def _chained(ex, x, w, b, topk, scale, logits=None, out_dtype=None):
    from mi355moe import ops
    lg = ops.router_logits(x, w) if logits is None else logits
    ids, wts = ops.router_topk(lg, topk, b, routed_scale=scale)
    return ops.moe_forward_ids(ex, x, ids, wts, out_dtype=out_dtype), ids, wts


@pytest.mark.parametrize("T,given_logits", [(1, False), (8, False), (8, True), (64, False), (65, False)])
def test_layer_equals_chained_entries(cuda, model, T, given_logits):
    from mi355moe import ops, synthetic
    ex, w, b = model
    _say(f"moe_layer T={T} logits_given={given_logits}")
    x = synthetic.activations(T, K, seed=T + 3, device=cuda)
    lg = ops.router_logits(x, w) if given_logits else None
    ref, rid, rw = _chained(ex, x, w, b, 8, 2.5, logits=lg)
    for out_dtype in (torch.bfloat16, torch.float32):
        ref_o = ref if out_dtype == torch.bfloat16 else _chained(ex, x, w, b, 8, 2.5, logits=lg, out_dtype=out_dtype)[0]
        got, ids, wts = ops.moe_layer(ex, x, router_w=None if given_logits else w, logits=lg, topk=8, bias=b,
                                      routed_scale=2.5, out_dtype=out_dtype, return_picks=True)
        torch.cuda.synchronize()
        assert torch.equal(ids, rid)
        assert torch.equal(wts, rw)
        assert torch.equal(got, ref_o), out_dtype


@pytest.mark.parametrize("E2,topk,T", [(1024, 32, 5), (32, 4, 3), (320, 8, 16), (321, 8, 16)])
def test_layer_router_widths(cuda, E2, topk, T):
    """Router widths on both sides of the one-wave top-k's 320-candidate unroll, and top-32 of 1024: the layer's
    picks against the oracle router and its output against the chained entry points."""
    from mi355moe import ops, synthetic
    K2, N2 = 512, 256
    _say(f"moe_layer E={E2} topk={topk} T={T}")
    ex = synthetic.exl3_layer(E2, K2, N2, seed=E2 + topk, device=cuda, svh_scale=0.05)
    w, b = synthetic.router(E2, K2, seed=E2 + 1, device=cuda)
    x = synthetic.activations(T, K2, seed=E2 + 2, device=cuda)
    got, ids, wts = ops.moe_layer(ex, x, router_w=w, topk=topk, bias=b, routed_scale=2.5, return_picks=True)
    ref, rid, rw = _chained(ex, x, w, b, topk, 2.5)
    torch.cuda.synchronize()
    lg = routing.router_logits(x.float().cpu().numpy(), w.float().cpu().numpy())
    oid, ow = routing.topk_sigmoid_bias(lg, b.float().cpu().numpy(), topk, 2.5)
    assert np.array_equal(ids.cpu().numpy(), oid)
    assert np.array_equal(wts.cpu().numpy(), ow)
    assert torch.equal(ids, rid) and torch.equal(wts, rw)
    assert torch.equal(got, ref)


def test_layer_routing_vs_oracle(cuda, model):
    from mi355moe import ops, synthetic
    ex, w, b = model
    T = 8
    _say("moe_layer picks vs the oracle router")
    x = synthetic.activations(T, K, seed=77, device=cuda)
    _, ids, wts = ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, return_picks=True)
    lg = routing.router_logits(x.float().cpu().numpy(), w.float().cpu().numpy())
    rid, rw = routing.topk_sigmoid_bias(lg, b.float().cpu().numpy(), 8, 2.5)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(wts.cpu().numpy(), rw)


def test_layer_repeat_graph_and_shared_workspace(cuda, model):
    from mi355moe import ops, synthetic
    ex, w, b = model
    T = 8
    _say("moe_layer repeats, graph replay, shared workspace")
    x = synthetic.activations(T, K, seed=91, device=cuda)
    a = ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5)
    for _ in range(3):
        assert torch.equal(ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5), a)
    # a larger call of another entry point through the same workspace, then the layer again
    xb = synthetic.activations(300, K, seed=92, device=cuda)
    ids = synthetic.random_ids(300, E, 8, seed=93, device=cuda)
    wts = synthetic.softmax_weights(300, 8, seed=94, device=cuda)
    ops.moe_forward_ids(ex, xb, ids, wts)
    assert torch.equal(ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5), a)
    out = torch.empty_like(a)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, out=out)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, a), i
        ops.moe_forward_ids(ex, xb, ids, wts)                # eager work between replays
        torch.cuda.synchronize()


def test_graph_survives_workspace_growth(cuda, model):
    """A decode layer call captured in a graph, then an eager call that outgrows the workspace (T=8192 on the
    grouped tier): the larger call gets a new workspace and the captured graph keeps replaying into the old one,
    which stays allocated; every replay equals the eager result."""
    from mi355moe import ops, synthetic
    ex, w, b = model
    T = 8
    _say("graph capture, workspace growth, replay")
    x = synthetic.activations(T, K, seed=95, device=cuda)
    a = ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5)
    out = torch.empty_like(a)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.moe_layer(ex, x, router_w=w, topk=8, bias=b, routed_scale=2.5, out=out)
    before = ops.workspace(cuda, 0)
    xb = synthetic.activations(8192, K, seed=96, device=cuda)
    ids = synthetic.random_ids(8192, E, 8, seed=97, device=cuda)
    wts = synthetic.softmax_weights(8192, 8, seed=98, device=cuda)
    need = ops.workspace_bytes(ex, 8192, 8)
    ops.reserve_workspace(cuda, max(need, before.numel() + (64 << 20)))   # grows, whatever ran before this test
    assert ops.workspace(cuda, 0).data_ptr() != before.data_ptr()
    del before
    big = ops.moe_forward_ids(ex, xb, ids, wts)
    torch.cuda.synchronize()
    assert torch.isfinite(big.float()).all()
    filler = torch.full((64 << 20,), 7, dtype=torch.uint8, device=cuda)   # memory handed out after the growth
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, a), i
        ops.moe_forward_ids(ex, xb, ids, wts)
        torch.cuda.synchronize()
    del filler
