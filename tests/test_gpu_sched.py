"""GPU checks of the one-launch schedule of the grouped path (MI355MOE_OPT_PERSISTENT): gate/up and down tiles taken
from one ticket counter, a down tile waiting on its segment's gate/up count. Same tile code, so the output equals
the separate launches' bit for bit: uniform and Zipf routing, full size, fewer segments than compute units, one-block
routing, bf16 accumulators, lags that make down tiles wait, stage-split calls (the call's gather zeroes the
control words), and the trellis-sourced e4m3 variant with its down-input quantisation inside the launch."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _separate_by_default(monkeypatch):
    """The reference calls run the separate launches (the library would take the schedule by itself for calls on
    the 256-row tiles); the calls under test force it with persistent=True."""
    monkeypatch.setenv("MI355MOE_SCHED", "separate")


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("n,K,N,T,routing,uniform", [(16, 1024, 512, 700, "uniform", False),
                                                     (64, 1024, 512, 4096, "zipf", True),
                                                     (4, 1024, 256, 20, "uniform", False),
                                                     (16, 1024, 512, 100, "zipf", False),
                                                     (288, 4096, 1024, 8192, "uniform", True)])
def test_persistent_equals_separate_launches(cuda, n, K, N, T, routing, uniform):
    from mi355moe import _lib, ops, synthetic
    _say(f"persistent schedule n={n} K={K} N={N} T={T} {routing} uniform_suh={uniform}")
    ex = synthetic.calibrated_layer(n, K, N, seed=n + T, device=cuda, uniform_suh=uniform)
    topk = min(8, n)
    x = synthetic.activations(T, K, seed=T + 1, device=cuda)
    ids = (synthetic.zipf_ids(T, n, topk, seed=T + 2, device=cuda) if routing == "zipf" else
           synthetic.random_ids(T, n, topk, seed=T + 2, device=cuda))
    ids[0, 1] = -1
    w = synthetic.softmax_weights(T, topk, seed=T + 3, device=cuda)
    for b16 in (False, True):
        ref = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL, bf16_contrib=b16)
        got = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL, bf16_contrib=b16,
                                  persistent=True)
        again = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL,
                                    bf16_contrib=b16, persistent=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), (got - ref).abs().max().item()
        assert torch.equal(again, ref)


@pytest.mark.parametrize("lag", [1, 3, 12])
def test_persistent_lag_waits(cuda, lag, monkeypatch):
    """Small lags put a segment's down tiles right behind its gate/up tiles, so down tiles wait on the counts."""
    from mi355moe import _lib, ops, synthetic
    _say(f"persistent schedule, lag {lag}")
    monkeypatch.setenv("MI355MOE_SCHED_LAG", str(lag))
    n, K, N, T = 64, 2048, 512, 3000
    ex = synthetic.calibrated_layer(n, K, N, seed=11, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=12, device=cuda)
    ids = synthetic.zipf_ids(T, n, 8, seed=13, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=14, device=cuda)
    ref = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    for _ in range(2):
        got = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL, persistent=True)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (got - ref).abs().max().item()


def test_persistent_stage_split_calls(cuda):
    """Route once, then the gate/up + down + combine stages twice with new activations: each call's gather zeroes the
    ticket and segment counts the previous launch left, and the result equals the separate launches."""
    from mi355moe import _lib, ops, synthetic
    _say("persistent schedule, stage-split calls")
    n, K, N, T = 32, 1024, 512, 1500
    ex = synthetic.calibrated_layer(n, K, N, seed=5, device=cuda)
    ids = synthetic.random_ids(T, n, 8, seed=6, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=7, device=cuda)
    kw = dict(path=_lib.PATH_PREFILL, persistent=True)
    out = torch.empty(T, K, dtype=torch.float32, device=cuda)
    x0 = synthetic.activations(T, K, seed=8, device=cuda)
    ops.moe_forward_ids(ex, x0, ids, w, out=out, stages=_lib.STAGE_ROUTE, **kw)
    for seed in (9, 10):
        x = synthetic.activations(T, K, seed=seed, device=cuda)
        ops.moe_forward_ids(ex, x, ids, w, out=out, stages=_lib.STAGE_GATEUP | _lib.STAGE_DOWN | _lib.STAGE_COMBINE,
                            **kw)
        ref = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


@pytest.mark.parametrize("n,K,N,T,routing,down16", [(16, 1024, 512, 700, "uniform", False),
                                                    (16, 1024, 512, 700, "uniform", True),
                                                    (64, 1024, 512, 4096, "zipf", False),
                                                    (4, 1024, 256, 20, "uniform", False),
                                                    (8, 1024, 2048, 600, "uniform", False),
                                                    (288, 4096, 1024, 8192, "uniform", False)])
def test_persistent_e4m3_equals_separate_launches(cuda, n, K, N, T, routing, down16):
    """The trellis-sourced e4m3 variant: the segment's last gate/up item quantises its rows' down inputs in the same
    launch (or, DOWN16, the gate/up items write the fp16 down input directly)."""
    from mi355moe import ops, synthetic
    _say(f"persistent schedule e4m3 n={n} K={K} N={N} T={T} {routing} down16={down16}")
    ex = synthetic.calibrated_layer(n, K, N, seed=n + T + 1, device=cuda, uniform_suh=True)
    topk = min(8, n)
    x = synthetic.activations(T, K, seed=T + 5, device=cuda)
    ids = (synthetic.zipf_ids(T, n, topk, seed=T + 6, device=cuda) if routing == "zipf" else
           synthetic.random_ids(T, n, topk, seed=T + 6, device=cuda))
    w = synthetic.softmax_weights(T, topk, seed=T + 7, device=cuda)
    ref = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32, down16=down16)
    for _ in range(2):
        got = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32, down16=down16, persistent=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), (got - ref).abs().max().item()


@pytest.mark.parametrize("lag", [1, 4])
def test_persistent_e4m3_lag_waits(cuda, lag, monkeypatch):
    """Small lags make the down items wait on segments whose quantisation runs in the same launch."""
    from mi355moe import ops, synthetic
    _say(f"persistent schedule e4m3, lag {lag}")
    monkeypatch.setenv("MI355MOE_SCHED_LAG", str(lag))
    n, K, N, T = 48, 2048, 512, 3000
    ex = synthetic.calibrated_layer(n, K, N, seed=31, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=32, device=cuda)
    ids = synthetic.zipf_ids(T, n, 8, seed=33, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=34, device=cuda)
    ref = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32)
    got = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32, persistent=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (got - ref).abs().max().item()


def test_automatic_choice_equals_separate_launches(cuda, monkeypatch):
    """Without the option, a call on the 256-row tiles takes the schedule by itself; MI355MOE_SCHED=separate turns
    that off. Both give the same bits."""
    from mi355moe import _lib, ops, synthetic
    _say("automatic one-launch choice")
    n, K, N, T = 32, 1024, 512, 4000
    ex = synthetic.calibrated_layer(n, K, N, seed=21, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=22, device=cuda)
    ids = synthetic.random_ids(T, n, 8, seed=23, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=24, device=cuda)
    ref = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    monkeypatch.delenv("MI355MOE_SCHED")
    got = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("down16", [False, True])
def test_e4m3_extension_fused_takes_the_schedule(cuda, monkeypatch, down16):
    """The e4m3 extension's fused entry over its row tables: a call on the 256-row tiles runs the one-launch schedule
    by itself (the e4m3 down GEMM with its in-launch quantisation, and DOWN16) and gives the separate launches'
    bits."""
    from mi355moe import e4m3_ext, synthetic
    _say(f"e4m3 extension fused, one-launch schedule, down16={down16}")
    n, K, N, T = 8, 1024, 512, 600
    ex = synthetic.calibrated_layer(n, K, N, seed=41, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=42, device=cuda)
    ids = synthetic.random_ids(T, n, 8, seed=43, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=44, device=cuda)
    ref = e4m3_ext.run(x, ids, w, ex, 10.0, sched={"down16": down16})
    monkeypatch.delenv("MI355MOE_SCHED")
    for _ in range(2):
        got = e4m3_ext.run(x, ids, w, ex, 10.0, sched={"down16": down16})
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


def _random_cases(count=14, seed=2026):
    import random
    rnd = random.Random(seed)
    out = []
    for i in range(count):
        n = rnd.choice([2, 3, 5, 8, 13, 24, 40, 64])
        K = 256 * rnd.randint(1, 8)
        N = 128 * rnd.randint(1, 8)
        T = rnd.randint(1, 1500)
        out.append((i, n, K, N, T, rnd.choice(["uniform", "zipf"]), rnd.choice(["e3", "e4m3", "down16"]),
                    rnd.random() < 0.3, rnd.choice([0, 1, 2, 5])))
    return out


@pytest.mark.parametrize("i,n,K,N,T,routing,numerics,b16,lag", _random_cases())
def test_persistent_random_shapes(cuda, monkeypatch, i, n, K, N, T, routing, numerics, b16, lag):
    """Seeded ragged shapes (hidden 256..2048, intermediate 128..1024, 1..1500 tokens, 2..64 experts, lags 0..5):
    the forced one-launch schedule gives the separate launches' bits in every numerics."""
    from mi355moe import _lib, ops, synthetic
    _say(f"random case {i}: n={n} K={K} N={N} T={T} {routing} {numerics} bf16={b16} lag={lag}")
    monkeypatch.setenv("MI355MOE_SCHED_LAG", str(lag))
    ex = synthetic.calibrated_layer(n, K, N, seed=100 + i, device=cuda, uniform_suh=(i % 2 == 0))
    topk = min(8, n)
    x = synthetic.activations(T, K, seed=200 + i, device=cuda)
    ids = (synthetic.zipf_ids(T, n, topk, seed=300 + i, device=cuda) if routing == "zipf" else
           synthetic.random_ids(T, n, topk, seed=300 + i, device=cuda))
    w = synthetic.softmax_weights(T, topk, seed=400 + i, device=cuda)
    if numerics == "e3":
        call = lambda pers: ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL,
                                                bf16_contrib=b16, persistent=pers)
    else:
        call = lambda pers: ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32, bf16_contrib=b16,
                                                     down16=numerics == "down16", persistent=pers)
    ref = call(False)
    got = call(True)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref), (got - ref).abs().max().item()


def test_schedule_in_a_replayed_graph(cuda, monkeypatch):
    """A grouped call on the 256-row tiles (the one-launch schedule, taken by itself) captured in a HIP graph: every
    replay, with eager calls between replays, equals the separate launches (the gather re-zeroes the control words
    inside the graph)."""
    from mi355moe import _lib, ops, synthetic
    _say("one-launch schedule, graph replays")
    n, K, N, T = 16, 1024, 512, 700
    ex = synthetic.calibrated_layer(n, K, N, seed=51, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=52, device=cuda)
    ids = synthetic.random_ids(T, n, 8, seed=53, device=cuda)
    w = synthetic.softmax_weights(T, 8, seed=54, device=cuda)
    ref = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    monkeypatch.delenv("MI355MOE_SCHED")
    ops.reserve(ex, T)
    out = torch.empty(T, K, dtype=torch.float32, device=cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.moe_forward_ids(ex, x, ids, w, out=out, path=_lib.PATH_PREFILL)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.moe_forward_ids(ex, x, ids, w, out=out, path=_lib.PATH_PREFILL)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)   # eager between
        torch.cuda.synchronize()
