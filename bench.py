#!/usr/bin/env python3
"""Benchmark of the routed-MoE layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|decode|prefill|fp8|e4m3t|stack]

Default workload (one "step" = one MoE layer call): the decode MoE layer, T=8 tokens, hidden 4096, 288 experts,
sigmoid router + bias, top-8, routed scale 2.5, intermediate 1024 (one tensor-parallel rank's shard), EXL3 4-bit
synthetic experts. A step runs the router GEMM, the sigmoid/bias top-k, the permutation, the grouped gate/up and
down trellis GEMVs and the combine, replayed from one HIP graph holding a layer call for every (layer, input) pair (as a
served model's forward graph holds its layers). Steps cycle over
several distinct layers so every step streams cold expert weights (the set exceeds the 256 MiB last-level cache).

Printed (one JSON line): value = achieved HBM GB/s over the timed steps, counting per step the bytes a layer call
must read: D distinct routed experts x (6,291,456 B trellis + 30,720 B fp16 scales) + router weight and bias +
activations in and out. The roofline entry times the dominant kernel (the grouped gate/up GEMV) alone with HIP
events on the launch stream. cpu_baseline times the oracle's C port of the same layer call on the host cores.
Every workload runs SETTLE_MS of untimed back-to-back calls before its warm-up steps, so that the timed steps see the
clock of a busy GPU rather than the transient that follows the idle spell of building the workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "glm-5.3-flash-dgx-spark-vllm-optimization_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer µs @T=8 + achieved HBM GB/s; prefill MoE tokens/s @T=8192"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
K, N, E, TOPK, SCALE, LIMIT = 4096, 1024, 288, 8, 2.5, 10.0
EXPERT_TRELLIS = 3 * K * N // 2            # 6,291,456
EXPERT_SCALES = 2 * (3 * K + 3 * N)        # 30,720


# A spin kernel ahead of each event-bracketed launch keeps the stream busy while the host enqueues the start event
# and the launch, so the start event is timestamped right before the kernel runs, not while the GPU idles waiting
# for the host.
HOLD_CYCLES = 200_000


# Untimed work, in ms of GPU time, run right before each workload's warm-up steps. After an idle spell (the host
# building the workload) the first ~25 ms of work runs at a transient clock: T=8192 prefill calls measured 2.68,
# 3.11, 2.82, 2.64, 2.53, 2.61, 2.45, ... then ~2.40 ms, decode calls ~5 % slow for the first ~15 ms. The timed steps
# follow SETTLE_MS of back-to-back calls, so they measure the sustained rate of a busy GPU.
SETTLE_MS = 60.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def settle(torch, fn, ms=SETTLE_MS):
    """Run fn() back to back until ms of GPU time have passed (event-timed in chunks)."""
    done, n = 0.0, 1
    while done < ms:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        t = a.elapsed_time(b)
        done += t
        n = max(1, min(4 * n, int(n * (ms - done) / max(t, 1e-3)) + 1))


def build_problem(torch, synthetic, ops, dev, T, n_layers, n_inputs):
    layers, routers, xs = [], [], []
    for l in range(n_layers):
        w, b = synthetic.router(E, K, seed=100 + l, device=dev)
        routers.append((w, b))
        layers.append(synthetic.exl3_layer(E, K, N, seed=200 + l, device=dev))
    for i in range(n_inputs):
        xs.append(synthetic.activations(T, K, seed=300 + i, device=dev))
    return layers, routers, xs


def step_fn(ops, layer, router, x, bufs):
    """One decode layer call from hidden states: the whole-layer entry (router GEMV, top-k, permutation, expert
    GEMVs, combine)."""
    w, b = router
    _, ids, wts = ops.moe_layer(layer, x, router_w=w, topk=TOPK, bias=b, routed_scale=SCALE, limit=LIMIT,
                                out=bufs["out"], picks_out=(bufs["ids"], bufs["wts"]))
    return ids, wts


def cpu_baseline(torch, layer, x, ids, wts, threads, min_seconds=10.0):
    """The oracle's C port of one full layer call (decode rounding points) on the host, repeated >= min_seconds."""
    import numpy as np
    from oracle import moe, routing
    ids_np = ids.cpu().numpy()
    used = np.unique(ids_np[ids_np >= 0])
    remap = {int(e): i for i, e in enumerate(used)}
    sel = torch.as_tensor(used, dtype=torch.long, device=layer.device)
    lay = {k: getattr(layer, k).index_select(0, sel).cpu().numpy() for k in
           ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
    local = np.vectorize(lambda e: remap.get(int(e), len(used)))(ids_np)
    tok, ex, w16 = moe.pairs_from_routing(local, wts.cpu().numpy(), len(used), ids_np.shape[1])
    x16 = x.to(torch.float16).cpu().numpy()
    moe.lib()
    reps, t0 = 0, time.perf_counter()
    while True:
        moe.forward(lay, x16, tok, ex, w16, LIMIT, "decode", threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_seconds and reps >= 2:
            break
    del routing
    return el / reps, reps, len(used)


def _repeat(fn, min_seconds=10.0):
    """Run fn until at least min_seconds have passed (two runs at least); (seconds per run, runs)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_seconds and reps >= 2:
            return el / reps, reps


def cpu_threads() -> int:
    """Threads for the CPU baselines: every host core this process may run on, capped by OMP_NUM_THREADS where the
    environment sets it (a shared host gives each GPU's jobs a share of its cores and says so there)."""
    avail = len(os.sched_getaffinity(0))
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(avail, omp) if omp > 0 else avail)


def host_cores() -> dict:
    """The host's core count (os.cpu_count), the cores this process may run on, and OMP_NUM_THREADS."""
    return {"host_cores": os.cpu_count(), "cores_available": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def _sample_pairs(ids, wts, n_tok):
    """The first n_tok tokens' routing as (used experts, local ids [n_tok, topk], weights) with the experts renumbered
    0..len(used)-1 in id order."""
    import numpy as np
    ids_np = ids[:n_tok].cpu().numpy()
    used = np.unique(ids_np[ids_np >= 0])
    remap = {int(e): i for i, e in enumerate(used)}
    local = np.vectorize(lambda e: remap.get(int(e), len(used)))(ids_np)
    return used, local, wts[:n_tok].cpu().numpy()


def cpu_baseline_prefill(torch, layer, x, ids, wts, threads, n_tok=512):
    """The oracle's C port (E3 rounding points, OpenMP) on a reduced sample of the prefill workload: its first n_tok
    tokens with their routing. At n_tok = 512 (4,096 pairs) every one of the 288 experts is routed, so each is decoded
    once, as in the full T=8192 call; tokens/s of the sample is therefore a lower bound on the full call's (the decode
    is amortised over 16x fewer tokens)."""
    from oracle import moe
    used, local, w = _sample_pairs(ids, wts, n_tok)
    sel = torch.as_tensor(used, dtype=torch.long, device=layer.device)
    lay = {k: getattr(layer, k).index_select(0, sel).cpu().numpy() for k in
           ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
    tok, ex, w16 = moe.pairs_from_routing(local, w, len(used), local.shape[1])
    x16 = x[:n_tok].to(torch.float16).cpu().numpy()
    moe.lib()
    sec, reps = _repeat(lambda: moe.forward(lay, x16, tok, ex, w16, LIMIT, "e3", threads=threads))
    return {"value": round(n_tok / sec, 2), "unit": "tokens/s", "cores": threads, **host_cores(), "kind": "port",
            "seconds_per_call": round(sec, 3),
            "sample": f"{reps} repetitions of the first {n_tok} tokens of the T=8192 prefill call ({len(used)} "
                      "distinct experts, each decoded once per repetition) through the oracle's C port "
                      f"(oracle/csrc/oracle.c, E3 rounding points, OpenMP {threads} threads); a lower bound on the "
                      "full call's tokens/s"}


def cpu_baseline_fp8(torch, layer, x, ids, wts, threads, n_tok=256):
    """The oracle's C port of the block-scaled e4m3 layer (weights dequantised per 128x128 block, fp32 sums) on the
    first n_tok tokens of the e4m3 workload with their routing (at 256 tokens all 288 experts are routed)."""
    from oracle import e4m3
    used, local, w = _sample_pairs(ids, wts, n_tok)
    sel = torch.as_tensor(used, dtype=torch.long, device=layer.w13.device)
    lay = {"w13": layer.w13.index_select(0, sel).cpu().numpy(), "w13_scale": layer.w13_scale.index_select(0, sel).cpu().numpy(),
           "w2": layer.w2.index_select(0, sel).cpu().numpy(), "w2_scale": layer.w2_scale.index_select(0, sel).cpu().numpy()}
    tok, ex, pw = e4m3.pairs_fp32(local, w, len(used))
    xs = x[:n_tok].float().cpu().numpy()
    sec, reps = _repeat(lambda: e4m3.forward(lay, xs, tok, ex, pw, LIMIT, "kernel", threads=threads))
    return {"value": round(n_tok / sec, 2), "unit": "tokens/s", "cores": threads, **host_cores(), "kind": "port",
            "seconds_per_call": round(sec, 3),
            "sample": f"{reps} repetitions of the first {n_tok} tokens of the T=2048 e4m3 call ({len(used)} distinct "
                      "experts) through the oracle's C port (oracle/csrc/fp8.c: dequantise-then-fp32 GEMM per "
                      f"128-block, OpenMP {threads} threads)"}


def _bracket(torch, fn):
    """(start, end) events around fn()'s launches on the current stream; a spin kernel ahead keeps the stream busy
    while the host enqueues them, so the start event is stamped right before the first bracketed kernel runs."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(HOLD_CYCLES)
    a.record()
    fn()
    b.record()
    return a, b


def run_decode(args, torch, mi355moe, dev):
    from mi355moe import _lib, ops, synthetic
    T = args.tokens
    n_layers, n_inputs = args.layers, 4
    log(f"[bench] building {n_layers} layers x {E} experts ({n_layers * E * (EXPERT_TRELLIS + EXPERT_SCALES) / 1e9:.1f}"
        " GB) ...")
    layers, routers, xs = build_problem(torch, synthetic, ops, dev, T, n_layers, n_inputs)
    combos = [(l, i) for i in range(n_inputs) for l in range(n_layers)]
    bufs = {c: {"out": torch.empty(T, K, dtype=torch.bfloat16, device=dev),
                "ids": torch.empty(T, TOPK, dtype=torch.int32, device=dev),
                "wts": torch.empty(T, TOPK, dtype=torch.float32, device=dev)} for c in combos}
    # eager pass: routing of every combo (distinct experts per call) and workspace sizing before capture
    info = {}
    for c in combos:
        ids, wts = step_fn(ops, layers[c[0]], routers[c[0]], xs[c[1]], bufs[c])
        torch.cuda.synchronize()
        d = int(torch.unique(ids).numel())
        info[c] = (d, ids.clone(), wts.clone())
    graphs = {}
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for c in combos:
            step_fn(ops, layers[c[0]], routers[c[0]], xs[c[1]], bufs[c])
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    for c in combos:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step_fn(ops, layers[c[0]], routers[c[0]], xs[c[1]], bufs[c])
        graphs[c] = g
    # every combo's layer call in one graph, as a served model's forward graph holds its layers: the timed steps
    # replay it whole (one graph launch per len(combos) layer calls), the remainder through the per-combo graphs
    chain = torch.cuda.CUDAGraph()
    with torch.cuda.graph(chain):
        for c in combos:
            step_fn(ops, layers[c[0]], routers[c[0]], xs[c[1]], bufs[c])
    torch.cuda.synchronize()
    # correctness guard: a replay equals the eager result
    ref = bufs[combos[0]]["out"].clone()
    graphs[combos[0]].replay()
    torch.cuda.synchronize()
    if not torch.equal(ref, bufs[combos[0]]["out"]):
        raise RuntimeError("graph replay differs from the eager step")
    refs = []
    for c in combos:
        graphs[c].replay()
        torch.cuda.synchronize()
        refs.append(bufs[c]["out"].clone())
    chain.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(r, bufs[c]["out"]) for r, c in zip(refs, combos)):
        raise RuntimeError("the chained graph differs from the per-call graphs")

    def step_bytes(c):
        d = info[c][0]
        return d * (EXPERT_TRELLIS + EXPERT_SCALES) + E * K * 2 + E * 4 + 2 * T * K * 2

    settle(torch, chain.replay)
    for w in range(args.warmup):
        graphs[combos[w % len(combos)]].replay()
    chain.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    total_bytes = 0
    dsum = 0
    k = 0
    while k + len(combos) <= args.steps:
        chain.replay()
        for c in combos:
            total_bytes += step_bytes(c)
            dsum += info[c][0]
        k += len(combos)
    for c in combos[:args.steps - k]:
        graphs[c].replay()
        total_bytes += step_bytes(c)
        dsum += info[c][0]
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1)
    us_per_step = ms * 1000.0 / args.steps
    gbs = total_bytes / (ms / 1000.0) / 1e9

    # the GEMVs alone: route staged untimed, then the gate/up launch and the down launch each event-bracketed
    gu_t, dn_t, gu_bytes, dn_bytes = [], [], [], []
    for k in range(args.steps):
        c = combos[k % len(combos)]
        d, ids, wts = info[c]
        lay, x = layers[c[0]], xs[c[1]]
        call = lambda st: ops.moe_forward_ids(lay, x, ids, wts, limit=LIMIT, out=bufs[c]["out"], stages=st)
        call(_lib.STAGE_ROUTE)
        gu_t.append(_bracket(torch, lambda: call(_lib.STAGE_GATEUP)))
        dn_t.append(_bracket(torch, lambda: call(_lib.STAGE_DOWN)))
        call(_lib.STAGE_COMBINE)
        P = T * TOPK
        # weights + scales of the d experts, the inputs read, the outputs written
        gu_bytes.append(d * (2 * K * N // 2 + 2 * (2 * K + 3 * N)) + T * K * 2 + P * N * 2)
        dn_bytes.append(d * (N * K // 2 + 2 * K) + P * N * 2 + P * K * 4)
    torch.cuda.synchronize()
    gu_t = [a.elapsed_time(b) * 1000.0 for a, b in gu_t]
    dn_t = [a.elapsed_time(b) * 1000.0 for a, b in dn_t]
    gu_avg_us, dn_avg_us = sum(gu_t) / len(gu_t), sum(dn_t) / len(dn_t)
    gu_gbs = (sum(gu_bytes) / len(gu_bytes)) / (gu_avg_us * 1e-6) / 1e9
    dn_gbs = (sum(dn_bytes) / len(dn_bytes)) / (dn_avg_us * 1e-6) / 1e9

    res = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"decode MoE layer T={T}: hidden {K}, {E} experts, sigmoid+bias top-{TOPK} x{SCALE}, "
                               f"intermediate {N}, EXL3 4-bit synthetic experts, {n_layers} layers cycled (cold)",
                   "tokens": T, "hidden": K, "experts": E, "topk": TOPK, "intermediate": N,
                   "graph": f"{len(combos)} layer calls per HIP graph"},
        "decode_us_per_layer": round(us_per_step, 2),
        "distinct_experts_mean": round(dsum / args.steps, 2),
        "hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": "dec_gateup_kernel", "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": _traffic(dsum / args.steps), "avg_launch_us": round(gu_avg_us, 2)},
        "roofline_down": {"bound": "hbm", "kernel": "dec_down_kernel", "achieved": round(dn_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dn_gbs / HBM_PEAK_GBS, 4),
                          "avg_launch_us": round(dn_avg_us, 2)},
        "wall_s": round(wall, 3),
        "settle_ms": SETTLE_MS,
    }
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        c = combos[0]
        sec, reps, d = cpu_baseline(torch, layers[c[0]], xs[c[1]], info[c][1], info[c][2], threads)
        res["cpu_block_a"] = cpu_block_a(torch, threads)
        res["cpu_baseline"] = {"value": round(step_bytes(c) / sec / 1e9, 4), "unit": "GB/s", "cores": threads,
                               **host_cores(),
                               "kind": "port", "seconds_per_call": round(sec, 4),
                               "sample": f"{reps} repetitions of one full T={T} layer call ({d} distinct experts) "
                                         "through the oracle's C port (oracle/csrc/oracle.c, decode rounding "
                                         f"points, OpenMP {threads} threads)"}
    return res


def _time_calls(torch, fn, n_layers, warmup, steps):
    """ms per call of fn(layer index), layers alternated, event-bracketed on the current stream."""
    for w in range(warmup):
        fn(w % n_layers)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for k in range(steps):
        fn(k % n_layers)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def run_prefill(args, torch, dev):
    """Prefill MoE chunk, T=8192 (same layer shapes), uniform-random router logits; the grouped MFMA path."""
    from mi355moe import _lib, ops, synthetic
    T = args.prefill_tokens
    n_layers = 2
    layers = [synthetic.exl3_layer(E, K, N, seed=400 + l, device=dev, uniform_suh=True) for l in range(n_layers)]
    x = synthetic.activations(T, K, seed=500, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(501)
    logits = [torch.rand(T, E, generator=g, device=dev) * 4 - 2 for _ in range(n_layers)]
    outs = [torch.empty(T, K, dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]

    def step(l):
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        ops.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l])
        return ids, wts

    info = [step(l) for l in range(n_layers)]
    torch.cuda.synchronize()
    pairs = [int((i >= 0).sum().item()) for i, _ in info]
    turn = [0]

    def step_next():
        step(turn[0] % n_layers)
        turn[0] += 1

    settle(torch, step_next)
    for w in range(max(2, args.warmup // 4)):
        step(w % n_layers)
    torch.cuda.synchronize()
    steps = max(4, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for k in range(steps):
        step(k % n_layers)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the stages alone: route staged untimed, then gather + gate/up, down and combine each event-bracketed
    gu, dn, cb, one = [], [], [], []
    for k in range(steps):
        l = k % n_layers
        ids, wts = info[l]
        call = lambda st: ops.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], stages=st)
        call(_lib.STAGE_ROUTE)
        gu.append(_bracket(torch, lambda: call(_lib.STAGE_GATEUP)))
        dn.append(_bracket(torch, lambda: call(_lib.STAGE_DOWN)))
        cb.append(_bracket(torch, lambda: call(_lib.STAGE_COMBINE)))
        # gather + the one-launch gate/up -> down kernel (both GEMM stages in one call)
        one.append(_bracket(torch, lambda: call(_lib.STAGE_GATEUP | _lib.STAGE_DOWN)))
    torch.cuda.synchronize()
    gu_ms = sum(a.elapsed_time(b) for a, b in gu) / len(gu)
    dn_ms = sum(a.elapsed_time(b) for a, b in dn) / len(dn)
    cb_ms = sum(a.elapsed_time(b) for a, b in cb) / len(cb)
    one_ms = sum(a.elapsed_time(b) for a, b in one) / len(one)

    if args.workload == "prefill-uniform":                # the profiling window: these calls only
        P = sum(pairs) / len(pairs)
        return {"prefill_ms_per_layer": round(ms, 4), "prefill_gateup_ms": round(gu_ms, 4),
                "prefill_gateup_frac": round(2.0 * P * K * 2 * N / (gu_ms / 1000.0) / 1e12 / MFMA_FP16_PEAK_TFLOPS,
                                             4),
                "prefill_down_ms": round(dn_ms, 4),
                "prefill_down_frac": round(2.0 * P * N * K / (dn_ms / 1000.0) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                "prefill_combine_ms": round(cb_ms, 4), "prefill_one_launch_ms": round(one_ms, 4)}

    def step_fold(l):
        # bf16 down accumulators, routed sum added into out (which stands for the shared experts' bf16 output)
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        ops.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], accumulate=True, bf16_contrib=True)

    ms_fold = _time_calls(torch, step_fold, n_layers, 2, steps)

    # the same layer call with gate/up and down as separate launches instead of the one-launch ticket-ordered
    # schedule the library takes by itself for this size (bit-identical output)
    prev = os.environ.get("MI355MOE_SCHED")
    os.environ["MI355MOE_SCHED"] = "separate"
    ms_sep = _time_calls(torch, step, n_layers, 2, steps)
    if prev is None:
        del os.environ["MI355MOE_SCHED"]
    else:
        os.environ["MI355MOE_SCHED"] = prev
    # the whole routed layer from the hidden states: router GEMM (float64 matrix cores), top-k, permutation, experts
    w_r, b_r = synthetic.router(E, K, seed=502, device=dev)

    def step_layer(l):
        ops.moe_layer(layers[l], x, router_w=w_r, topk=TOPK, bias=b_r, routed_scale=SCALE, limit=LIMIT, out=outs[l])

    ms_layer = _time_calls(torch, step_layer, n_layers, 2, steps)
    P = sum(pairs) / len(pairs)
    flops = 2.0 * P * (K * 2 * N + N * K)
    gu_flops = 2.0 * P * K * 2 * N
    dn_flops = 2.0 * P * N * K
    cb_bytes = int(P * K * 4 + T * K * 2)            # fp32 raw accumulators of every pair read, bf16 out written
    pe = run_prefill_per_expert_suh(args, torch, dev, x, logits, steps)
    extra = {}
    if not args.no_cpu_baseline:
        extra["cpu_baseline_prefill"] = cpu_baseline_prefill(torch, layers[0], x, info[0][0], info[0][1],
                                                             cpu_threads())
    return {**extra, "prefill_tokens_per_s": round(T / (ms / 1000.0), 1), "prefill_ms_per_layer": round(ms, 4),
            "prefill_bf16acc_fold_ms_per_layer": round(ms_fold, 4),
            "prefill_separate_launches_ms_per_layer": round(ms_sep, 4),
            "prefill_layer_with_router_ms": round(ms_layer, 4),
            "prefill_tflops": round(flops / (ms / 1000.0) / 1e12, 2),
            "roofline_prefill": {"bound": "mfma", "kernel": "pf_gateup_kernel (includes the gather launch)",
                                 "achieved": round(gu_flops / (gu_ms / 1000.0) / 1e12, 2),
                                 "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(gu_flops / (gu_ms / 1000.0) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                                 "avg_launch_us": round(gu_ms * 1000.0, 1)},
            "roofline_prefill_down": {"bound": "mfma", "kernel": "pf_down_kernel",
                                      "achieved": round(dn_flops / (dn_ms / 1000.0) / 1e12, 2),
                                      "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                      "frac": round(dn_flops / (dn_ms / 1000.0) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                                      "avg_launch_us": round(dn_ms * 1000.0, 1)},
            "roofline_prefill_one_launch": {"bound": "mfma",
                                            "kernel": "pf_sched_kernel (includes the gather launch)",
                                            "achieved": round((gu_flops + dn_flops) / (one_ms / 1000.0) / 1e12, 2),
                                            "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                            "frac": round((gu_flops + dn_flops) / (one_ms / 1000.0) / 1e12 /
                                                          MFMA_FP16_PEAK_TFLOPS, 4),
                                            "avg_launch_us": round(one_ms * 1000.0, 1)},
            "prefill_combine": {"kernel": "pf_combine_kernel", "avg_launch_us": round(cb_ms * 1000.0, 1),
                                "gbs": round(cb_bytes / (cb_ms / 1000.0) / 1e9, 1),
                                "bytes": cb_bytes},
            **pe,
            "prefill_config": f"T={T}, {E} experts, top-{TOPK}, uniform-random router logits, EXL3 4-bit synthetic "
                              f"experts sharing one w13 suh as the real checkpoints' layers do (one gathered row "
                              f"per token), {n_layers} layers alternated, {steps} timed steps"}


def run_prefill_per_expert_suh(args, torch, dev, x, logits, steps):
    """The T=8192 prefill call on layers whose experts each draw their own w13 input signs (suh): every pair gets its
    own rotated gate/up input row (T x top-8 rows instead of T)."""
    from mi355moe import _lib, ops, synthetic
    n_layers = len(logits)
    layers = [synthetic.exl3_layer(E, K, N, seed=600 + l, device=dev, uniform_suh=False) for l in range(n_layers)]
    outs = [torch.empty(x.shape[0], K, dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]
    info = [ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE) for l in range(n_layers)]

    def step(l):
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        ops.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l])

    ms = _time_calls(torch, step, n_layers, 2, steps)
    gu = []
    for k in range(steps):
        l = k % n_layers
        ids, wts = info[l]
        call = lambda st: ops.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], stages=st)
        call(_lib.STAGE_ROUTE)
        gu.append(_bracket(torch, lambda: call(_lib.STAGE_GATEUP)))
        call(_lib.STAGE_DOWN | _lib.STAGE_COMBINE)
    torch.cuda.synchronize()
    gu_ms = sum(a.elapsed_time(b) for a, b in gu) / len(gu)
    del layers
    torch.cuda.empty_cache()
    return {"prefill_per_expert_suh_ms_per_layer": round(ms, 4),
            "prefill_per_expert_suh_tokens_per_s": round(x.shape[0] / (ms / 1000.0), 1),
            "prefill_per_expert_suh_gateup_ms": round(gu_ms, 4),
            "prefill_per_expert_suh_config": "the same call on layers whose 288 experts each have their own w13 suh "
                                             "(one rotated gate/up input row per pair; gather and gate/up bracketed "
                                             "together)"}


def run_prefill_zipf(args, torch, dev, caps=(0, 16, 32, 64, 128)):
    """Prefill chunk T=8192 with Zipf(1.2)-skewed routing (top-8 of 288 drawn with probability ~ 1 / (rank + 1)^1.2
    over a random ranking): the thin/fat split at several caps (0 = every expert on the grouped kernels; cap c: experts
    with at most c rows on the decode kernels). Reports ms per layer call for each cap."""
    from mi355moe import ops, synthetic
    T = args.prefill_tokens
    layer = synthetic.exl3_layer(E, K, N, seed=450, device=dev, uniform_suh=True)
    x = synthetic.activations(T, K, seed=451, device=dev)
    ids = synthetic.zipf_ids(T, E, TOPK, seed=452, device=dev)
    wts = synthetic.softmax_weights(T, TOPK, seed=453, device=dev)
    out = torch.empty(T, K, dtype=torch.bfloat16, device=dev)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
    settle(torch, lambda: ops.moe_forward_ids_split(layer, x, ids, wts, caps[0], limit=LIMIT, out=out))
    res = {}
    for cap in caps:
        for _ in range(2):
            ops.moe_forward_ids_split(layer, x, ids, wts, cap, limit=LIMIT, out=out)
        torch.cuda.synchronize()
        steps = max(4, args.steps // 4)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            ops.moe_forward_ids_split(layer, x, ids, wts, cap, limit=LIMIT, out=out)
        e1.record()
        torch.cuda.synchronize()
        res[str(cap)] = round(e0.elapsed_time(e1) / steps, 4)
    best = min(res, key=lambda c: res[c])
    return {"prefill_zipf_ms_by_cap": res, "prefill_zipf_best_cap": int(best),
            "prefill_zipf_tokens_per_s": round(T / (res[best] / 1000.0), 1),
            "prefill_zipf_config": f"T={T}, {E} experts, Zipf(1.2) top-{TOPK} (rows per expert "
                                   f"{int(counts.min())}..{int(counts.max())}, {int((counts <= 64).sum())} experts "
                                   "with <= 64 rows), EXL3 4-bit synthetic experts; ms per layer call by thin cap"}


def run_prefill_chunks(args, torch, dev, sizes=(2048, 4096)):
    """Smaller prefill chunks (uniform-random router logits, the T=8192 workload's layer shapes): ms per layer call
    of the grouped path at each chunk size. At ~57 and ~114 rows per expert these run the mid-tile GEMMs (128-row
    halves of the segments, two workgroups per CU)."""
    from mi355moe import _lib, ops, synthetic
    layer = synthetic.exl3_layer(E, K, N, seed=470, device=dev, uniform_suh=True)
    res = {}
    for T in sizes:
        x = synthetic.activations(T, K, seed=471, device=dev)
        g = torch.Generator(device=dev)
        g.manual_seed(472)
        ids, wts = ops.router_topk(torch.rand(T, E, generator=g, device=dev) * 4 - 2, TOPK, None, routed_scale=SCALE)
        out = torch.empty(T, K, dtype=torch.bfloat16, device=dev)
        call = lambda: ops.moe_forward_ids(layer, x, ids, wts, limit=LIMIT, out=out, path=_lib.PATH_PREFILL)
        settle(torch, call, 20.0)
        steps = max(4, args.steps // 2)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        res[str(T)] = round(e0.elapsed_time(e1) / steps, 4)
    return {"prefill_chunk_ms_by_tokens": res,
            "prefill_chunk_config": f"{E} experts, top-{TOPK}, uniform-random router logits, EXL3 4-bit synthetic "
                                    "experts sharing one w13 suh; grouped path, ms per layer call by chunk tokens"}


def run_fp8(args, torch, dev):
    """e4m3 expert variant, T=2048 (hidden 4096, 288 experts, top-8, intermediate 1024): block-scaled e4m3 experts
    (N(0, 0.02) weights, fp32 scale per 128x128 block), bf16 activations quantised per token, sigmoid top-8 x2.5 of
    uniform-random router logits (the top-k runs inside the step; the router GEMM is not part of this workload).
    HBM-bound: bytes = distinct experts x 3 x K x N + scales."""
    from mi355moe import _lib, fp8, ops, synthetic
    T = args.fp8_tokens
    n_layers = 2
    layers = [synthetic.fp8_layer(E, K, N, seed=600 + l, device=dev) for l in range(n_layers)]
    x = synthetic.activations(T, K, seed=620, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(621)
    logits = [torch.rand(T, E, generator=g, device=dev) * 4 - 2 for _ in range(n_layers)]
    outs = [torch.empty(T, K, dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]

    def step(l):
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        fp8.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l])
        return ids, wts

    info = [step(l) for l in range(n_layers)]
    torch.cuda.synchronize()
    distinct = [int(torch.unique(i).numel()) for i, _ in info]
    settle(torch, lambda: step(0))
    for w in range(max(2, args.warmup // 4)):
        step(w % n_layers)
    torch.cuda.synchronize()
    steps = max(4, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for k in range(steps):
        step(k % n_layers)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gu = []
    for k in range(steps):
        l = k % n_layers
        ids, wts = info[l]
        fp8.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], stages=_lib.STAGE_ROUTE)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(HOLD_CYCLES)     # the stream is busy while the host enqueues the bracketed launch
        a.record()
        fp8.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], stages=_lib.STAGE_GATEUP)
        b.record()
        fp8.moe_forward_ids(layers[l], x, ids, wts, limit=LIMIT, out=outs[l],
                            stages=_lib.STAGE_DOWN | _lib.STAGE_COMBINE)
        gu.append((a, b))
    torch.cuda.synchronize()
    gu_ms = sum(a.elapsed_time(b) for a, b in gu) / len(gu)
    D = sum(distinct) / len(distinct)
    scales = 4 * 3 * (K // 128) * (N // 128)
    layer_bytes = D * (3 * K * N + scales) + T * K * 2 * 2
    gu_bytes = D * (2 * K * N + 4 * 2 * (K // 128) * (N // 128))
    P = T * TOPK
    extra = {}
    if not args.no_cpu_baseline:
        extra["cpu_baseline_fp8"] = cpu_baseline_fp8(torch, layers[0], x, info[0][0], info[0][1],
                                                     cpu_threads())
    return {**extra, "fp8_tokens_per_s": round(T / (ms / 1000.0), 1), "fp8_ms_per_layer": round(ms, 4),
            "fp8_gbs": round(layer_bytes / (ms / 1000.0) / 1e9, 1),
            "fp8_tflops": round(2.0 * P * 3 * K * N / (ms / 1000.0) / 1e12, 2),
            "fp8_distinct_experts": D,
            "roofline_fp8": {"bound": "hbm", "kernel": "fp8_gateup_kernel",
                             "achieved": round(gu_bytes / (gu_ms / 1000.0) / 1e9, 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(gu_bytes / (gu_ms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
                             "avg_launch_us": round(gu_ms * 1000.0, 1)},
            "fp8_config": f"T={T}, {E} experts, sigmoid top-{TOPK} x{SCALE} of uniform-random logits, block-scaled e4m3 experts "
                          f"(128x128 fp32 scales), per-token e4m3 activations, {n_layers} layers alternated, "
                          f"{steps} timed steps"}


def run_e4m3_trellis(args, torch, dev):
    """Trellis-sourced e4m3 variant, T=2048 (hidden 4096, 288 EXL3 4-bit experts, top-8, intermediate 1024):
    activations quantised per row to e4m3 after the input rotation, weights rounded to e4m3, the down input
    requantised per row; sigmoid top-8 x2.5 of uniform-random router logits inside the step."""
    from mi355moe import ops, synthetic
    T = args.fp8_tokens
    n_layers = 2
    layers = [synthetic.exl3_layer(E, K, N, seed=640 + l, device=dev, uniform_suh=True) for l in range(n_layers)]
    x = synthetic.activations(T, K, seed=660, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(661)
    logits = [torch.rand(T, E, generator=g, device=dev) * 4 - 2 for _ in range(n_layers)]
    outs = [torch.empty(T, K, dtype=torch.bfloat16, device=dev) for _ in range(n_layers)]

    def step(l):
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        ops.moe_forward_ids_e4m3(layers[l], x, ids, wts, limit=LIMIT, out=outs[l])

    settle(torch, lambda: step(0))
    for w in range(max(2, args.warmup // 4)):
        step(w % n_layers)
    torch.cuda.synchronize()
    steps = max(4, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for k in range(steps):
        step(k % n_layers)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps

    def step_fold(l):
        ids, wts = ops.router_topk(logits[l], TOPK, None, routed_scale=SCALE)
        ops.moe_forward_ids_e4m3(layers[l], x, ids, wts, limit=LIMIT, out=outs[l], accumulate=True,
                                 bf16_contrib=True)

    ms_fold = _time_calls(torch, step_fold, n_layers, 2, steps)
    P = T * TOPK
    return {"e4m3t_tokens_per_s": round(T / (ms / 1000.0), 1), "e4m3t_ms_per_layer": round(ms, 4),
            "e4m3t_bf16acc_fold_ms_per_layer": round(ms_fold, 4),
            "e4m3t_tflops": round(2.0 * P * 3 * K * N / (ms / 1000.0) / 1e12, 2),
            "e4m3t_config": f"T={T}, {E} EXL3 4-bit experts, trellis-sourced e4m3 numerics (per-row e4m3 activations, "
                            f"weights rounded to e4m3, fp32 sums), sigmoid top-{TOPK} x{SCALE} of uniform-random "
                            f"logits, {n_layers} layers alternated, {steps} timed steps"}


def run_stack(args, torch, dev):
    """42-layer stacked decode, T=8, captured as one HIP graph and replayed: each layer has its own 288 EXL3 experts
    (42 x 1.82 GB = 76.4 GB, far beyond every cache) and its own router; the layer's output is added to the residual
    stream that feeds the next layer's router. Expert popularity is Zipf(1.2)-skewed in the router logits: one
    hidden channel is held at a constant c and the router column that reads it is -1.2 ln(rank + 1) / c over a
    per-layer random ranking of the experts, so logit_e = x.W_e - 1.2 ln(rank_e + 1). Bytes per replay = sum over
    layers of D_l x (6,291,456 + 30,720) + router weight and bias + activations, D_l counted per layer."""
    from mi355moe import ops, synthetic
    T, nl, c0 = args.tokens, args.stack_layers, 8.0
    log(f"[bench] building {nl} layers x {E} experts ({nl * E * (EXPERT_TRELLIS + EXPERT_SCALES) / 1e9:.1f} GB) ...")
    layers, routers = [], []
    for l in range(nl):
        layers.append(synthetic.exl3_layer(E, K, N, seed=700 + l, device=dev))
        routers.append(synthetic.zipf_router(E, K, seed=800 + l, rank_seed=900 + l, device=dev, c0=c0))
    xs = [synthetic.zipf_activations(T, K, seed=950, device=dev, c0=c0)] + [
        torch.empty(T, K, dtype=torch.bfloat16, device=dev) for _ in range(nl)]
    outs = [torch.empty(T, K, dtype=torch.bfloat16, device=dev) for _ in range(nl)]
    ids = [torch.empty(T, TOPK, dtype=torch.int32, device=dev) for _ in range(nl)]
    wts = [torch.empty(T, TOPK, dtype=torch.float32, device=dev) for _ in range(nl)]

    def forward():
        for l in range(nl):
            w, b = routers[l]
            ops.moe_layer(layers[l], xs[l], router_w=w, topk=TOPK, bias=b, routed_scale=SCALE, limit=LIMIT,
                          out=outs[l], picks_out=(ids[l], wts[l]))
            torch.add(xs[l], outs[l], out=xs[l + 1])

    forward()                                                 # eager: sizes the workspace, fixes the routing
    torch.cuda.synchronize()
    ref = xs[nl].clone()
    distinct = [int(torch.unique(i).numel()) for i in ids]
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        forward()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward()
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(ref, xs[nl]):
        raise RuntimeError("stacked-layer graph replay differs from the eager pass")
    settle(torch, graph.replay)
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(4, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = sum(d * (EXPERT_TRELLIS + EXPERT_SCALES) for d in distinct) + nl * (E * K * 2 + E * 4 + 3 * T * K * 2)
    gbs = nbytes / (ms / 1000.0) / 1e9
    # the dominant kernel (the grouped gate/up GEMV) alone, every layer once with its own routing: route staged
    # untimed, the gate/up launch bracketed by HIP events on its stream
    from mi355moe import _lib
    gu, gu_bytes = [], 0
    for l in range(nl):
        ops.moe_forward_ids(layers[l], xs[l], ids[l], wts[l], limit=LIMIT, out=outs[l], stages=_lib.STAGE_ROUTE)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(HOLD_CYCLES)
        a.record()
        ops.moe_forward_ids(layers[l], xs[l], ids[l], wts[l], limit=LIMIT, out=outs[l], stages=_lib.STAGE_GATEUP)
        b.record()
        gu.append((a, b))
        gu_bytes += distinct[l] * (2 * K * N // 2 + 2 * (2 * K + 3 * N)) + T * K * 2
    torch.cuda.synchronize()
    gu_us = sum(a.elapsed_time(b) for a, b in gu) * 1000.0 / nl
    gu_gbs = gu_bytes / nl / (gu_us * 1e-6) / 1e9
    return {"roofline_stack": {"bound": "hbm", "kernel": "dec_gateup_kernel", "achieved": round(gu_gbs, 1),
                               "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                               "avg_launch_us": round(gu_us, 2)},
            "stack_us_per_layer": round(ms * 1000.0 / nl, 2), "stack_ms_per_replay": round(ms, 4),
            "stack_gbs": round(gbs, 1), "stack_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "stack_distinct_mean": round(sum(distinct) / nl, 2),
            "stack_config": f"{nl}-layer stacked decode, T={T}, {E} EXL3 experts per layer "
                            f"({nl * E * (EXPERT_TRELLIS + EXPERT_SCALES) / 1e9:.1f} GB), Zipf(1.2) expert popularity "
                            f"in the router logits, residual stream between layers, one HIP graph, {reps} replays"}


def cpu_block_a(torch, threads: int):
    """Configuration A, the CPU-runnable case: a dense MoE block (T=64, hidden 1024, 32 experts, softmax top-4
    renormalised, intermediate 512, SwiGLU, bf16 weights ~N(0, 0.02), activations ~N(0, 1)) in torch on the host,
    fp32 accumulation on the bf16 weights; seeded draws in the order router, w13, w2, x. A reported baseline only
    (median of 9 calls after 3 warm-ups)."""
    import statistics
    T_, d, n, k, inter = 64, 1024, 32, 4, 512
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(20261201)
    wr = (torch.randn(n, d, generator=g) * 0.02).to(torch.bfloat16)
    w13 = (torch.randn(n, 2 * inter, d, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(n, d, inter, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(T_, d, generator=g).to(torch.bfloat16)

    def block():
        p = torch.softmax(x.float() @ wr.float().t(), dim=-1)
        w, ids = torch.topk(p, k, dim=-1)
        w = w / w.sum(-1, keepdim=True)
        out = torch.zeros(T_, d)
        for e in ids.unique().tolist():
            rows, slot = (ids == e).nonzero(as_tuple=True)
            h = x[rows].float() @ w13[e].float().t()
            a = torch.nn.functional.silu(h[:, :inter]) * h[:, inter:]
            out.index_add_(0, rows, (a @ w2[e].float().t()) * w[rows, slot, None])
        return out.to(torch.bfloat16)

    for _ in range(3):
        block()
    ts = []
    for _ in range(9):
        t0 = time.perf_counter()
        block()
        ts.append(time.perf_counter() - t0)
    ms = statistics.median(ts) * 1000.0
    flop = 2.0 * T_ * k * 3 * d * inter
    return {"value": round(ms, 3), "unit": "ms per block call", "cores": threads, "kind": "torch",
            "gflops": round(flop / (ms / 1000.0) / 1e9, 2),
            "sample": f"T={T_}, hidden {d}, {n} experts, softmax top-{k}, intermediate {inter}, bf16 weights, "
                      "fp32 accumulation, median of 9 calls"}


def _traffic(distinct: float):
    """HBM bytes per gate/up launch from the committed PMC measurement (profiles/decode_gateup_traffic.json: FETCH_SIZE
    and WRITE_SIZE per launch, each scaled by what the counter reads for a device copy of known size), rescaled to
    this run's mean number of distinct experts (the kernel's traffic is proportional to it); None without the file."""
    path = os.path.join(ROOT, "profiles", "decode_gateup_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return round(t["hbm_bytes_per_launch"] * distinct / t["distinct_experts_per_launch"])


def copy_probe(torch, dev, mib: int):
    """Three device-to-device copies of `mib` MiB: a plain copy of known size, the reference that PMC byte counters
    (FETCH_SIZE / WRITE_SIZE) are scaled by."""
    a = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="all",
                    choices=["all", "decode", "prefill", "prefill-uniform", "zipf", "fp8", "e4m3t", "stack"])
    ap.add_argument("--stack-layers", type=int, default=42)
    ap.add_argument("--prefill-tokens", type=int, default=8192)
    ap.add_argument("--fp8-tokens", type=int, default=2048)
    ap.add_argument("--tokens", type=int, default=8)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--window-only", action="store_true",
                    help="run only the named workload, without the decode lead-in (a profiling window: the JSON line "
                         "then carries that workload's fields only)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the workload, copy a tensor of this many MiB three times (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this benchmark runs on one MI355X; --gpus {args.gpus} is not supported "
              "(the layer's tensor- and expert-parallel sharding is designed, not run)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    import mi355moe
    mi355moe._lib.lib()
    dev = torch.device("cuda", 0)
    if args.window_only and args.workload not in ("all", "decode"):
        args.no_cpu_baseline = True
        res = {"metric": METRIC, "workload": args.workload, "window_only": True}
    elif args.workload in ("prefill", "prefill-uniform", "zipf", "fp8", "e4m3t", "stack"):
        args.no_cpu_baseline = True
        res = run_decode(argparse.Namespace(**{**vars(args), "steps": 8, "warmup": 2}), torch, mi355moe, dev)
    else:
        res = run_decode(args, torch, mi355moe, dev)
    if args.workload in ("all", "prefill", "prefill-uniform"):
        log("[bench] prefill ...")
        res.update(run_prefill(args, torch, dev))
    if args.workload in ("all", "prefill", "zipf"):
        log("[bench] prefill, Zipf routing, thin/fat split ...")
        res.update(run_prefill_zipf(args, torch, dev))
    if args.workload in ("all", "prefill"):
        log("[bench] prefill chunks T=2048, 4096 ...")
        res.update(run_prefill_chunks(args, torch, dev))
    if args.workload in ("all", "fp8"):
        log("[bench] fp8 ...")
        res.update(run_fp8(args, torch, dev))
    if args.workload in ("all", "e4m3t"):
        log("[bench] e4m3 trellis ...")
        res.update(run_e4m3_trellis(args, torch, dev))
    if args.workload in ("all", "stack"):
        log("[bench] stacked decode ...")
        res.update(run_stack(args, torch, dev))
    if args.copy_probe_mib > 0:
        copy_probe(torch, dev, args.copy_probe_mib)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
