"""GPU parity of the trellis-sourced e4m3 variant (mi355moe_e4m3_moe_forward_ids): activations quantised per row to
e4m3 after the input rotation, EXL3 weights rounded to e4m3, fp32 sums, the down input requantised per row.

Reference: oracle/e4m3_trellis.forward (float64 sums of the same e4m3 operands; its quantisers follow the reference's
fp32 rotation, so the GPU's e4m3 codes match the oracle's except where an fp32 summation-order difference moves a
value across a rounding midpoint). Bound: rel_l2 <= 1e-3, five times below the reference's own e4m3 tolerance
(code/fork/overlay/glm53_moe_e4m3.py:110); measured values are far below it and printed.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import e4m3_trellis, exl3, moe, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _np_layer(ex) -> dict:
    return {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                      "w2_svh")}


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("n,K,N,T,topk,limit,xdt,calib", [(8, 1024, 512, 300, 8, 10.0, torch.bfloat16, False),
                                                          (16, 512, 256, 33, 4, 0.0, torch.float16, False),
                                                          (4, 4096, 1024, 40, 4, 10.0, torch.bfloat16, False),
                                                          (8, 1024, 512, 300, 8, 10.0, torch.bfloat16, True),
                                                          (4, 4096, 1024, 64, 4, 10.0, torch.bfloat16, True)])
def test_e4m3_trellis_vs_oracle(cuda, n, K, N, T, topk, limit, xdt, calib):
    """calib: scales calibrated as the reference's harness (std of the gate/up pre-activations 5), so the SwiGLU
    limit clamps a few per cent of the gate values and more of the up values (the rates are asserted)."""
    from mi355moe import ops, synthetic
    _say(f"e4m3 trellis n={n} K={K} N={N} T={T} topk={topk} L={limit} x={xdt} calibrated={calib}")
    if calib:
        ex = synthetic.calibrated_layer(n, K, N, seed=n * 5 + T, device=cuda)
    else:
        ex = synthetic.exl3_layer(n, K, N, seed=n * 5 + T, device=cuda, svh_scale=0.05)
    x = synthetic.activations(T, K, seed=T + 11, device=cuda).to(xdt)
    ids = synthetic.random_ids(T, n, topk, seed=T + 12, device=cuda)
    ids[1, 0] = -1
    w = synthetic.softmax_weights(T, topk, seed=T + 13, device=cuda)
    got = ops.moe_forward_ids_e4m3(ex, x, ids, w, limit=limit, out_dtype=torch.float32)
    again = ops.moe_forward_ids_e4m3(ex, x, ids, w, limit=limit, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, again)                                    # deterministic (no atomics in the sums)
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, _ = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    lay = _np_layer(ex)
    x16 = x.to(torch.float16).cpu().numpy()
    if calib:
        over_g = over_u = total = 0
        for e in np.unique(exx[exx >= 0]):
            rows = x16[tok[exx == e]].astype(np.float64)
            gv = exl3.linear_f64(rows, lay["w13_trellis"][e, 0], lay["w13_suh"][e, 0], lay["w13_svh"][e, 0])
            uv = exl3.linear_f64(rows, lay["w13_trellis"][e, 1], lay["w13_suh"][e, 1], lay["w13_svh"][e, 1])
            over_g += int((gv > limit).sum())
            over_u += int((np.abs(uv) > limit).sum())
            total += gv.size
        _say(f"  clamped: gate {over_g / total:.3%}, up {over_u / total:.3%}")
        assert 0.01 <= over_g / total <= 0.05 and 0.025 <= over_u / total <= 0.08
    ref = e4m3_trellis.forward(lay, x16, tok, exx, w.cpu().numpy().reshape(-1), limit)
    g = got.cpu().numpy()
    assert np.isfinite(g).all()
    r = _rel(g, ref)
    _say(f"  rel_l2 vs oracle {r:.3e}")
    assert r <= 1e-3, r                                              # measured 2e-5 .. 2e-4
    # an invalid slot contributes nothing: token 1's output is its other slots' sum only (checked by the oracle)
    assert np.abs(g[1]).max() > 0


def test_e4m3_trellis_full_size_token_sample(cuda):
    """The trellis-sourced e4m3 configuration at its bench size (T=2048, 288 experts sharing one w13 suh, hidden
    4096, intermediate 1024, top-8 x2.5 of uniform-random logits): the whole-call entry against the stage path (same
    kernels), and four sampled tokens against the oracle: the output from the kernel's own e4m3 down inputs (the
    reference's A4 bar, rel_l2 <= 1e-5, and elementwise rtol 2e-2 / atol 1e-3), end to end rel_l2 <= 1e-3 (the
    elementwise share is printed: the oracle requantises its own float64-summed SwiGLU output)."""
    from mi355moe import e4m3_ext, ops, synthetic
    from oracle import e4m3
    n, K, N, T, topk = 288, 4096, 1024, 2048, 8
    _say(f"e4m3 trellis full size T={T} n={n}: sampled tokens vs the oracle")
    ex = synthetic.exl3_layer(n, K, N, seed=41, device=cuda, uniform_suh=True)
    x = synthetic.activations(T, K, seed=42, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(43)
    logits = torch.rand(T, n, generator=g, device=cuda) * 4 - 2
    ids, w = ops.router_topk(logits, topk, None, routed_scale=2.5)
    whole = ops.moe_forward_ids_e4m3(ex, x, ids, w, limit=10.0, out_dtype=torch.float32)
    keep: dict = {}
    staged = e4m3_ext.run(x, ids, w, ex, 10.0, keep=keep)
    torch.cuda.synchronize()
    assert torch.isfinite(whole).all()
    assert _rel(staged.cpu().numpy(), whole.cpu().numpy()) <= 1e-5
    sample = np.array([0, 777, 1500, 2047])
    ids_np, w_np = ids.cpu().numpy(), w.cpu().numpy()
    used = np.unique(ids_np[sample])
    remap = {int(e): i for i, e in enumerate(used)}
    sel = torch.as_tensor(used, dtype=torch.long, device=cuda)
    lay = {k: getattr(ex, k).index_select(0, sel).cpu().numpy() for k in
           ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
    local = np.vectorize(remap.get)(ids_np[sample])
    tok, exx, _ = moe.pairs_from_routing(local, w_np[sample], len(used), topk)
    x16 = x.to(torch.float16).cpu().numpy()[sample]
    ref = e4m3_trellis.forward(lay, x16, tok, exx, w_np[sample].reshape(-1), 10.0)
    got = whole.cpu().numpy()[sample].astype(np.float64)
    r = _rel(got, ref)
    # A4 for the sampled tokens: their rows' e4m3 down inputs as the kernels wrote them
    nr = int(keep["num_rows"].item())
    rt = keep["row_token"][:nr].cpu().numpy()
    rows = np.nonzero(np.isin(rt, sample))[0]
    re_ = keep["row_expert"][:nr].cpu().numpy()[rows]
    qd = e4m3.decode(e4m3_trellis.from_storage(keep["a8d"][torch.from_numpy(rows).to(cuda)].cpu().numpy()))
    dsc = keep["dsc"][:nr].cpu().numpy()[rows]
    rw = keep["row_weight"][:nr].cpu().numpy()[rows].astype(np.float64)
    y4 = np.zeros((sample.size, K))
    pos = {int(t): i for i, t in enumerate(sample)}
    for i, r_ in enumerate(rows):
        e = remap[int(re_[i])]
        yd = e4m3_trellis.down_rows(qd[i:i + 1].astype(np.float32), dsc[i:i + 1], lay["w2_trellis"][e],
                                    lay["w2_svh"][e])
        y4[pos[int(rt[r_])]] += rw[i] * yd[0]
    r4 = _rel(got, y4)
    bad = ~np.isclose(got, ref, rtol=2e-2, atol=1e-3)
    _say(f"  rel_l2 vs oracle {r:.3e}; from the kernel's down inputs {r4:.2e}; end to end {bad.mean():.4%} of "
         f"elements outside rtol 2e-2 / atol 1e-3")
    assert r <= 1e-3, r
    assert r4 <= 1e-5 and np.allclose(got, y4, rtol=2e-2, atol=1e-3), r4
