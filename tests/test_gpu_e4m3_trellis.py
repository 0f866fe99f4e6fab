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
