"""GPU parity of the grouped prefill path (gather, fp16 MFMA gate/up and down GEMMs over 256-row expert tiles).

References (oracle/moe.py): "e3" mode (the kernels' rounding points; only fp32 summation orders differ, so the fp32
outputs agree to rel_l2 <= 5e-4) and float64 with the limit before SiLU (rel_l2 <= 5e-3, elementwise rtol 2e-2 /
atol 1e-3 of the bf16 output). At the full prefill size the path is checked against the decode path on the same
inputs (both are within the float64 bound, so they agree to rel_l2 <= 5e-3).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _np_layer(ex) -> dict:
    return {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                      "w2_svh")}


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("n,K,N,T,topk,limit", [(8, 1024, 512, 300, 8, 10.0),     # ~300 rows/expert: 2 tiles
                                                (16, 1024, 256, 129, 4, 0.0),
                                                (4, 4096, 1024, 160, 4, 10.0)])
def test_prefill_vs_oracle(cuda, n, K, N, T, topk, limit):
    from mi355moe import _lib, ops, synthetic
    _say(f"prefill n={n} K={K} N={N} T={T} topk={topk} L={limit}")
    ex = synthetic.exl3_layer(n, K, N, seed=n * 7 + T, device=cuda, svh_scale=0.05 if K < 4096 else 0.01)
    assert ex.shared_suh
    x = synthetic.activations(T, K, seed=T + 1, device=cuda)
    ids = synthetic.random_ids(T, n, topk, seed=T + 2, device=cuda)
    ids[3, 0] = -1
    w = synthetic.softmax_weights(T, topk, seed=T + 3, device=cuda)
    out32 = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    out_bf = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.bfloat16, path=_lib.PATH_PREFILL)
    torch.cuda.synchronize()
    lay = _np_layer(ex)
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, w16 = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    x16 = x.to(torch.float16).cpu().numpy()
    ref_k = moe.forward(lay, x16, tok, exx, w16, limit, "e3")
    ref64 = moe.forward(lay, x16, tok, exx, w16, limit, "f64_pre")
    got = out32.cpu().numpy()
    assert np.isfinite(got).all()
    assert _rel(got, ref_k) <= 5e-4, _rel(got, ref_k)
    assert _rel(got, ref64) <= 5e-3, _rel(got, ref64)
    gb = out_bf.float().cpu().numpy()
    scale = np.abs(ref64).max()
    assert np.allclose(gb, ref64, rtol=2e-2, atol=1e-3 * max(1.0, scale / 1.0))


def test_prefill_full_size_vs_decode_path(cuda):
    """T=8192, 288 experts, K=4096, N=1024: the prefill path (auto-selected) against the decode path."""
    from mi355moe import _lib, ops, synthetic
    _say("prefill full size T=8192 vs decode path")
    ex = synthetic.exl3_layer(288, 4096, 1024, seed=99, device=cuda)
    T = 8192
    x = synthetic.activations(T, 4096, seed=100, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(101)
    logits = torch.rand(T, 288, generator=g, device=cuda) * 4 - 2
    ids, w = ops.router_topk(logits, 8, None, routed_scale=2.5)
    a = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32)                        # auto: prefill
    b = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_DECODE)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    r = (torch.linalg.norm((a - b).double()) / torch.linalg.norm(b.double())).item()
    _say(f"prefill vs decode rel_l2 {r:.3e}")
    assert r <= 5e-3
