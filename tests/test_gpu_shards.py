"""GPU parity at tensor-parallel shard shapes and other hidden sizes: the layer's intermediate size per rank at TP = 2,
4 and 8 (N = 512, 256, 128 of GLM-5.3-Flash's 1024-wide shard at TP = 1, as code/fork/docs/prod_exl3_reference.py:
644-676 slices it), a smaller hidden size, and a hidden size whose staged decode inputs exceed one workgroup's LDS
(K = 6144: the decode GEMV then splits K and adds the partial sums of the splits in split order).

Both paths against the oracle (oracle/moe.py): the decode kernels against the "decode_x" rounding points
(rel_l2 <= 5e-4) and float64 (rel_l2 <= 5e-3); the grouped prefill kernels against the "e3" rounding points
(rel_l2 <= 5e-4) and float64 with the limit before SiLU (rel_l2 <= 5e-3); the bf16 output elementwise within
rtol 2e-2 / atol 1e-3 of float64 on both.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe, routing

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 512), (4096, 256), (4096, 128), (2048, 1024), (6144, 512)]


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _np_layer(ex) -> dict:
    return {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                      "w2_svh")}


def _check(ex, x, ids, w, n, topk, limit, out32, out_bf, kmode, fmode):
    lay = _np_layer(ex)
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, w16 = moe.pairs_from_routing(local, w.float().cpu().numpy(), n, topk)
    x16 = x.to(torch.float16).cpu().numpy()
    ref_k = moe.forward(lay, x16, tok, exx, w16, limit, kmode)
    ref64 = moe.forward(lay, x16, tok, exx, w16, limit, fmode)
    got = out32.cpu().numpy()
    assert np.isfinite(got).all()
    rk, r64 = _rel(got, ref_k), _rel(got, ref64)
    _say(f"  rel_l2 vs {kmode} {rk:.2e}, vs {fmode} {r64:.2e}")
    assert rk <= 5e-4, rk
    assert r64 <= 5e-3, r64
    assert np.allclose(out_bf.float().cpu().numpy(), ref64, rtol=2e-2, atol=1e-3)


@pytest.mark.parametrize("K,N", SHAPES)
def test_decode_path_at_shard_shapes(cuda, K, N):
    from mi355moe import _lib, ops, synthetic
    n, T, topk, limit = 16, 8, 8, 10.0
    _say(f"decode path K={K} N={N} n={n} T={T}")
    ex = synthetic.calibrated_layer(n, K, N, seed=K + N, device=cuda)
    x = synthetic.activations(T, K, seed=K + 1, device=cuda)
    ids = synthetic.random_ids(T, n, topk, seed=N + 2, device=cuda)
    w = synthetic.softmax_weights(T, topk, seed=N + 3, device=cuda)
    out32 = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.float32, path=_lib.PATH_DECODE)
    out_bf = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.bfloat16, path=_lib.PATH_DECODE)
    torch.cuda.synchronize()
    _check(ex, x, ids, w, n, topk, limit, out32, out_bf, "decode_x", "f64")


@pytest.mark.parametrize("K,N", SHAPES)
def test_prefill_path_at_shard_shapes(cuda, K, N):
    from mi355moe import _lib, ops, synthetic
    n, T, topk, limit = 4, 96, 4, 10.0
    _say(f"prefill path K={K} N={N} n={n} T={T}")
    ex = synthetic.calibrated_layer(n, K, N, seed=2 * K + N, device=cuda)
    assert ex.shared_suh
    x = synthetic.activations(T, K, seed=K + 5, device=cuda)
    ids = synthetic.random_ids(T, n, topk, seed=N + 6, device=cuda)
    w = synthetic.softmax_weights(T, topk, seed=N + 7, device=cuda)
    out32 = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    out_bf = ops.moe_forward_ids(ex, x, ids, w, limit=limit, out_dtype=torch.bfloat16, path=_lib.PATH_PREFILL)
    torch.cuda.synchronize()
    _check(ex, x, ids, w, n, topk, limit, out32, out_bf, "e3", "f64_pre")
