"""GPU parity of the thin/fat split (mi355moe_moe_forward_ids_split): experts routed at most `cap` rows on the decode
kernels (limit after SiLU), the others on the grouped kernels (limit before SiLU), one slot-order combine. Checked
on Zipf(1.2)-skewed routing against the oracle (each pair in its kernel's rounding points, rel_l2 <= 5e-4; float64
with each pair's limit order, rel_l2 <= 5e-3 and bf16 elementwise rtol 2e-2 / atol 1e-3), and at the extremes against
the single-path entries: cap 0 equals the grouped path bit for bit, a cap above every count the decode path."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe, routing

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def case(cuda):
    from mi355moe import synthetic
    n, K, N, T, topk = 64, 1024, 512, 600, 8
    ex = synthetic.calibrated_layer(n, K, N, seed=71, device=cuda)
    x = synthetic.activations(T, K, seed=72, device=cuda)
    ids = synthetic.zipf_ids(T, n, topk, 73, device="cpu")
    ids[5, 1] = -1
    w = synthetic.softmax_weights(T, topk, seed=74, device=cuda)
    return ex, x, ids.to(cuda), w, n, topk


@pytest.mark.parametrize("cap", [16, 48, 150])
def test_split_vs_oracle(cuda, case, cap):
    from mi355moe import ops
    ex, x, ids, w, n, topk = case
    counts = np.bincount(ids.cpu().numpy().reshape(-1)[ids.cpu().numpy().reshape(-1) >= 0], minlength=n)
    thin = (counts > 0) & (counts <= cap)
    print(f"split cap={cap}: {int(thin.sum())} thin experts, {int((counts > cap).sum())} fat (counts {counts.min()}.."
          f"{counts.max()})", flush=True)
    got = ops.moe_forward_ids_split(ex, x, ids, w, cap, out_dtype=torch.float32)
    got_bf = ops.moe_forward_ids_split(ex, x, ids, w, cap, out_dtype=torch.bfloat16)
    again = ops.moe_forward_ids_split(ex, x, ids, w, cap, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    lay = {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                     "w2_svh")}
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, w16 = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    is_thin = np.where(exx >= 0, thin[np.maximum(exx, 0)], False)
    e_thin = np.where(is_thin, exx, -1).astype(np.int32)
    e_fat = np.where(is_thin, -1, exx).astype(np.int32)
    x16 = x.to(torch.float16).cpu().numpy()
    ref_k = (moe.forward(lay, x16, tok, e_thin, w16, 10.0, "decode_x").astype(np.float64)
             + moe.forward(lay, x16, tok, e_fat, w16, 10.0, "e3"))
    ref64 = moe.forward(lay, x16, tok, e_thin, w16, 10.0, "f64") + moe.forward(lay, x16, tok, e_fat, w16, 10.0,
                                                                               "f64_pre")
    g = got.cpu().numpy()
    r_k, r64 = _rel(g, ref_k), _rel(g, ref64)
    print(f"  rel_l2 vs kernel rounding {r_k:.3e}, vs float64 {r64:.3e}", flush=True)
    assert r_k <= 5e-4 and r64 <= 5e-3
    assert np.allclose(got_bf.float().cpu().numpy(), ref64, rtol=2e-2, atol=1e-3)


def test_split_extremes_equal_single_paths(cuda, case):
    from mi355moe import _lib, ops
    ex, x, ids, w, n, topk = case
    grouped = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    decode = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_DECODE)
    s0 = ops.moe_forward_ids_split(ex, x, ids, w, 0, out_dtype=torch.float32)
    sall = ops.moe_forward_ids_split(ex, x, ids, w, ids.numel(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(s0, grouped)
    assert _rel(sall.cpu().numpy(), decode.cpu().numpy()) <= 1e-6
