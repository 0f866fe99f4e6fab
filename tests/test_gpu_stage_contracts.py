"""GPU parity of the stage entry points over caller-built row tables: the grouped (E3) trio with production's
table builder and apply (code/fork/docs/prod_exl3_reference.py:1316-1435), and the e4m3 extension's seg_tables /
gather2 / fused as the overlay's run() chains them (code/fork/overlay/glm53_moe_e4m3.py:450-592), each against the
oracle, the segment tables bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import e4m3_trellis, moe, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _np_layer(ex) -> dict:
    return {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                      "w2_svh")}


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("cap", [0, 140, 10 ** 6])
def test_e3_trio_apply(cuda, cap):
    """apply_exl3_grouped_fat over production's routing prelude: out (fp32, pre-filled) += the fat experts' (count >
    cap) routed output; cap 0 = every expert, 10**6 = none (out untouched)."""
    from mi355moe import e3, synthetic
    n, K, N, T, topk = 16, 1024, 512, 300, 8
    _say(f"E3 trio n={n} K={K} N={N} T={T} topk={topk} cap={cap}")
    ex = synthetic.calibrated_layer(n, K, N, seed=5, device=cuda)
    x16 = synthetic.activations(T, K, seed=6, device=cuda).to(torch.float16)
    ids = synthetic.random_ids(T, n, topk, seed=7, device=cuda)
    w = synthetic.softmax_weights(T, topk, seed=8, device=cuda)
    local = ids.reshape(-1).long()
    order = torch.argsort(local, stable=True)
    counts = torch.bincount(local, minlength=n + 1)[:n].contiguous()
    token_sorted = torch.div(order, topk, rounding_mode="floor")
    weight_sorted = w.reshape(-1)[order].to(torch.float16)
    base = torch.randn(T, K, device=cuda) * 0.1
    out = base.clone()
    e3.apply_exl3_grouped_fat(x16, out, counts, token_sorted, weight_sorted, ex, cap, 10.0)
    again = base.clone()
    e3.apply_exl3_grouped_fat(x16, again, counts, token_sorted, weight_sorted, ex, cap, 10.0)
    torch.cuda.synchronize()
    assert torch.equal(out, again)                                 # deterministic (row-order sums, no atomics)
    fat = (counts > cap).cpu().numpy()
    lid = local.cpu().numpy()
    exx = np.where(fat[lid], lid, -1).astype(np.int32)
    tok = (np.arange(T * topk) // topk).astype(np.int32)
    w16 = w.reshape(-1).cpu().numpy().astype(np.float16)
    got = (out - base).cpu().numpy()
    if not fat.any():
        assert not got.any()
        return
    lay = _np_layer(ex)
    xs = x16.cpu().numpy()
    ref_k = moe.forward(lay, xs, tok, exx, w16, 10.0, "e3")
    ref64 = moe.forward(lay, xs, tok, exx, w16, 10.0, "f64_pre")
    r_k, r64 = _rel(got, ref_k), _rel(got, ref64)
    _say(f"  fat experts {int(fat.sum())}/{n}: rel_l2 vs E3 rounding {r_k:.3e}, vs float64 {r64:.3e}")
    assert r_k <= 5e-4 and r64 <= 5e-3
    assert np.allclose(got, ref64, rtol=2e-2, atol=1e-3)


def test_e4m3_seg_tables_bit_exact(cuda):
    from mi355moe import e4m3_ext
    g = torch.Generator().manual_seed(3)
    counts = torch.randint(0, 400, (288,), generator=g)          # P ~ 49,000 <= 65,536 rows
    counts[::7] = 0
    P = int(counts.sum())
    se, sr0, sr, ns, nr = e4m3_ext.seg_tables(counts.to(cuda), e4m3_ext.tile_rows(), P)
    local = np.repeat(np.arange(288), counts.numpy())
    o = routing.permutation(local, 288, 1, 1 << 30, e4m3_ext.tile_rows())
    k = int(ns.item())
    assert k == len(o["seg_expert"]) and int(nr.item()) == P
    assert np.array_equal(se[:k].cpu().numpy(), o["seg_expert"])
    assert np.array_equal(sr0[:k].cpu().numpy(), o["seg_row0"])
    assert np.array_equal(sr[:k].cpu().numpy(), o["seg_rows"])


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_e4m3_ext_run(cuda, out_dtype):
    """plan + gather2 + fused (the overlay's run() in its fused schedule) against the oracle's e4m3 spec, and against
    the whole-call entry mi355moe_e4m3_moe_forward_ids (same kernels; the sums differ only in order)."""
    from mi355moe import e4m3_ext, ops, synthetic
    n, K, N, T, topk = 8, 1024, 512, 300, 8
    _say(f"e4m3 extension run n={n} K={K} N={N} T={T} out={out_dtype}")
    ex = synthetic.calibrated_layer(n, K, N, seed=15, device=cuda)
    x = synthetic.activations(T, K, seed=16, device=cuda)
    ids = synthetic.random_ids(T, n, topk, seed=17, device=cuda)
    ids[1, 0] = -1
    w = synthetic.softmax_weights(T, topk, seed=18, device=cuda)
    if out_dtype == torch.float32:
        got = e4m3_ext.run(x, ids, w, ex, 10.0)
    else:
        got = torch.full((T, K), 0.5, dtype=torch.bfloat16, device=cuda)     # accumulated into, not zeroed
        e4m3_ext.run(x, ids, w, ex, 10.0, out=got)
    whole = ops.moe_forward_ids_e4m3(ex, x, ids, w, limit=10.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    local = routing.map_topk_to_local(ids.cpu().numpy(), n)
    tok, exx, _ = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    ref = e4m3_trellis.forward(_np_layer(ex), x.to(torch.float16).cpu().numpy(), tok, exx,
                               w.cpu().numpy().reshape(-1), 10.0)
    g = got.float().cpu().numpy() - (0.5 if out_dtype == torch.bfloat16 else 0.0)
    r = _rel(g, ref)
    _say(f"  rel_l2 vs oracle {r:.3e}")
    if out_dtype == torch.float32:
        assert r <= 1e-3
        assert _rel(g, whole.cpu().numpy()) <= 1e-5
    else:
        assert r <= 2e-2                       # one bf16 rounding of (0.5 + contribution), steps of 2^-8 .. 2^-7
        assert np.allclose(got.float().cpu().numpy(), 0.5 + ref, rtol=2.0 ** -8, atol=2.0 ** -8)
