"""GPU parity of the grouped prefill path (gather, fp16 MFMA gate/up and down GEMMs over 256-row expert tiles).

References (oracle/moe.py): "e3" mode (the kernels' rounding points; only fp32 summation orders differ, so the fp32
outputs agree to rel_l2 <= 5e-4) and float64 with the limit before SiLU (rel_l2 <= 5e-3, elementwise rtol 2e-2 /
atol 1e-3 of the bf16 output). At the full prefill size sampled tokens are checked against both, and the whole
output against the decode path on the same inputs (both are within the float64 bound, so they agree to
rel_l2 <= 5e-3).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import exl3, moe, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _np_layer(ex) -> dict:
    return {k: getattr(ex, k).cpu().numpy() for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                      "w2_svh")}


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _clamp_rates(lay: dict, x16: np.ndarray, tok: np.ndarray, exx: np.ndarray, limit: float) -> tuple[float, float]:
    """Fractions of the routed pairs' gate values above the limit and up values outside [-limit, limit] (float64
    pre-activations of the oracle's dequantised matrices)."""
    over_g = over_u = total = 0
    for e in np.unique(exx[exx >= 0]):
        rows = x16[tok[exx == e]].astype(np.float64)
        g = exl3.linear_f64(rows, lay["w13_trellis"][e, 0], lay["w13_suh"][e, 0], lay["w13_svh"][e, 0])
        u = exl3.linear_f64(rows, lay["w13_trellis"][e, 1], lay["w13_suh"][e, 1], lay["w13_svh"][e, 1])
        over_g += int((g > limit).sum())
        over_u += int((np.abs(u) > limit).sum())
        total += g.size
    return over_g / total, over_u / total


@pytest.mark.parametrize("n,K,N,T,topk,limit", [(8, 1024, 512, 300, 8, 10.0),     # ~300 rows/expert: 2 tiles
                                                (16, 1024, 256, 129, 4, 0.0),
                                                (4, 4096, 1024, 160, 4, 10.0)])
def test_prefill_vs_oracle(cuda, n, K, N, T, topk, limit):
    """Layers calibrated as the reference's harness (std of the gate/up pre-activations 5, so the SwiGLU limit 10
    clamps a few per cent of the values; routed outputs of RMS ~0.2): fp32 output against the kernels' rounding
    points (rel_l2 <= 5e-4) and float64 (rel_l2 <= 5e-3); bf16 output elementwise within rtol 2e-2 / atol 1e-3 of
    float64."""
    from mi355moe import _lib, ops, synthetic
    _say(f"prefill n={n} K={K} N={N} T={T} topk={topk} L={limit}")
    ex = synthetic.calibrated_layer(n, K, N, seed=n * 7 + T, device=cuda)
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
    if limit:
        rg, ru = _clamp_rates(lay, x16, tok, exx, limit)
        _say(f"  clamped: gate {rg:.3%}, up {ru:.3%}")
        assert 0.01 <= rg <= 0.05 and 0.025 <= ru <= 0.08, (rg, ru)
    ref_k = moe.forward(lay, x16, tok, exx, w16, limit, "e3")
    ref64 = moe.forward(lay, x16, tok, exx, w16, limit, "f64_pre")
    got = out32.cpu().numpy()
    assert np.isfinite(got).all()
    assert _rel(got, ref_k) <= 5e-4, _rel(got, ref_k)
    assert _rel(got, ref64) <= 5e-3, _rel(got, ref64)
    gb = out_bf.float().cpu().numpy()
    assert np.allclose(gb, ref64, rtol=2e-2, atol=1e-3)


def test_prefill_full_size_token_sample(cuda):
    """The prefill configuration at full size (T=8192, 288 experts, K=4096, N=1024, uniform-random router logits,
    top-8 x2.5; the automatic path is the grouped tier): eight sampled tokens against the oracle's E3 rounding points
    (rel_l2 <= 5e-4) and float64 (rel_l2 <= 5e-3, bf16 elementwise rtol 2e-2 / atol 1e-3)."""
    from mi355moe import ops, synthetic
    _say("prefill full size T=8192: sampled tokens vs the oracle")
    n, T, topk = 288, 8192, 8
    ex = synthetic.exl3_layer(n, 4096, 1024, seed=99, device=cuda)
    x = synthetic.activations(T, 4096, seed=100, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(101)
    logits = torch.rand(T, n, generator=g, device=cuda) * 4 - 2
    ids, w = ops.router_topk(logits, topk, None, routed_scale=2.5)
    out32 = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32)
    out_bf = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(out32).all()
    sample = np.array([0, 1, 2047, 4096, 5000, 8000, 8190, 8191])
    sel_t = torch.from_numpy(sample).to(cuda)
    ids_s = ids[sel_t].cpu().numpy()
    w_s = w[sel_t].cpu().numpy()
    used = np.unique(ids_s)
    remap = {int(e): i for i, e in enumerate(used)}
    local = np.vectorize(remap.get)(ids_s)
    sel = torch.as_tensor(used, dtype=torch.long, device=cuda)
    lay = {k: getattr(ex, k).index_select(0, sel).cpu().numpy() for k in
           ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
    tok, exx, w16 = moe.pairs_from_routing(local, w_s, len(used), topk)
    x16 = x[sel_t].to(torch.float16).cpu().numpy()
    ref_k = moe.forward(lay, x16, tok, exx, w16, 10.0, "e3")
    ref64 = moe.forward(lay, x16, tok, exx, w16, 10.0, "f64_pre")
    got = out32[sel_t].cpu().numpy()
    r_k, r64 = _rel(got, ref_k), _rel(got, ref64)
    _say(f"  rel_l2 vs E3 rounding {r_k:.3e}, vs float64 {r64:.3e}")
    assert r_k <= 5e-4 and r64 <= 5e-3, (r_k, r64)
    assert np.allclose(out_bf[sel_t].float().cpu().numpy(), ref64, rtol=2e-2, atol=1e-3)


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


@pytest.mark.parametrize("numerics,T,n,K,N", [("e3", 700, 16, 1024, 512), ("e4m3", 700, 16, 1024, 512),
                                              ("e3", 8192, 288, 4096, 1024), ("split", 2000, 64, 1024, 512)])
def test_token_rows_gather_bit_exact(cuda, numerics, T, n, K, N):
    """Experts sharing one w13 suh (MI355MOE_LAYER_UNIFORM_W13_SUH): the grouped path gathers one row per token and
    the gate/up GEMM reads rows through their tokens. The output equals the per-pair gather's (the same layer with the
    flag cleared) bit for bit, for E3 and e4m3 numerics and the thin/fat split; E3 is also checked against the
    oracle's rounding points on sampled tokens."""
    from mi355moe import _lib, ops, synthetic
    _say(f"token-row gather {numerics} T={T} n={n} K={K} N={N}")
    ex = synthetic.calibrated_layer(n, K, N, seed=T + n, device=cuda, uniform_suh=True)
    assert ex.uniform_suh and ex.desc.flags == _lib.LAYER_SHARED_W13_SUH | _lib.LAYER_UNIFORM_W13_SUH
    x = synthetic.activations(T, K, seed=T + 1, device=cuda)
    ids = (synthetic.zipf_ids(T, n, 8, seed=T + 2, device=cuda) if numerics == "split" else
           synthetic.random_ids(T, n, 8, seed=T + 2, device=cuda))
    ids[1, 2] = -1
    w = synthetic.softmax_weights(T, 8, seed=T + 3, device=cuda)

    def run():
        if numerics == "e4m3":
            return ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32)
        if numerics == "split":
            return ops.moe_forward_ids_split(ex, x, ids, w, 16, out_dtype=torch.float32)
        return ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)

    a = run()
    ex.desc.flags = _lib.LAYER_SHARED_W13_SUH
    b = run()
    ex.desc.flags = _lib.LAYER_SHARED_W13_SUH | _lib.LAYER_UNIFORM_W13_SUH
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
    if numerics == "e3":
        sample = np.array([0, 1, 2, T // 2, T - 1])
        sel_t = torch.from_numpy(sample).to(cuda)
        ids_s, w_s = ids[sel_t].cpu().numpy(), w[sel_t].cpu().numpy()
        used = np.unique(ids_s[ids_s >= 0])
        remap = {int(e): i for i, e in enumerate(used)}
        local = np.vectorize(lambda v: remap.get(int(v), len(used)))(ids_s)
        sel = torch.as_tensor(used, dtype=torch.long, device=cuda)
        lay = {k: getattr(ex, k).index_select(0, sel).cpu().numpy() for k in
               ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
        tok, exx, w16 = moe.pairs_from_routing(local, w_s, len(used), 8)
        ref_k = moe.forward(lay, x[sel_t].to(torch.float16).cpu().numpy(), tok, exx, w16, 10.0, "e3")
        r = _rel(a[sel_t].cpu().numpy(), ref_k)
        _say(f"  rel_l2 vs E3 rounding points {r:.3e}")
        assert r <= 5e-4, r


@pytest.mark.parametrize("case", ["one_token", "t17", "eight_experts_hold_every_row", "half_non_local"])
def test_prefill_edge_cases(cuda, case):
    """Edge cases of the reference's accumulator tests (code/fork/docs/OPT_MOE.md:25-27: T=1 and 17, one expert
    holding every row, half the experts non-local) on the grouped path, against the oracle's E3 rounding points
    (rel_l2 <= 5e-4) and float64 (bf16 elementwise rtol 2e-2 / atol 1e-3); tokens with no local expert get exact
    zeros."""
    from mi355moe import _lib, ops, synthetic
    _say(f"prefill edge case {case}")
    n, K, N, topk = 16, 1024, 512, 8
    T = {"one_token": 1, "t17": 17, "eight_experts_hold_every_row": 700, "half_non_local": 600}[case]
    ex = synthetic.calibrated_layer(n, K, N, seed=31 + T, device=cuda, uniform_suh=(case == "t17"))
    x = synthetic.activations(T, K, seed=T + 5, device=cuda)
    w = synthetic.softmax_weights(T, topk, seed=T + 6, device=cuda)
    emap = None
    if case == "eight_experts_hold_every_row":
        ids = torch.arange(topk, dtype=torch.int32, device=cuda).repeat(T, 1)      # 700 rows in each of 8 experts
    elif case == "half_non_local":
        n_global = 2 * n                                                           # 32 global experts, 16 local
        ids = synthetic.random_ids(T, n_global, topk, seed=T + 7, device=cuda)
        ids[:5] = torch.arange(0, 2 * topk, 2, dtype=torch.int32, device=cuda)     # tokens 0..4: no local expert
        em = torch.full((n_global,), -1, dtype=torch.int64)
        em[1::2] = torch.arange(n)                                                 # odd global ids are local
        emap = em.to(cuda)
    else:
        ids = synthetic.random_ids(T, n, topk, seed=T + 7, device=cuda)
    out32 = ops.moe_forward_ids(ex, x, ids, w, expert_map=emap, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
    out_bf = ops.moe_forward_ids(ex, x, ids, w, expert_map=emap, out_dtype=torch.bfloat16, path=_lib.PATH_PREFILL)
    torch.cuda.synchronize()
    lay = _np_layer(ex)
    local = routing.map_topk_to_local(ids.cpu().numpy(), n, None if emap is None else emap.cpu().numpy())
    tok, exx, w16 = moe.pairs_from_routing(local, w.cpu().numpy(), n, topk)
    x16 = x.to(torch.float16).cpu().numpy()
    ref_k = moe.forward(lay, x16, tok, exx, w16, 10.0, "e3")
    ref64 = moe.forward(lay, x16, tok, exx, w16, 10.0, "f64_pre")
    got = out32.cpu().numpy()
    assert np.isfinite(got).all()
    assert _rel(got, ref_k) <= 5e-4, _rel(got, ref_k)
    assert np.allclose(out_bf.float().cpu().numpy(), ref64, rtol=2e-2, atol=1e-3)
    if case == "half_non_local":
        assert not got[:5].any()


def _hot_ids(T, n, topk, seed, cuda):
    """Random distinct experts per token with expert 0 in every token's slot 0 (expert 0 then holds T rows, so a
    small-tile call runs its later 64-row quarters too)."""
    from mi355moe import synthetic
    ids = synthetic.random_ids(T, n, topk, seed=seed, device=cuda).cpu().numpy()
    for t in range(T):
        row = list(ids[t])
        if 0 in row:
            j = row.index(0)
            row[0], row[j] = row[j], row[0]
        else:
            row[0] = 0
        ids[t] = row
    return torch.from_numpy(ids).to(cuda)


@pytest.mark.parametrize("uniform", [False, True])
@pytest.mark.parametrize("numerics,n,K,N,T,topk", [("e3", 16, 1024, 512, 200, 4), ("e4m3", 16, 1024, 512, 200, 4),
                                                   ("e3", 32, 2048, 256, 300, 2), ("e4m3", 8, 4096, 1024, 130, 3)])
def test_tile_kinds_bit_equal(cuda, monkeypatch, numerics, n, K, N, T, topk, uniform):
    """The grouped GEMMs on 64-row tiles and on 128-row tiles (two workgroups per CU; chosen when the routed experts
    average at most 128 rows), on 256-row tiles, and split between small and 256-row tiles by segment size, forced
    with MI355MOE_PREFILL_TILES: bit-identical outputs, including a hot expert whose 130..300 rows span up to four
    64-row quarters or three 128-row halves of its segments. uniform: every expert shares one w13 suh, so the GEMMs
    read one gathered row per token through the rows' tokens; bit-identical as well to the same layer run with one
    gathered row per pair (the layer's uniform flag cleared)."""
    from mi355moe import _lib, ops, synthetic
    _say(f"tile kinds: {numerics} n={n} K={K} N={N} T={T} topk={topk} uniform_suh={uniform}")
    ex = synthetic.calibrated_layer(n, K, N, seed=n + K + T, device=cuda, uniform_suh=uniform)
    assert ex.uniform_suh == uniform
    x = synthetic.activations(T, K, seed=T + 11, device=cuda)
    ids = _hot_ids(T, n, topk, T + 12, cuda)
    w = synthetic.softmax_weights(T, topk, seed=T + 13, device=cuda)
    outs = []
    for kind in ("small", "large", "hybrid", "mid"):
        monkeypatch.setenv("MI355MOE_PREFILL_TILES", kind)
        if numerics == "e3":
            o = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
        else:
            o = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32)
        torch.cuda.synchronize()
        outs.append(o)
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(outs[0], outs[2])
    assert torch.equal(outs[0], outs[3])
    if uniform:                                                      # per-pair rows, every tile kind
        ex.desc.flags &= ~_lib.LAYER_UNIFORM_W13_SUH
        for kind in ("small", "large", "hybrid", "mid"):
            monkeypatch.setenv("MI355MOE_PREFILL_TILES", kind)
            if numerics == "e3":
                o = ops.moe_forward_ids(ex, x, ids, w, out_dtype=torch.float32, path=_lib.PATH_PREFILL)
            else:
                o = ops.moe_forward_ids_e4m3(ex, x, ids, w, out_dtype=torch.float32)
            torch.cuda.synchronize()
            assert torch.equal(outs[0], o), kind


def test_few_row_tiles_vs_oracle(cuda):
    """The automatic choice at ~27 rows per expert (P = 432 <= 64 n: the mid-tile kernels, 128-row halves) with a hot
    expert of 144 rows (two halves): fp32 output against the E3 rounding points (rel_l2 <= 5e-4) and float64
    (rel_l2 <= 5e-3), bf16 elementwise rtol 2e-2 / atol 1e-3."""
    from mi355moe import _lib, ops, synthetic
    n, K, N, T, topk, limit = 16, 1024, 512, 144, 3, 10.0
    _say(f"few-row tiles vs oracle n={n} K={K} N={N} T={T} topk={topk}")
    ex = synthetic.calibrated_layer(n, K, N, seed=77, device=cuda)
    x = synthetic.activations(T, K, seed=78, device=cuda)
    ids = _hot_ids(T, n, topk, 79, cuda)
    w = synthetic.softmax_weights(T, topk, seed=80, device=cuda)
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
    assert _rel(got, ref_k) <= 5e-4, _rel(got, ref_k)
    assert _rel(got, ref64) <= 5e-3, _rel(got, ref64)
    assert np.allclose(out_bf.float().cpu().numpy(), ref64, rtol=2e-2, atol=1e-3)
