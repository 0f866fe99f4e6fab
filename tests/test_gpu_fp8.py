"""GPU parity of the e4m3 expert variant (mi355moe.fp8) against the oracle (oracle/e4m3.py, oracle/csrc/fp8.c):

  - the per-row e4m3 quantiser is bit-exact (codes and scales);
  - the layer forward agrees with the oracle's fp32 mode (the spec's exact e4m3 products summed in fp32 per
    128-k block) to rel_l2 <= 1e-6 and with float64 to rel_l2 <= 1e-4 (the reference's own e4m3 tolerance is 5e-3,
    code/fork/overlay/glm53_moe_e4m3.py:110): the kernels form every block sum from exact products on the fp16
    matrix cores (measured 2-4e-8 and <= 8.4e-6). The bf16 output is elementwise within rtol 2e-2 / atol 1e-3 of the
    fp32 oracle. Against float64 only rel_l2 <= 5e-3 holds in general: the float64 layer rounds its own intermediate
    to fp16 before the per-row requantisation, and one fp16 ulp on a row's largest element changes that row's e4m3
    scale and so every code of the row (token 77 of the full configuration: 1 % of its row).
  - at the full e4m3 configuration (T=2048, 288 experts, hidden 4096, intermediate 1024, top-8) a sample of tokens
    is checked against the oracle evaluated for those tokens only (the output of a token depends only on its own
    pairs).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import e4m3

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _host_layer(ex, experts=None):
    sel = slice(None) if experts is None else torch.as_tensor(experts, device=ex.device)
    return {"w13": ex.w13[sel].cpu().numpy(), "w13_scale": ex.w13_scale[sel].cpu().numpy(),
            "w2": ex.w2[sel].cpu().numpy(), "w2_scale": ex.w2_scale[sel].cpu().numpy()}


@pytest.mark.parametrize("K", [1024, 4096, 256, 384])   # one wave per row (256 .. 4096), one workgroup per row (384)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_quant_rows_bit_exact(cuda, dt, K):
    from mi355moe import fp8
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(37, K, generator=g, device="cuda")
    x *= torch.logspace(-3, 3, 37, device="cuda")[:, None]
    x[5] = 0
    x[9, 100] = 3e4
    x = x.to(dt)
    q, s = fp8.quant_rows(x)
    qo, so = e4m3.quant_rows(x.float().cpu().numpy())
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy(), qo)


def _routing(T, n, topk, seed, sentinel=False):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(n)[:topk] for _ in range(T)]).astype(np.int64)
    if sentinel:
        ids[0, 0] = -1
        ids[T // 2, topk - 1] = n + 3
    w = rng.random((T, topk)).astype(np.float32) + 0.1
    w = w / w.sum(-1, keepdims=True) * 2.5
    return ids, w


@pytest.mark.parametrize("n,K,N,T,topk,limit", [(8, 512, 256, 40, 4, 10.0), (16, 1024, 512, 100, 8, 0.0),
                                                (4, 256, 128, 3, 2, 10.0), (6, 512, 384, 70, 6, 1.0)])
def test_forward_vs_oracle(cuda, n, K, N, T, topk, limit):
    from mi355moe import fp8, synthetic
    ex = synthetic.fp8_layer(n, K, N, seed=11 + n, device="cuda")
    x = synthetic.activations(T, K, seed=12 + T, device="cuda")
    ids, w = _routing(T, n, topk, seed=13 + K, sentinel=True)
    out = fp8.moe_forward_ids(ex, x, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), limit=limit,
                              out_dtype=torch.float32)
    got = out.cpu().numpy()
    lay = _host_layer(ex)
    xf = x.float().cpu().numpy()
    local = np.where((ids >= 0) & (ids < n), ids, -1)
    tok, exs, pw = e4m3.pairs_fp32(local, w, n)
    ref_k = e4m3.forward(lay, xf, tok, exs, pw, limit, "kernel")
    ref64 = e4m3.forward(lay, xf, tok, exs, pw, limit, "f64")
    assert _rel(got, ref_k) <= 1e-6, _rel(got, ref_k)
    assert _rel(got, ref64) <= 1e-4, _rel(got, ref64)
    outb = fp8.moe_forward_ids(ex, x, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), limit=limit)
    assert outb.dtype == torch.bfloat16
    assert np.allclose(outb.float().cpu().numpy(), ref_k, rtol=2e-2, atol=1e-3)


def test_expert_map_and_stages(cuda):
    from mi355moe import _lib, fp8, synthetic
    n, K, N, T, topk = 6, 512, 256, 24, 4
    ex = synthetic.fp8_layer(n, K, N, seed=21, device="cuda")
    x = synthetic.activations(T, K, seed=22, device="cuda")
    n_global = 20
    emap = torch.full((n_global,), -1, dtype=torch.int64)
    emap[torch.tensor([3, 5, 7, 11, 13, 17])] = torch.arange(n)
    ids, w = _routing(T, n_global, topk, seed=23)
    got = fp8.moe_forward_ids(ex, x, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                              expert_map=emap.cuda(), out_dtype=torch.float32)
    local = emap.numpy()[ids]
    tok, exs, pw = e4m3.pairs_fp32(local, w, n)
    ref = e4m3.forward(_host_layer(ex), x.float().cpu().numpy(), tok, exs, pw, 10.0, "kernel")
    assert _rel(got.cpu().numpy(), ref) <= 5e-3
    # the stage split reproduces the full call
    out = torch.empty(T, K, dtype=torch.float32, device="cuda")
    idt, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    for st in (_lib.STAGE_ROUTE, _lib.STAGE_GATEUP, _lib.STAGE_DOWN, _lib.STAGE_COMBINE):
        fp8.moe_forward_ids(ex, x, idt, wt, expert_map=emap.cuda(), out=out, stages=st)
    assert _rel(out.cpu().numpy(), ref) <= 5e-3


def test_full_configuration_token_sample(cuda):
    """T=2048, 288 experts, hidden 4096, intermediate 1024, top-8: eight sampled tokens against the oracle."""
    from mi355moe import fp8, ops, synthetic
    n, K, N, T, topk = 288, 4096, 1024, 2048, 8
    ex = synthetic.fp8_layer(n, K, N, seed=31, device="cuda")
    wr, br = synthetic.router(n, K, seed=32, device="cuda")
    x = synthetic.activations(T, K, seed=33, device="cuda")
    ids, w = ops.router_topk(ops.router_logits(x, wr), topk, br, routed_scale=2.5)
    out = fp8.moe_forward_ids(ex, x, ids, w, limit=10.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    sample = np.array([0, 1, 517, 1024, 1500, 2046, 2047, 77])
    ids_s = ids[torch.from_numpy(sample).cuda()].cpu().numpy()
    w_s = w[torch.from_numpy(sample).cuda()].cpu().numpy()
    used = np.unique(ids_s)
    remap = {int(e): i for i, e in enumerate(used)}
    local = np.vectorize(remap.get)(ids_s)
    tok, exs, pw = e4m3.pairs_fp32(local, w_s, len(used))
    lay = _host_layer(ex, used)
    xs = x[torch.from_numpy(sample).cuda()].float().cpu().numpy()
    ref = e4m3.forward(lay, xs, tok, exs, pw, 10.0, "kernel")
    ref64 = e4m3.forward(lay, xs, tok, exs, pw, 10.0, "f64")
    got = out[torch.from_numpy(sample).cuda()].cpu().numpy()
    assert _rel(got, ref) <= 1e-6, _rel(got, ref)
    assert np.allclose(torch.from_numpy(got).to(torch.bfloat16).float().numpy(), ref, rtol=2e-2, atol=1e-3)
    assert _rel(got, ref64) <= 5e-3, _rel(got, ref64)
    assert np.isfinite(out.cpu().numpy()).all()
