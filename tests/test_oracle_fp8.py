"""Pins the e4m3 part of the oracle (oracle/e4m3.py, oracle/csrc/fp8.c): the e4m3 rounding against torch's own
float8_e4m3fn conversion (a library routine, exhaustive over binary16 and random fp32 inputs and every tie), the
per-row quantisation against the reference's torch formula (code/fork/overlay/glm53_moe_e4m3.py:648-652) and known
answers, and the layer forward against an independent numpy float64 composition of dequantised matrices."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import e4m3


def _torch_e4m3(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_matches_torch_for_every_code():
    tab = e4m3.decode_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(tab), nan) and nan.sum() == 2
    assert np.array_equal(tab[~nan], ref[~nan])
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6


def test_encode_matches_torch_on_every_binary16_value():
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    v = np.clip(h, -448.0, 448.0)
    got = e4m3.encode(v)
    assert np.array_equal(got, _torch_e4m3(v))
    assert np.array_equal(e4m3.encode_fast(v), got)


def test_encode_matches_torch_on_random_fp32_and_ties():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(20000) * s for s in (1e-3, 0.02, 1.0, 30.0, 200.0)]).astype(np.float32)
    tab = e4m3.decode_table().astype(np.float64)
    finite = np.sort(np.unique(tab[np.isfinite(tab)]))
    mids = ((finite[1:] + finite[:-1]) / 2).astype(np.float32)           # exact ties between neighbours
    v = np.clip(np.concatenate([v, mids, -mids]), -448.0, 448.0).astype(np.float32)
    got = e4m3.encode(v)
    assert np.array_equal(got, _torch_e4m3(v))
    assert np.array_equal(e4m3.encode_fast(v), got)
    assert e4m3.encode(np.array([448.0, 1e6, -1e6], np.float32)).tolist() == [0x7E, 0x7E, 0xFE]   # saturating


def test_quant_rows_matches_reference_formula_and_known_answers():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((6, 512)) * np.array([[1e-3], [0.1], [1], [10], [1e3], [0]])).astype(np.float32)
    q, s = e4m3.quant_rows(x)
    # glm53_moe_e4m3.py:648-652: sc = amax / 448 (1 if 0); (x / sc).clamp(-448, 448).to(float8_e4m3fn)
    xt = torch.from_numpy(x)
    sc = xt.abs().amax(dim=-1, keepdim=True) / 448.0
    sc = torch.where(sc > 0, sc, torch.ones_like(sc))
    qt = (xt / sc).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(s, sc[:, 0].numpy())
    assert np.array_equal(q, qt)
    assert s[5] == 1.0 and not e4m3.decode(q[5]).any()               # an all-zero row (signed zeros)
    assert all(np.abs(e4m3.decode(q[r])).max() == 448.0 for r in range(5))   # the row maximum maps to 448


def _layer(rng, n, K, N):
    w13 = rng.standard_normal((n, 2 * N, K)).astype(np.float32) * 0.02
    w2 = rng.standard_normal((n, K, N)).astype(np.float32) * 0.02
    w13[:, :, :128] *= 4.0                                             # blocks of different scales
    q13, s13 = e4m3.block_quant(w13)
    q2, s2 = e4m3.block_quant(w2)
    return {"w13": q13, "w13_scale": s13, "w2": q2, "w2_scale": s2}


def _dequant(q, s):
    d = e4m3.decode(q).astype(np.float64)
    return d * np.repeat(np.repeat(s.astype(np.float64), 128, axis=-2), 128, axis=-1)


def test_block_quant_known_answers():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    q, s = e4m3.block_quant(w)
    assert s.shape == (2, 3)
    for i in range(2):
        for j in range(3):
            blk = w[128 * i:128 * i + 128, 128 * j:128 * j + 128]
            assert s[i, j] == np.float32(np.abs(blk).max() / np.float32(448.0))
            assert np.abs(e4m3.decode(q[128 * i:128 * i + 128, 128 * j:128 * j + 128])).max() == 448.0
    assert np.abs(_dequant(q, s) - w).max() <= np.abs(w).max() / 16      # e4m3 keeps 3 mantissa bits


@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_forward_f64_equals_numpy_composition(limit):
    rng = np.random.default_rng(3)
    n, K, N, T, k = 4, 256, 128, 5, 2
    lay = _layer(rng, n, K, N)
    x = rng.standard_normal((T, K)).astype(np.float32)
    ids = np.stack([rng.permutation(n)[:k] for _ in range(T)])
    ids[1, 1] = -1
    w = rng.random((T, k)).astype(np.float32)
    tok, ex, pw = e4m3.pairs_fp32(ids, w, n)
    got = e4m3.forward(lay, x, tok, ex, pw, limit, "f64")
    qx, sx = e4m3.quant_rows(x)
    xd = e4m3.decode(qx).astype(np.float64) * sx[:, None].astype(np.float64)
    ref = np.zeros((T, K))
    for t, e, wt in zip(tok, ex, pw):
        if e < 0:
            continue
        W13 = _dequant(lay["w13"][e], lay["w13_scale"][e])
        g = W13[:N] @ xd[t]
        u = W13[N:] @ xd[t]
        if limit:
            g = np.minimum(g, limit)
            u = np.clip(u, -limit, limit)
        a = (g / (1 + np.exp(-g)) * u).astype(np.float16).astype(np.float32)
        qa, sa = e4m3.quant_rows(a[None])
        ad = e4m3.decode(qa[0]).astype(np.float64) * float(sa[0])
        ref[t] += float(wt) * (_dequant(lay["w2"][e], lay["w2_scale"][e]) @ ad)
    assert np.allclose(got, ref, rtol=1e-9, atol=1e-12)
    assert got[1].any()                                                # token 1 keeps its valid slot


def test_kernel_mode_within_tolerance_of_f64():
    rng = np.random.default_rng(4)
    n, K, N, T, k = 6, 512, 256, 8, 4
    lay = _layer(rng, n, K, N)
    x = rng.standard_normal((T, K)).astype(np.float32)
    ids = np.stack([rng.permutation(n)[:k] for _ in range(T)])
    w = rng.random((T, k)).astype(np.float32)
    tok, ex, pw = e4m3.pairs_fp32(ids, w, n)
    a = e4m3.forward(lay, x, tok, ex, pw, 10.0, "kernel").astype(np.float64)
    b = e4m3.forward(lay, x, tok, ex, pw, 10.0, "f64")
    assert np.linalg.norm(a - b) / np.linalg.norm(b) < 2e-3
