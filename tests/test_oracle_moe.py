"""Pins the MoE forward of the oracle (oracle/csrc/oracle.c through oracle/moe.py) against an independent numpy
float64 composition of the layer definition (oracle/exl3.linear_f64, itself pinned by the explicit dequantized
matrix) and checks that the kernel-rounding modes stay within the reference's own end-to-end tolerance
(code/fork/tests/test_e2e_vs_f64.py:6: e <= 5e-3) of float64."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import exl3, moe, routing


def _layer(rng, n, K, N, svh=0.05, shared_suh=False):
    def sg(shape):
        return np.where(rng.random(shape) < 0.5, -1.0, 1.0)
    lay = {
        "w13_trellis": rng.integers(-32768, 32768, size=(n, 2, K // 16, N // 16, 64), dtype=np.int16),
        "w13_suh": sg((n, 2, K)).astype(np.float16),
        "w13_svh": (sg((n, 2, N)) * np.abs(rng.standard_normal((n, 2, N))) * svh).astype(np.float16),
        "w2_trellis": rng.integers(-32768, 32768, size=(n, N // 16, K // 16, 64), dtype=np.int16),
        "w2_suh": sg((n, N)).astype(np.float16),
        "w2_svh": (sg((n, K)) * np.abs(rng.standard_normal((n, K))) * svh).astype(np.float16),
    }
    if shared_suh:        # gate and up share one input rotation (production's E3 tier requires it)
        lay["w13_suh"][:, 1] = lay["w13_suh"][:, 0]
    return lay


def _numpy_f64(layer, x16, tok, ex, w16, L, pre):
    out = np.zeros((x16.shape[0], layer["w2_svh"].shape[1]))
    for t, e, w in zip(tok, ex, w16):
        if e < 0:
            continue
        xs = x16[t:t + 1].astype(np.float64)
        g = exl3.linear_f64(xs, layer["w13_trellis"][e, 0], layer["w13_suh"][e, 0], layer["w13_svh"][e, 0])
        u = exl3.linear_f64(xs, layer["w13_trellis"][e, 1], layer["w13_suh"][e, 1], layer["w13_svh"][e, 1])
        if pre:
            if L:
                g = np.minimum(g, L)
                u = np.clip(u, -L, L)
            a = g / (1 + np.exp(-g)) * u
        else:
            s = g / (1 + np.exp(-g))
            if L:
                s = np.minimum(s, L)
                u = np.clip(u, -L, L)
            a = s * u
        d = exl3.linear_f64(a, layer["w2_trellis"][e], layer["w2_suh"][e], layer["w2_svh"][e])
        out[t] += float(w) * d[0]
    return out


@pytest.mark.parametrize("L,pre", [(10.0, False), (0.0, False), (1.0, True)])
def test_c_f64_equals_numpy_f64(L, pre):
    rng = np.random.default_rng(0)
    n, K, N, T, topk = 4, 256, 128, 3, 2
    layer = _layer(rng, n, K, N, svh=0.2)
    x16 = rng.standard_normal((T, K)).astype(np.float16)
    ids = np.array([[0, 3], [1, 5], [2, 0]])
    local = routing.map_topk_to_local(ids, n)
    tok, ex, w16 = moe.pairs_from_routing(local, rng.random((T, topk)), n, topk)
    got = moe.forward(layer, x16, tok, ex, w16, L, "f64_pre" if pre else "f64")
    ref = _numpy_f64(layer, x16, tok, ex, w16, L, pre)
    assert np.allclose(got, ref, rtol=1e-9, atol=1e-12)
    assert np.all(got[1, :] == got[1, :])


@pytest.mark.parametrize("mode,ref_mode", [("decode", "f64"), ("decode_x", "f64"), ("e3", "f64_pre")])
def test_kernel_modes_within_e2e_tolerance_of_f64(mode, ref_mode):
    rng = np.random.default_rng(1)
    n, K, N, T, topk = 8, 512, 256, 4, 4
    layer = _layer(rng, n, K, N, svh=0.05, shared_suh=(mode == "e3"))
    x16 = rng.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([rng.permutation(n)[:topk] for _ in range(T)])
    local = routing.map_topk_to_local(ids, n)
    w = np.exp(rng.standard_normal((T, topk)))
    w = w / w.sum(-1, keepdims=True) * 2.5
    tok, ex, w16 = moe.pairs_from_routing(local, w, n, topk)
    got = moe.forward(layer, x16, tok, ex, w16, 10.0, mode).astype(np.float64)
    ref = moe.forward(layer, x16, tok, ex, w16, 10.0, ref_mode)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 5e-3, rel
    assert np.allclose(got, ref, rtol=2e-2, atol=1e-3 * np.abs(ref).max())


def _constant_tiles(rng, shape, patterns):
    """int16 trellis whose every 16x16 tile repeats one nibble (all 256 states of the tile equal n * 0x1111)."""
    pick = rng.choice(np.asarray(patterns, np.int64), size=shape[:-1])
    return np.repeat(pick[..., None], 64, axis=-1).astype(np.uint16).view(np.int16)


def test_decode_x_changes_only_the_weight_rounding():
    """decode_x differs from decode only in the codebook sums' final fp16 rounding: on tiles whose states all have
    fp16-exact sums the two modes agree bit for bit, and one tile of an inexact state makes them differ."""
    ex, cb = exl3.codebook_exact(), exl3.codebook().astype(np.float64)
    exact = [n * 0x1111 for n in range(16) if ex[n * 0x1111] == cb[n * 0x1111]]
    inexact = [n * 0x1111 for n in range(16) if ex[n * 0x1111] != cb[n * 0x1111]]
    assert len(exact) >= 8 and len(inexact) >= 3
    rng = np.random.default_rng(5)
    n, K, N, T = 4, 256, 128, 3
    layer = _layer(rng, n, K, N)
    layer["w13_trellis"] = _constant_tiles(rng, layer["w13_trellis"].shape, exact)
    layer["w2_trellis"] = _constant_tiles(rng, layer["w2_trellis"].shape, exact)
    x16 = rng.standard_normal((T, K)).astype(np.float16)
    tok = np.array([0, 1, 2, 2], np.int32)
    exs = np.array([0, 1, 2, 3], np.int32)
    w16 = np.array([1.0, 0.5, 0.25, 2.0], np.float16)
    a = moe.forward(layer, x16, tok, exs, w16, 10.0, "decode")
    b = moe.forward(layer, x16, tok, exs, w16, 10.0, "decode_x")
    assert np.array_equal(a, b) and np.any(a != 0)
    layer["w2_trellis"][1, :, 0, :] = np.uint16(inexact[0]).view(np.int16)
    a = moe.forward(layer, x16, tok, exs, w16, 10.0, "decode")
    b = moe.forward(layer, x16, tok, exs, w16, 10.0, "decode_x")
    assert not np.array_equal(a[1], b[1]) and np.array_equal(a[[0, 2]], b[[0, 2]])


def test_sentinel_pairs_contribute_nothing():
    rng = np.random.default_rng(2)
    n, K, N = 4, 256, 128
    layer = _layer(rng, n, K, N)
    x16 = rng.standard_normal((2, K)).astype(np.float16)
    tok = np.array([0, 0, 1, 1], np.int32)
    ex = np.array([1, -1, -1, -1], np.int32)
    w16 = np.ones(4, np.float16)
    out = moe.forward(layer, x16, tok, ex, w16, 10.0, "decode")
    assert np.all(out[1] == 0) and np.any(out[0] != 0)
