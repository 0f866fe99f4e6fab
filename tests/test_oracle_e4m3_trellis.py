"""Pins of the trellis-sourced e4m3 oracle (oracle/e4m3_trellis.py) on the CPU: closed-form properties of the
activation quantiser and of the weight rounding, and the whole forward against an independent torch statement of the
reference's spec (code/fork/overlay/glm53_moe_e4m3.py:654-674: spec_decode, _spec_rot as an fp32 matrix product,
_spec_q through torch's float8_e4m3fn, spec_ffn with DOWN16 off) within the reference's own e4m3 tolerance
(glm53_moe_e4m3.py:110, 5e-3)."""
import numpy as np
import torch

from oracle import e4m3, e4m3_trellis, exl3


def _rng(seed):
    return np.random.default_rng(seed)


def _layer(n, K, N, seed):
    g = _rng(seed)
    tr13 = g.integers(-32768, 32768, size=(n, 2, K // 16, N // 16, 64), dtype=np.int64).astype(np.int16)
    tr2 = g.integers(-32768, 32768, size=(n, N // 16, K // 16, 64), dtype=np.int64).astype(np.int16)
    suh = (np.where(g.random((n, 1, K)) < 0.5, -1.0, 1.0) * (0.5 + g.random((n, 1, K)))).astype(np.float16)
    return {"w13_trellis": tr13, "w13_suh": np.concatenate([suh, suh], axis=1),
            "w13_svh": (np.abs(g.standard_normal((n, 2, N))) * 0.05).astype(np.float16),
            "w2_trellis": tr2,
            "w2_suh": (np.where(g.random((n, N)) < 0.5, -1.0, 1.0)).astype(np.float16),
            "w2_svh": (np.abs(g.standard_normal((n, K))) * 0.05).astype(np.float16)}


def test_act_quant_properties():
    g = _rng(1)
    x = g.standard_normal((5, 512)).astype(np.float16)
    suh = (np.where(g.random(512) < 0.5, -1.0, 1.0) * (0.5 + g.random(512))).astype(np.float16)
    q, s = e4m3_trellis.act_quant(x, np.broadcast_to(suh, x.shape))
    v64 = exl3.rotate_f64(x.astype(np.float64) * suh.astype(np.float64))
    amax = np.abs(v64).max(axis=1)
    # the scale is amax / 448 of the fp32 rotation (within fp32 rounding of the butterflies)
    assert np.allclose(s.astype(np.float64), amax / 448.0, rtol=1e-5)
    # every value is on the e4m3 grid and the row maximum lands on +-448
    grid = set(e4m3.decode_table()[~np.isnan(e4m3.decode_table())].tolist())
    assert set(np.unique(q).tolist()) <= grid
    assert np.array_equal(np.abs(q).max(axis=1), np.full(5, 448.0, np.float32))
    # q * s is v to within half an e4m3 step (3 mantissa bits: 2^-4 relative; 2^-10 absolute in the subnormals)
    err = np.abs(q.astype(np.float64) * s[:, None] - v64)
    bound = np.maximum(np.abs(v64) * 2.0 ** -4, s[:, None].astype(np.float64) * 2.0 ** -10) * 1.0001 + 1e-6 * amax[:, None]
    assert np.all(err <= bound)


def test_act_quant_zero_row():
    q, s = e4m3_trellis.act_quant(np.zeros((2, 256), np.float16), np.ones((2, 256), np.float16))
    assert np.array_equal(s, np.ones(2, np.float32)) and not q.any()


def test_weights_rounding_is_nearest():
    tr = _rng(2).integers(-32768, 32768, size=(4, 4, 64), dtype=np.int64).astype(np.int16)
    wq = exl3.unpack(tr).astype(np.float64)
    w8 = e4m3_trellis.weights_e4m3(tr).astype(np.float64)
    tab = e4m3.decode_table()
    vals = np.unique(tab[~np.isnan(tab)].astype(np.float64))
    # brute force: no grid value is strictly closer to W_q than the chosen one
    d_best = np.abs(vals[None, :] - wq.reshape(-1, 1)).min(axis=1)
    assert np.allclose(np.abs(w8.reshape(-1) - wq.reshape(-1)), d_best, rtol=0, atol=0)


def _spec_torch(layer, x16, tok, ex, w, limit):
    """The reference's spec_ffn in torch, written from glm53_moe_e4m3.py:654-674 (fp32 matrix Hadamard, float8 casts)."""
    h = torch.ones(1, 1, dtype=torch.float32)
    while h.shape[0] < 128:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    h = h / 128 ** 0.5

    def rot(v):
        s = v.shape
        return (v.reshape(-1, s[-1] // 128, 128) @ h.t()).reshape(s)

    def q8(v):
        sc = v.abs().amax(dim=-1, keepdim=True) / 448.0
        sc = torch.where(sc > 0, sc, torch.ones_like(sc))
        return (v / sc).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).to(torch.float32) * sc

    def proj(xh, tr, suh, svh):
        wq = torch.from_numpy(exl3.unpack(tr).astype(np.float32))
        w8 = wq.to(torch.float8_e4m3fn).to(torch.float32)
        y = q8(rot(xh.float() * torch.from_numpy(suh.astype(np.float32)))) @ w8
        return rot(y) * torch.from_numpy(svh.astype(np.float32))

    T, K = x16.shape
    out = torch.zeros(T, K, dtype=torch.float64)
    xt = torch.from_numpy(x16)
    for e in np.unique(ex[ex >= 0]):
        rows = np.nonzero(ex == e)[0]
        xs = xt[torch.from_numpy(tok[rows])]
        gv = proj(xs, layer["w13_trellis"][e, 0], layer["w13_suh"][e, 0], layer["w13_svh"][e, 0])
        uv = proj(xs, layer["w13_trellis"][e, 1], layer["w13_suh"][e, 1], layer["w13_svh"][e, 1])
        a = torch.nn.functional.silu(gv.clamp(max=limit)) * uv.clamp(min=-limit, max=limit)
        y = proj(a.half(), layer["w2_trellis"][e], layer["w2_suh"][e], layer["w2_svh"][e])
        for i, r in enumerate(rows):
            out[tok[r]] += float(w[r]) * y[i].double()
    return out.numpy()


def test_forward_vs_torch_spec():
    n, K, N, T, topk = 4, 256, 128, 6, 2
    layer = _layer(n, K, N, 3)
    g = _rng(4)
    x16 = g.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([g.permutation(n)[:topk] for _ in range(T)])
    ids[0, 1] = -1                                                    # an invalid slot is skipped
    tok = np.repeat(np.arange(T), topk)
    ex = ids.reshape(-1)
    w = g.random(T * topk).astype(np.float32)
    got = e4m3_trellis.forward(layer, x16, tok, ex, w, 10.0)
    ref = _spec_torch(layer, x16, tok, ex, w, 10.0)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 1e-5, rel                                          # no e4m3 code differs on these seeds
    assert np.abs(got).max() > 0
    # and far from the E3 fp16 numerics only by the e4m3 rounding (not a dropped term): same order of magnitude
    assert 0.5 < np.linalg.norm(got) / np.linalg.norm(ref) < 2.0
