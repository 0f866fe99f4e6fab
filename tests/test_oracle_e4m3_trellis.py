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


def test_storage_order_matches_both_reference_forms():
    """The byte order of the extension's e4m3 rows, pinned to the reference's two independent statements of it: its
    test's perm_cols (byte p -> column, code/fork/tests/moee4m3/test_moe_e4m3.py:36-42: 32-groups, halves of 16,
    q = (p % 16) / 4, i = p % 4, column 2q + (i & 1) + 8 (i >> 1)) and the kernel's perm_pos (even column k -> byte,
    code/fork/kernels/moe_e4m3.cu:150-156: a = k % 16, byte 2a below 8, 2 (a - 8) + 2 from 8 on)."""
    p = np.arange(4096)
    g, pp = p // 32, p % 32
    half, pq = pp // 16, pp % 16
    q, i = pq // 4, pq % 4
    perm_cols = g * 32 + half * 16 + 2 * q + (i & 1) + 8 * (i >> 1)
    assert np.array_equal(e4m3_trellis.storage_columns(4096), perm_cols)
    k = np.arange(0, 4096, 2)
    a = k & 15
    perm_pos = (k & ~31) + (k & 16) + np.where(a < 8, 2 * a, 2 * (a - 8) + 2)
    assert np.array_equal(e4m3_trellis.storage_columns(4096)[perm_pos], k)          # byte perm_pos(k) holds k
    assert np.array_equal(e4m3_trellis.storage_columns(4096)[perm_pos + 1], k + 1)  # pairs stay adjacent
    rows = _rng(9).integers(0, 256, size=(3, 256)).astype(np.uint8)
    assert np.array_equal(e4m3_trellis.from_storage(e4m3_trellis.to_storage(rows)), rows)


def test_act_quant_codes_are_act_quant():
    g = _rng(11)
    x = g.standard_normal((4, 256)).astype(np.float16)
    suh = np.ones((4, 256), np.float16)
    c, s = e4m3_trellis.act_quant_codes(x, suh)
    q, s2 = e4m3_trellis.act_quant(x, suh)
    assert c.dtype == np.uint8 and np.array_equal(s, s2)
    assert np.array_equal(e4m3.decode(c).astype(np.float32), q)


def _spec_proj16_torch(a16, tr, suh, svh):
    """spec_proj16 (code/fork/overlay/glm53_moe_e4m3.py:660-664) in torch: fp32 matrix Hadamard, fp16 rounding of
    the rotated input, fp32 product with the fp16 W_q."""
    h = torch.ones(1, 1, dtype=torch.float32)
    while h.shape[0] < 128:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    h = h / 128 ** 0.5

    def rot(v):
        s = v.shape
        return (v.reshape(-1, s[-1] // 128, 128) @ h.t()).reshape(s)

    w = torch.from_numpy(exl3.unpack(tr).astype(np.float32))
    x = torch.from_numpy(a16).float() * torch.from_numpy(suh.astype(np.float32))
    y = rot(x).half().float() @ w
    return (rot(y) * torch.from_numpy(svh.astype(np.float32))).double().numpy()


def test_down16_rows_vs_torch_spec():
    """down16_rows against spec_proj16 in torch; a dropped fp16 rounding of the rotated input (the variant's point)
    moves the result far more than the two Hadamard orders do."""
    n, K, N = 1, 512, 256
    layer = _layer(n, K, N, 21)
    a16 = (_rng(22).standard_normal((7, N)) * 2.0).astype(np.float16)
    suh = layer["w2_suh"][0]
    got = e4m3_trellis.down16_rows(a16, np.broadcast_to(suh, a16.shape), layer["w2_trellis"][0], layer["w2_svh"][0])
    ref = _spec_proj16_torch(a16, layer["w2_trellis"][0], suh, layer["w2_svh"][0])
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    # the butterfly and the matrix Hadamard round h to a different fp16 value for 1 of these 1,792 elements (1.2e-5)
    assert rel <= 4e-5, rel
    # the same projection without the fp16 rounding of h differs by 2.1e-4: the pin resolves that rounding
    p = a16.astype(np.float32) * suh.astype(np.float32)
    h = exl3.rotate_f64(p.astype(np.float64))
    y = exl3.rotate_f64(h @ exl3.unpack(layer["w2_trellis"][0]).astype(np.float64)) * layer["w2_svh"][0]
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) > 1.5e-4


def test_forward_down16_vs_torch_spec():
    n, K, N, T, topk = 3, 256, 128, 5, 2
    layer = _layer(n, K, N, 23)
    g = _rng(24)
    x16 = g.standard_normal((T, K)).astype(np.float16)
    ids = np.stack([g.permutation(n)[:topk] for _ in range(T)])
    tok = np.repeat(np.arange(T), topk)
    ex = ids.reshape(-1)
    w = g.random(T * topk).astype(np.float32)
    got = e4m3_trellis.forward(layer, x16, tok, ex, w, 10.0, down16=True)
    plain = e4m3_trellis.forward(layer, x16, tok, ex, w, 10.0)
    # the same gate/up, then spec_proj16 per row
    ref = np.zeros_like(got)
    for e in np.unique(ex):
        rows = np.nonzero(ex == e)[0]
        q, s = e4m3_trellis.act_quant(x16[tok[rows]], np.broadcast_to(layer["w13_suh"][e, 0], (rows.size, K)))
        a16 = e4m3_trellis.gateup_rows(q, s, layer["w13_trellis"][e, 0], layer["w13_trellis"][e, 1],
                                       layer["w13_svh"][e, 0], layer["w13_svh"][e, 1], 10.0)
        y = _spec_proj16_torch(a16, layer["w2_trellis"][e], layer["w2_suh"][e], layer["w2_svh"][e])
        np.add.at(ref, tok[rows], w[rows, None].astype(np.float64) * y)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 4e-5
    assert np.linalg.norm(got - plain) / np.linalg.norm(plain) > 1e-3       # e4m3 down differs from fp16 down
