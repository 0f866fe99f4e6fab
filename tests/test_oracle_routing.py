"""Pins the routing part of the oracle (oracle/routing.py): brute force on tiny inputs (Python sorting and loops),
float64 matrix products, torch's stable argsort and a torch-op restatement of the segment tables (the form of the
reference's own route oracle, code/fork/tests/test_units.py:51-78)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import routing


def _bf16_values(rng, shape, scale=1.0):
    return routing.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(10000) * 10.0 ** rng.integers(-5, 5, 10000)).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(routing.bf16_round(v), ref)


def _round_dyadic(num: int, shift: int, bits: int) -> tuple[int, int]:
    """num / 2**shift rounded to `bits` significant bits, nearest even, as (m, e) with value m * 2**e (integers
    only; no subnormals are involved at router magnitudes)."""
    if num == 0:
        return 0, 0
    sign = -1 if num < 0 else 1
    a = abs(num)
    drop = a.bit_length() - bits
    if drop <= 0:
        return sign * a, -shift
    q, r = divmod(a, 1 << drop)
    half = 1 << (drop - 1)
    if r > half or (r == half and q & 1):
        q += 1
    return sign * q, drop - shift


def _exact_router_logit(xrow, wrow) -> float:
    """bf16(fp32(exact dot)) by integer arithmetic: every bf16 value is m * 2**e with integer m, so the dot product is
    an integer over a power of two; it is rounded to 24 then to 8 significant bits (nearest even) with integers."""
    terms = []
    for a, b in zip(xrow, wrow):
        ma, ea = math.frexp(float(a))
        mb, eb = math.frexp(float(b))
        terms.append((int(ma * (1 << 24)) * int(mb * (1 << 24)), ea + eb - 48))
    lo = min(e for _, e in terms)
    num = sum(m << (e - lo) for m, e in terms)
    m24, e24 = _round_dyadic(num, -lo, 24)
    m8, e8 = _round_dyadic(m24, -e24, 8)
    return math.ldexp(m8, e8)


def test_router_logits_exact_rational():
    """Every oracle logit equals the bf16 rounding (through fp32) of the exact dot product, computed with integers."""
    rng = np.random.default_rng(1)
    T, E, K = 3, 5, 1024
    x, w = _bf16_values(rng, (T, K)), _bf16_values(rng, (E, K), 0.02)
    got = routing.router_logits(x, w)
    for t in range(T):
        for e in range(E):
            assert float(got[t, e]) == _exact_router_logit(x[t], w[e]), (t, e)


def test_router_logits_double_rounding_through_fp32():
    """A dot product of exactly 1 + 2**-8 + 2**-30: rounded straight to bf16 it is 1 + 2**-7, but fp32 first rounds
    it onto the bf16 midpoint 1 + 2**-8, which then ties to the even 1.0 -- what torch's double -> bf16 and an fp32
    GEMM with a bf16 output both give."""
    K = 512
    x = np.zeros((2, K), np.float32)
    w = np.zeros((1, K), np.float32)
    x[0, :3] = [1.0, 2.0 ** -8, 2.0 ** -15]
    w[0, :3] = [1.0, 1.0, 2.0 ** -15]
    x[1, :3] = [1.0, 2.0 ** -8, 2.0 ** -7]          # 1 + 2**-8 + 2**-22: fp32 keeps it above the midpoint
    got = routing.router_logits(x, w)
    assert got[0, 0] == np.float32(1.0)
    assert got[1, 0] == np.float32(1.0 + 2.0 ** -7)
    ref = (torch.from_numpy(x).double() @ torch.from_numpy(w).double().t()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)


def test_router_logits_match_reference_oracle_expression():
    """The reference's own router oracle, (X.double() @ W.t()).to(bfloat16).float()
    (code/fork/tests/router_topk_agreement.py:82), evaluated by torch at the decode configuration's shapes."""
    rng = np.random.default_rng(2)
    x, w = _bf16_values(rng, (64, 4096)), _bf16_values(rng, (288, 4096), 0.02)
    got = routing.router_logits(x, w)
    ref = (torch.from_numpy(x).double() @ torch.from_numpy(w).double().t()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)
    # and the values are bf16 (low 16 bits clear) within one bf16 step of the float64 dot product
    assert not np.any(got.view(np.uint32) & 0xFFFF)
    f64 = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.all(np.abs(got - f64) <= np.abs(f64) * 2.0 ** -8 + 1e-30)


def test_sigmoid_is_correctly_rounded_on_samples():
    z = np.array([-30, -5, -1, -1e-3, 0, 1e-3, 0.5, 1, 5, 30], np.float32)
    s = routing.sigmoid_f32(z)
    for zi, si in zip(z, s):
        exact = 1.0 / (1.0 + math.exp(-float(zi)))
        assert abs(float(si) - exact) <= abs(float(np.spacing(si))) / 2 + 1e-300


def test_sigmoid_bits_is_the_e3_formula():
    """The oracle's C sigmoid over a range of bit patterns (the GPU test's reference) equals numpy's statement of
    1 / (1 + (float)exp(-(double)g)) in float32, and its g are the patterns' floats."""
    from oracle import moe
    for first in (0x3F000000, 0xC1000000, 0x42AE0000 - (1 << 18)):
        g, s = moe.sigmoid_bits(first, 1 << 18)
        assert np.array_equal(g.view(np.uint32), np.arange(first, first + (1 << 18), dtype=np.uint32))
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
        ref = (np.float32(1.0) / (np.float32(1.0) + e)).astype(np.float32)
        assert np.array_equal(s.view(np.uint32), ref.view(np.uint32))


def _brute_topk(logits, bias, topk, scale):
    s = routing.sigmoid_f32(logits)
    ids, ws = [], []
    for t in range(s.shape[0]):
        choice = [(float(np.float32(s[t, e] + bias[e])), e) for e in range(s.shape[1])]
        picked = [e for _, e in sorted(choice, key=lambda ce: (-ce[0], ce[1]))[:topk]]
        tot = np.float32(0)
        for e in picked:
            tot = np.float32(tot + s[t, e])
        ids.append(picked)
        ws.append([np.float32(np.float32(s[t, e] / np.float32(tot + np.float32(1e-20))) * np.float32(scale))
                   for e in picked])
    return np.array(ids, np.int32), np.array(ws, np.float32)


def test_topk_sigmoid_bias_brute_force_and_ties():
    rng = np.random.default_rng(3)
    for trial in range(20):
        E = int(rng.integers(8, 40))
        lg = rng.standard_normal((3, E)).astype(np.float32)
        b = (rng.standard_normal(E) * 0.01).astype(np.float32)
        if trial % 3 == 0:
            lg[:, 3] = lg[:, 5]
            b[3] = b[5]                      # an exact tie: the lower id first
        ids, w = routing.topk_sigmoid_bias(lg, b, 4, 2.5)
        bi, bw = _brute_topk(lg, b, 4, 2.5)
        assert np.array_equal(ids, bi)
        assert np.array_equal(w, bw)
        assert np.allclose(w.sum(-1), 2.5, rtol=1e-6)


def test_topk_uses_bias_for_choice_only():
    lg = np.zeros((1, 4), np.float32)
    b = np.array([0.0, 0.0, 1.0, 0.0], np.float32)
    ids, w = routing.topk_sigmoid_bias(lg, b, 1, 1.0, renormalize=False)
    assert ids[0, 0] == 2 and w[0, 0] == np.float32(0.5)   # weight is sigmoid(0), not sigmoid + bias


def test_map_topk_to_local_cases():
    ids = np.array([[0, 5, 287, 288, -1, 3]])
    assert routing.map_topk_to_local(ids, 288).tolist() == [0, 5, 287, 288, 288, 3]
    emap = np.array([-1, 0, 1, -1, 2, 3], np.int64)     # global 6 experts, 4 local
    ids = np.array([[0, 1, 2, 3, 4, 5, 6, -2]])
    assert routing.map_topk_to_local(ids, 4, emap).tolist() == [4, 0, 1, 4, 2, 3, 4, 4]
    assert routing.map_topk_to_local(ids, 4, np.zeros(0, np.int64)).tolist() == [4] * 8


def _torch_route_oracle(local: np.ndarray, n: int, R: int, seg: int):
    """Segments restated with torch ops (cumsum / searchsorted), the form of test_units.py:51-78."""
    lt = torch.from_numpy(local.astype(np.int64))
    c = torch.bincount(lt, minlength=n + 1)
    cnt = c[:n]
    end = torch.cumsum(cnt, 0)
    start = end - cnt
    elig = (cnt > 0) & (cnt <= R)
    nsg = torch.where(elig, (cnt + seg - 1) // seg, torch.zeros_like(cnt))
    send = torch.cumsum(nsg, 0)
    soff = send - nsg
    S = int(send[-1])
    s = torch.arange(S)
    se = torch.searchsorted(send, s, right=True)
    q = s - soff[se]
    return se.numpy(), (start[se] + seg * q).numpy(), torch.minimum(torch.full_like(q, seg), cnt[se] - seg * q).numpy()


@pytest.mark.parametrize("seed,T,n,topk,R,seg", [(0, 8, 288, 8, 1 << 30, 16), (1, 64, 32, 4, 20, 16),
                                                 (2, 300, 16, 8, 1 << 30, 64), (3, 5, 288, 8, 1, 1)])
def test_permutation_vs_torch_stable_sort(seed, T, n, topk, R, seg):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-2, n + 3, size=(T, topk))
    local = routing.map_topk_to_local(ids, n)
    p = routing.permutation(local, n, topk, R, seg)
    order = torch.argsort(torch.from_numpy(local), stable=True).numpy()
    assert np.array_equal(p["order"], order)
    assert np.array_equal(p["inv"][order], np.arange(local.size))
    assert np.array_equal(p["token"], order // topk)
    assert p["counts"].sum() == local.size
    se, s0, sr = _torch_route_oracle(local, n, R, seg)
    assert np.array_equal(p["seg_expert"], se) and np.array_equal(p["seg_row0"], s0)
    assert np.array_equal(p["seg_rows"], sr)
    # invariants: segments cover every eligible row exactly once; pe = -1 elsewhere
    cover = np.zeros(local.size, int)
    for e, r0, rn in zip(se, s0, sr):
        cover[r0:r0 + rn] += 1
        assert np.all(p["pair_expert"][r0:r0 + rn] == e)
    assert np.array_equal(cover == 1, p["pair_expert"] >= 0)
    assert len(se) <= routing.s_cap(local.size, n, seg)
