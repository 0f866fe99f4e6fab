"""GPU parity of the bit-exact stages against the oracle: trellis dequant, input rotation, router logits and top-k,
and the token -> expert permutation (single-block and multi-block)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import exl3, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def test_sigmoid_against_the_e3_formula(cuda):
    """The epilogues' sigmoid over every float32 in [-87, 88] (2.24 billion values, in chunks of 2^26 bit patterns):
    variant 0 (decode epilogue) equals E3's 1 / (1 + (float)exp(-(double)g)) with IEEE float32 add and division
    (exl3_fat_moe.cu:366-369; exp from the host's libm, rounded once to float32, through the oracle's C port) bit for
    bit; variant 1 (grouped prefill epilogues) stays within 5 ulp of it (the exhaustive maximum)."""
    from mi355moe import ops
    from oracle import moe
    ranges = [(0, int(np.array([88.0], np.float32).view(np.uint32)[0]) + 1),                  # +0 .. 88
              (0x80000000, int(np.array([-87.0], np.float32).view(np.uint32)[0]) + 1)]       # -0 .. -87
    total = sum(hi - lo for lo, hi in ranges)
    _say(f"sigmoid over {total} values")
    chunk = 1 << 26
    bad0, worst1, differ1, worst_g = 0, 0, 0, 0.0
    for lo, hi in ranges:
        for first in range(lo, hi, chunk):
            n = min(chunk, hi - first)
            g, ref = moe.sigmoid_bits(first, n)
            gt = torch.from_numpy(g).to(cuda)
            got0 = ops.sigmoid(gt, 0).cpu().numpy()
            bad0 += int(np.count_nonzero(got0.view(np.uint32) != ref.view(np.uint32)))
            got1 = ops.sigmoid(gt, 1).cpu().numpy()
            ulp = np.abs(got1.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))   # both >= 0
            i = int(np.argmax(ulp))
            if int(ulp[i]) > worst1:
                worst1, worst_g = int(ulp[i]), float(g[i])
            differ1 += int(np.count_nonzero(ulp))
            del gt, got0, got1, ulp
    _say(f"  exact variant: {bad0} differ; fast variant: max {worst1} ulp (first at g = {worst_g!r}), "
         f"{differ1 / total:.3%} of values differ")
    assert bad0 == 0, bad0
    assert worst1 <= 5, worst1


@pytest.mark.parametrize("kt,nt", [(1, 8), (16, 64), (256, 64), (64, 256)])
def test_dequant_bit_exact(cuda, kt, nt):
    from mi355moe import ops
    _say(f"dequant kt={kt} nt={nt}")
    g = torch.Generator().manual_seed(kt * 1000 + nt)
    t = torch.randint(-32768, 32768, (kt, nt, 64), generator=g, dtype=torch.int32).to(torch.int16)
    got = ops.dequant(t.to(cuda)).cpu().numpy()
    ref = exl3.unpack(t.numpy())
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_dequant_every_state(cuda):
    """Tiles whose words make every 16-bit state occur: state 8l+j of a tile reads bits of words l-1, l; tiles
    of constant words w repeat the states of (w:w); 65536 such words cover all states at offset 16."""
    from mi355moe import ops
    w = np.arange(65536, dtype=np.uint32) * 0x10001                 # word = s:s
    tiles = np.repeat(w[:, None], 32, axis=1).view(np.int16).reshape(65536 // 8, 8, 64)
    got = ops.dequant(torch.from_numpy(tiles.copy()).to(cuda)).cpu().numpy()
    ref = exl3.unpack(tiles)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    states = exl3.states(tiles)
    assert len(np.unique(states)) == 65536


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_rot_in_bit_exact(cuda, xdt):
    from mi355moe import ops
    from mi355moe.layer import _table
    _say(f"rot_in {xdt}")
    g = torch.Generator().manual_seed(5)
    n, K, P, T = 6, 1024, 40, 7
    x = (torch.randn(T, K, generator=g) * 3).to(xdt)
    suh = (torch.randn(n, K, generator=g)).to(torch.float16)
    tok = torch.randint(0, T, (P,), generator=g, dtype=torch.int32)
    pe = torch.randint(0, n, (P,), generator=g, dtype=torch.int32)
    pe[3] = -1
    suh_d = suh.to(cuda)
    got = ops.rot_in(x.to(cuda), tok.to(cuda), pe.to(cuda), _table(suh_d, ())).cpu()
    x16 = x.to(torch.float16).numpy()
    for j in range(P):
        if pe[j] < 0:
            assert torch.isnan(got[j]).all()
            continue
        ref = exl3.rot_in(x16[tok[j]][None], suh[pe[j]].numpy())[0]
        assert np.array_equal(got[j].numpy().view(np.uint16), ref.view(np.uint16)), j


@pytest.mark.parametrize("T", [8, 300])
def test_router_logits_bit_exact(cuda, T):
    """Logits = bf16(x . W) through fp32, bit for bit; the first rows hold constructed dot products on either side of
    a bf16 midpoint after fp32 rounding (1 + 2**-8 + 2**-30 ties to 1.0, 1 + 2**-8 + 2**-22 rounds up)."""
    from mi355moe import ops, synthetic
    _say(f"router_logits T={T} E=288 K=4096")
    w, _ = synthetic.router(288, 4096, seed=1, device="cpu")
    x = synthetic.activations(T, 4096, seed=2, device="cpu")
    x[:2] = 0
    w[0] = 0
    x[0, :3] = torch.tensor([1.0, 2.0 ** -8, 2.0 ** -15])
    x[1, :3] = torch.tensor([1.0, 2.0 ** -8, 2.0 ** -7])
    w[0, :3] = torch.tensor([1.0, 1.0, 2.0 ** -15])
    got = ops.router_logits(x.to(cuda), w.to(cuda)).cpu().numpy()
    ref = routing.router_logits(x.float().numpy(), w.float().numpy())
    assert got[0, 0] == 1.0 and got[1, 0] == 1.0 + 2.0 ** -7
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T,E,K", [(255, 288, 4096), (256, 288, 4096), (1000, 100, 1024), (4097, 17, 512),
                                   (300, 1, 8192)])
def test_router_logits_large_t_bit_exact(cuda, T, E, K):
    """From 256 tokens the logits come from the float64 MFMA GEMM (16 tokens x 32 experts per wave, each lane group
    walking its own quarter of K): ragged tokens and experts, the smallest and largest K, bit for bit against the
    oracle, and the constructed midpoint cases in the first rows."""
    from mi355moe import ops, synthetic
    _say(f"router_logits T={T} E={E} K={K}")
    w, _ = synthetic.router(E, K, seed=E + K, device="cpu")
    x = synthetic.activations(T, K, seed=T, device="cpu")
    x[:2] = 0
    w[0] = 0
    x[0, :3] = torch.tensor([1.0, 2.0 ** -8, 2.0 ** -15])
    x[1, K - 3:] = torch.tensor([1.0, 2.0 ** -8, 2.0 ** -15])      # in the last lane group's quarter of K
    w[0, :3] = torch.tensor([1.0, 1.0, 2.0 ** -15])
    w[0, K - 3:] = torch.tensor([1.0, 1.0, 2.0 ** -7])
    got = ops.router_logits(x.to(cuda), w.to(cuda)).cpu().numpy()
    ref = routing.router_logits(x.float().numpy(), w.float().numpy())
    assert got[0, 0] == 1.0 and got[1, 0] == 1.0 + 2.0 ** -7
    assert np.array_equal(got, ref)


def test_router_picks_4096_tokens(cuda):
    """Top-8 sets of 4,096 tokens from the GPU router (logits + top-k) against the top-8 of the reference's router
    oracle, bf16(float64 dot) (code/fork/tests/router_topk_agreement.py:82): ids in pick order bit for bit (largest
    score + bias first, lower id among equals), and the weights of the first 64 tokens against the oracle's loop."""
    from mi355moe import ops, synthetic
    _say("router logits + top-8, T=4096 E=288")
    T = 4096
    w, b = synthetic.router(288, 4096, seed=11, device="cpu")
    x = synthetic.activations(T, 4096, seed=12, device="cpu")
    ids, wts = ops.router_topk(ops.router_logits(x.to(cuda), w.to(cuda)), 8, b.to(cuda), routed_scale=2.5)
    lg = routing.router_logits(x.float().numpy(), w.float().numpy())
    choice = (routing.sigmoid_f32(lg) + b.numpy()[None, :]).astype(np.float32)
    want = np.argsort(-choice.astype(np.float64), axis=1, kind="stable")[:, :8]
    assert np.array_equal(ids.cpu().numpy(), want)
    rid, rw = routing.topk_sigmoid_bias(lg[:64], b.numpy(), 8, 2.5)
    assert np.array_equal(ids[:64].cpu().numpy(), rid)
    assert np.array_equal(wts[:64].cpu().numpy(), rw)


@pytest.mark.parametrize("T,E,topk", [(64, 288, 8), (5, 32, 4), (3, 1024, 32), (8193, 288, 8), (7, 320, 8),
                                      (6, 321, 8), (2, 1, 1)])
def test_router_topk_bit_exact(cuda, T, E, topk):
    from mi355moe import ops
    _say(f"router_topk T={T} E={E} topk={topk}")
    g = torch.Generator().manual_seed(T + E)
    lg = torch.randn(T, E, generator=g) * 2
    b = torch.randn(E, generator=g) * 0.01
    if E > 9:
        lg[0, 7] = lg[0, 9]
        b[7] = b[9]                               # an exact tie
    ids, w = ops.router_topk(lg.to(cuda), topk, b.to(cuda), routed_scale=2.5)
    rid, rw = routing.topk_sigmoid_bias(lg.numpy(), b.numpy(), topk, 2.5)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(w.cpu().numpy(), rw)


@pytest.mark.parametrize("T,topk,n,seg,ids64,emap", [(8, 8, 288, 8, False, False), (1, 8, 288, 1, True, False),
                                                     (64, 8, 288, 16, False, True), (2048, 8, 288, 256, False, False),
                                                     (8192, 8, 288, 256, True, False), (130, 8, 64, 16, True, True),
                                                     (2048, 8, 4000, 64, False, False),
                                                     # per-block placement by ballots up to 1024 ids, the scan beyond
                                                     (2048, 8, 1023, 64, False, False), (2048, 8, 1024, 64, False, False),
                                                     # few ids: long runs of one id inside every wave and block
                                                     (1024, 8, 3, 256, False, False)])
def test_route_bit_exact(cuda, T, topk, n, seg, ids64, emap):
    from mi355moe import ops
    _say(f"route T={T} topk={topk} n={n} seg={seg}")
    g = torch.Generator().manual_seed(T + n)
    ids = torch.randint(-1, n + 2, (T, topk), generator=g)
    ids = ids.to(torch.int64 if ids64 else torch.int32)
    w = torch.rand(T, topk, generator=g)
    em = None
    if emap:
        em = torch.randint(-1, n, (n + 2,), generator=g, dtype=torch.int64)
    r = ops.route(ids.to(cuda), w.to(cuda), n, R=1 << 30, seg_rows=seg, expert_map=None if em is None else em.to(cuda))
    local = routing.map_topk_to_local(ids.numpy(), n, None if em is None else em.numpy())
    o = routing.permutation(local, n, topk, 1 << 30, seg)
    P = T * topk
    assert np.array_equal(r["inv"].cpu().numpy(), o["inv"])
    assert np.array_equal(r["tok"].cpu().numpy(), o["token"])
    assert np.array_equal(r["pe"].cpu().numpy(), o["pair_expert"])
    assert np.array_equal(r["counts"].cpu().numpy(), o["counts"])
    ns = int(r["nseg"].item())
    assert ns == len(o["seg_expert"])
    assert np.array_equal(r["seg_expert"][:ns].cpu().numpy(), o["seg_expert"])
    assert np.array_equal(r["seg_row0"][:ns].cpu().numpy(), o["seg_row0"])
    assert np.array_equal(r["seg_rows"][:ns].cpu().numpy(), o["seg_rows"])
    w16 = w.numpy().reshape(-1).astype(np.float16)[o["order"]]
    assert np.array_equal(r["w16"].cpu().numpy().view(np.uint16), w16.view(np.uint16))
    assert P == o["order"].size
