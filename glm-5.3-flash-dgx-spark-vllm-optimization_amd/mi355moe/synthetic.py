"""Synthetic layers and routings of the benchmark configurations (no checkpoints are available offline).

EXL3 experts: uniform random int16 trellis words per 16x16 tile, suh = random +-1 (Hadamard signs), svh = random
sign x |N(0,1)| x svh_scale, all fp16 (the decode MoE layer configuration: K=4096, N=1024, 288 experts).
Router: W ~ N(0, 0.02) bf16 [E, K], bias ~ N(0, 0.01) fp32, x ~ N(0, 1) bf16; draw order router weights, expert
weights, activations, each from its own seeded generator.
"""
from __future__ import annotations

import math

import torch

from .layer import Exl3Experts


def _gen(seed: int, device: torch.device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _signs(shape, g, device) -> torch.Tensor:
    return (torch.randint(0, 2, shape, generator=g, device=device, dtype=torch.int32) * 2 - 1).to(torch.float32)


def exl3_layer(n: int, K: int, N: int, seed: int, device="cuda", svh_scale: float = 0.01,
               svh_d_scale: float | None = None, shared_suh: bool = True) -> Exl3Experts:
    """One layer of n random EXL3 4-bit experts in production's stacked layout. shared_suh: gate and up share
    one input rotation, as production's checkpoints do (its grouped prefill tier requires it,
    code/fork/docs/prod_exl3_reference.py:376)."""
    device = torch.device(device)
    g = _gen(seed, device)
    w13_trellis = torch.randint(-32768, 32768, (n, 2, K // 16, N // 16, 64), generator=g, device=device,
                                dtype=torch.int32).to(torch.int16)
    w13_suh = _signs((n, 2, K), g, device).to(torch.float16)
    if shared_suh:
        w13_suh[:, 1].copy_(w13_suh[:, 0])
    w13_svh = (_signs((n, 2, N), g, device) * torch.randn((n, 2, N), generator=g, device=device).abs()
               * svh_scale).to(torch.float16)
    w2_trellis = torch.randint(-32768, 32768, (n, N // 16, K // 16, 64), generator=g, device=device,
                               dtype=torch.int32).to(torch.int16)
    w2_suh = _signs((n, N), g, device).to(torch.float16)
    sd = svh_scale if svh_d_scale is None else svh_d_scale
    w2_svh = (_signs((n, K), g, device) * torch.randn((n, K), generator=g, device=device).abs() * sd).to(
        torch.float16)
    return Exl3Experts(w13_trellis, w13_suh, w13_svh, w2_trellis, w2_suh, w2_svh)


def block_quant_e4m3(w: torch.Tensor, block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """e4m3 codes (uint8) and fp32 scales of float32 matrices [..., R, C] with one scale per block x block tile:
    s = amax(tile) / 448 (1 if 0), codes = e4m3(clamp(w / s, -448, 448))."""
    *lead, R, C = w.shape
    wb = w.reshape(*lead, R // block, block, C // block, block)
    s = wb.abs().amax(dim=(-3, -1)) / 448.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = (wb / s[..., :, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(w.shape), s.to(torch.float32).contiguous()


def fp8_layer(n: int, K: int, N: int, seed: int, device="cuda", std: float = 0.02):
    """One layer of n block-scaled e4m3 experts (the e4m3 expert configuration): weights N(0, std), quantised per
    128x128 block (fp32 scale = block amax / 448). Returns mi355moe.fp8.Fp8Experts."""
    from .fp8 import Fp8Experts
    device = torch.device(device)
    g = _gen(seed, device)
    w13 = torch.empty(n, 2 * N, K, dtype=torch.uint8, device=device)
    w2 = torch.empty(n, K, N, dtype=torch.uint8, device=device)
    s13 = torch.empty(n, 2 * N // 128, K // 128, dtype=torch.float32, device=device)
    s2 = torch.empty(n, K // 128, N // 128, dtype=torch.float32, device=device)
    step = max(1, min(n, 16))
    for e0 in range(0, n, step):
        e1 = min(n, e0 + step)
        q, s = block_quant_e4m3(torch.randn(e1 - e0, 2 * N, K, generator=g, device=device) * std)
        w13[e0:e1].copy_(q)
        s13[e0:e1].copy_(s)
        q, s = block_quant_e4m3(torch.randn(e1 - e0, K, N, generator=g, device=device) * std)
        w2[e0:e1].copy_(q)
        s2[e0:e1].copy_(s)
    return Fp8Experts(w13, s13, w2, s2)


def router(E: int, K: int, seed: int, device="cuda") -> tuple[torch.Tensor, torch.Tensor]:
    """(W bf16 [E, K] ~ N(0, 0.02), e_score_correction_bias fp32 [E] ~ N(0, 0.01))."""
    device = torch.device(device)
    g = _gen(seed, device)
    w = (torch.randn((E, K), generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = torch.randn((E,), generator=g, device=device) * 0.01
    return w, b


def activations(T: int, K: int, seed: int, device="cuda", dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(seed, torch.device(device))
    return torch.randn((T, K), generator=g, device=device).to(dtype)


def random_ids(T: int, n: int, topk: int, seed: int, device="cuda") -> torch.Tensor:
    """Independent top-k per token: topk distinct experts chosen uniformly (int32 [T, topk])."""
    g = _gen(seed, torch.device("cpu"))
    ids = torch.stack([torch.randperm(n, generator=g)[:topk] for _ in range(T)]) if T else torch.zeros(0, topk)
    return ids.to(torch.int32).to(device)


def softmax_weights(T: int, topk: int, seed: int, device="cuda", scale: float = 2.5) -> torch.Tensor:
    g = _gen(seed, torch.device("cpu"))
    return (torch.softmax(torch.randn(T, topk, generator=g), -1) * scale).to(device)


def zipf_logits(T: int, E: int, seed: int, s: float = 1.2, noise: torch.Tensor | None = None,
                device="cuda") -> torch.Tensor:
    """Router logits skewed by Zipf(s) popularity: logit_e = -s * ln(rank_e + 1) over a random permutation of the
    experts, plus optional per-token noise [T, E]."""
    g = _gen(seed, torch.device("cpu"))
    rank = torch.randperm(E, generator=g).float()
    base = -s * torch.log(rank + 1.0)
    lg = base.unsqueeze(0).expand(T, E).clone().to(device)
    if noise is not None:
        lg = lg + noise
    return lg


def expected_distinct(n: int, topk: int, T: int) -> float:
    """E[#distinct experts] when T tokens each pick topk distinct experts uniformly."""
    return n * (1.0 - math.prod((n - topk) / n for _ in range(T)))
