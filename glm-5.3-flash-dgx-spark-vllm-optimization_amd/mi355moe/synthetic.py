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
               svh_d_scale: float | None = None, shared_suh: bool = True,
               uniform_suh: bool = False) -> Exl3Experts:
    """One layer of n random EXL3 4-bit experts in production's stacked layout. shared_suh: gate and up share
    one input rotation, as production's checkpoints do (its grouped prefill tier requires it,
    code/fork/docs/prod_exl3_reference.py:376). uniform_suh: every expert the same w13 suh too, as in the real
    checkpoints' layers (code/fork/docs/OPT_MOE.md:14)."""
    device = torch.device(device)
    g = _gen(seed, device)
    w13_trellis = torch.randint(-32768, 32768, (n, 2, K // 16, N // 16, 64), generator=g, device=device,
                                dtype=torch.int32).to(torch.int16)
    w13_suh = _signs((n, 2, K), g, device).to(torch.float16)
    if uniform_suh:
        w13_suh.copy_(w13_suh[:1, :1].clone().expand(n, 2, K))
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


def codebook_std() -> float:
    """Standard deviation of the 4-bit mcg codebook over all 65,536 states (uniform random trellis words give
    uniform states): x = s * 0xCBAC1FED mod 2^32, (x & 0x8FFF8FFF) ^ 0x3B603B60, fp16(lo) + fp16(hi)."""
    s = torch.arange(65536, dtype=torch.int64)
    x = ((s * 0xCBAC1FED) & 0xFFFFFFFF & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (x & 0xFFFF).to(torch.int32).to(torch.int16).view(torch.float16)
    hi = (x >> 16).to(torch.int32).to(torch.int16).view(torch.float16)
    return float((lo + hi).double().std())


def _scaled_signs(shape, scale, g, device) -> torch.Tensor:
    """fp16 of random sign x (1 + 0.25 U(-1, 1)) x scale."""
    mag = 1.0 + 0.25 * (torch.rand(shape, generator=g, device=device) * 2 - 1)
    return (_signs(shape, g, device) * mag * scale).to(torch.float16)


def calibrated_layer(n: int, K: int, N: int, seed: int, device="cuda", g_std: float = 5.0, svh_d: float = 0.001,
                     shared_suh: bool = True, uniform_suh: bool = False) -> Exl3Experts:
    """n random EXL3 4-bit experts with scales calibrated as the reference's test harness does
    (code/fork/tests/harness.py:178-200): suh, svh and down suh are random signs x (1 +- 25 %) x a scale, the gate/up
    svh scale chosen so that the gate and up pre-activations have standard deviation g_std for x ~ N(0, 1)
    (std(g) = sqrt(K) * codebook std * E|suh| * E|svh|); with g_std = 5 and the SwiGLU limit 10 about 5 % of the
    gate values are clamped. Down suh ~ 8 / sqrt(N) as there; the down svh scale (svh_d; the reference uses 1.0, which
    gives routed outputs of RMS ~200) is 0.001 by default, for routed outputs of RMS ~0.2. uniform_suh: every expert
    the same w13 suh (as in the real checkpoints' layers)."""
    device = torch.device(device)
    g = _gen(seed, device)
    mag_rms = math.sqrt(1 + 0.25 ** 2 / 3)
    s_svh = g_std / (math.sqrt(K) * codebook_std() * mag_rms * mag_rms)
    w13_trellis = torch.randint(-32768, 32768, (n, 2, K // 16, N // 16, 64), generator=g, device=device,
                                dtype=torch.int32).to(torch.int16)
    w13_suh = _scaled_signs((n, 2, K), 1.0, g, device)
    if uniform_suh:
        w13_suh.copy_(w13_suh[:1, :1].clone().expand(n, 2, K))
    if shared_suh:
        w13_suh[:, 1].copy_(w13_suh[:, 0])
    w13_svh = _scaled_signs((n, 2, N), s_svh, g, device)
    w2_trellis = torch.randint(-32768, 32768, (n, N // 16, K // 16, 64), generator=g, device=device,
                               dtype=torch.int32).to(torch.int16)
    w2_suh = _scaled_signs((n, N), 8.0 / math.sqrt(N), g, device)
    w2_svh = _scaled_signs((n, K), svh_d, g, device)
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


def zipf_ids(T: int, n: int, topk: int, seed: int, s: float = 1.2, device="cuda") -> torch.Tensor:
    """Top-k picks with Zipf(s)-skewed expert popularity: every token draws topk distinct experts with probability
    proportional to 1 / (rank + 1)^s over a random ranking of the experts (int32 [T, topk])."""
    g = _gen(seed, torch.device("cpu"))
    p = 1.0 / (torch.arange(n, dtype=torch.float64) + 1.0) ** s
    probs = torch.empty(n, dtype=torch.float64)
    probs[torch.randperm(n, generator=g)] = p
    ids = torch.multinomial(probs.expand(T, n), topk, replacement=False, generator=g) if T else torch.zeros(0, topk)
    return ids.to(torch.int32).to(device)


def zipf_router(E: int, K: int, seed: int, rank_seed: int, device="cuda", s: float = 1.2,
                c0: float = 8.0) -> tuple[torch.Tensor, torch.Tensor]:
    """A router (W, bias) whose GEMM itself produces Zipf(s)-skewed expert popularity: column 0 of W is
    -s ln(rank_e + 1) / c0 over a random ranking of the experts, so for activations whose channel 0 holds c0
    (zipf_activations) logit_e = x.W_e - s ln(rank_e + 1) plus the N(0, 0.02) weights' noise."""
    w, b = router(E, K, seed, device=device)
    g = _gen(rank_seed, torch.device("cpu"))
    rank = torch.empty(E, dtype=torch.float32)
    rank[torch.randperm(E, generator=g)] = torch.arange(E, dtype=torch.float32)
    w[:, 0] = (-s * torch.log(rank + 1.0) / c0).to(w.device, torch.bfloat16)
    return w, b


def zipf_activations(T: int, K: int, seed: int, device="cuda", c0: float = 8.0) -> torch.Tensor:
    """bf16 x ~ N(0, 1) [T, K] with channel 0 held at c0 (the channel zipf_router's skew column reads)."""
    x = activations(T, K, seed, device=device)
    x[:, 0] = c0
    return x


def expected_distinct(n: int, topk: int, T: int) -> float:
    """E[#distinct experts] when T tokens each pick topk distinct experts uniformly."""
    return n * (1.0 - math.prod((n - topk) / n for _ in range(T)))
