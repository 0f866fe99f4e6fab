"""The e4m3 expert variant: block-scaled e4m3 routed experts (vLLM's fp8 w8a8 block-quantised MoE layout, 128x128
blocks) with per-token dynamic e4m3 activations; exact products on gfx950's fp16 matrix cores, fp32 block sums.

  Fp8Experts          one layer's experts: w13 e4m3 [n, 2I, H] (gate rows then up rows), w13_scale fp32
                      [n, 2I/128, H/128], w2 e4m3 [n, H, I], w2_scale fp32 [n, H/128, I/128]
  quant_rows          per-row dynamic e4m3 quantisation (code/fork/kernels/moe_e4m3.cu:152-176)
  moe_forward_ids     routed output from router ids / weights (code/fork/overlay/glm53_moe_e4m3.py:484-592)
  fused_experts_fp8   the functional form apply(hidden, w13, w2, topk_weights, topk_ids, scales)
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .ops import _need_cuda, _p, _stream, ids_dtype_code, weight_dtype_code, workspace

E4M3_MAX = 448.0


def _as_u8(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    if t.dtype != torch.uint8:
        raise ValueError(f"e4m3 weights must be torch.float8_e4m3fn or uint8 codes, got {t.dtype}")
    return t


class Fp8Experts:
    """A layer's block-scaled e4m3 experts plus the C descriptor (the tensors stay owned by the caller)."""

    def __init__(self, w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor, w2_scale: torch.Tensor):
        w13, w2 = _as_u8(w13), _as_u8(w2)
        n, I2, H = w13.shape
        I = I2 // 2
        exp = {"w13": (w13, (n, 2 * I, H)), "w2": (w2, (n, H, I)),
               "w13_scale": (w13_scale, (n, 2 * I // 128, H // 128)), "w2_scale": (w2_scale, (n, H // 128, I // 128))}
        if I2 % 2 or H % 256 or I % 128:
            raise ValueError(f"w13 must be [n, 2I, H] with H % 256 == 0 and I % 128 == 0, got {tuple(w13.shape)}")
        for name, (t, shape) in exp.items():
            if tuple(t.shape) != shape:
                raise ValueError(f"{name}: expected {shape}, got {tuple(t.shape)}")
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
            if t.device != w13.device:
                raise ValueError(f"{name} is on {t.device}, w13 on {w13.device}")
        for name in ("w13_scale", "w2_scale"):
            if exp[name][0].dtype != torch.float32:
                raise ValueError(f"{name} must be float32")
        self.w13, self.w13_scale, self.w2, self.w2_scale = w13, w13_scale, w2, w2_scale
        self.n, self.K, self.N = n, H, I
        d = _lib.Fp8LayerDesc()
        d.n, d.hidden, d.intermediate = n, H, I
        d.w13, d.w13_scale = ctypes.c_void_p(w13.data_ptr()), ctypes.c_void_p(w13_scale.data_ptr())
        d.w2, d.w2_scale = ctypes.c_void_p(w2.data_ptr()), ctypes.c_void_p(w2_scale.data_ptr())
        self.desc = d

    @property
    def device(self) -> torch.device:
        return self.w13.device

    def expert_bytes(self) -> int:
        """Bytes of one expert's three matrices and their block scales."""
        return 3 * self.K * self.N + 4 * 3 * (self.K // 128) * (self.N // 128)


def _act_code(dt: torch.dtype) -> int:
    return weight_dtype_code(dt)


def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(q uint8 [rows, K] e4m3 codes, s float32 [rows]) with s = amax / 448 (1 if 0), q = e4m3(clamp(x / s))."""
    dev = _need_cuda(x)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [rows, K] with unit column stride")
    rows, K = x.shape
    q = torch.empty(rows, K, dtype=torch.uint8, device=dev)
    s = torch.empty(rows, dtype=torch.float32, device=dev)
    _lib.check("mi355moe_fp8_quant_rows", _lib.lib().mi355moe_fp8_quant_rows(
        _p(x), _act_code(x.dtype), rows, K, x.stride(0), _p(q), _p(s), _stream(dev)))
    return q, s


def moe_forward_ids(experts: Fp8Experts, x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                    limit: float = 10.0, expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None, stages: int = _lib.STAGE_ALL) -> torch.Tensor:
    """Routed-expert output [T, H] in x's dtype (unless out / out_dtype say otherwise), written (not accumulated).
    x: fp32, fp16 or bf16 [T, H]; topk_ids int32/int64 [T, k] (global ids; expert_map maps them to local ids or -1);
    topk_weights [T, k] (already scaled by the router). stages: a subset of the launches (_lib.STAGE_*)."""
    dev = _need_cuda(x, topk_ids, topk_weights, expert_map)
    if dev != experts.device:
        raise ValueError(f"activations on {dev}, experts on {experts.device}")
    if x.dim() != 2 or x.shape[1] != experts.K or x.stride(1) != 1:
        raise ValueError(f"x must be [T, {experts.K}] with unit column stride")
    T = x.shape[0]
    ids = topk_ids.reshape(T, -1).contiguous()
    w = topk_weights.reshape(T, -1).contiguous()
    topk = ids.shape[1]
    if w.shape != ids.shape:
        raise ValueError("topk_weights must be shaped like topk_ids")
    if out is None:
        out = torch.empty(T, experts.K, dtype=out_dtype or x.dtype, device=dev)
    if out.shape != (T, experts.K) or out.stride(1) != 1:
        raise ValueError("out must be [T, H] with unit column stride")
    L = _lib.lib()
    nb = L.mi355moe_fp8_moe_workspace_bytes(ctypes.byref(experts.desc), T, topk)
    if nb < 0:
        raise ValueError("mi355moe_fp8_moe_workspace_bytes rejected the shape")
    ws = workspace(dev, nb)
    em = None if expert_map is None else expert_map.to(torch.int64).contiguous()
    _lib.check("mi355moe_fp8_moe_forward_ids", L.mi355moe_fp8_moe_forward_ids(
        ctypes.byref(experts.desc), _p(x), _act_code(x.dtype), x.stride(0), T, _p(ids), ids_dtype_code(ids.dtype),
        _p(w), weight_dtype_code(w.dtype), topk, _p(em), 0 if em is None else em.numel(), float(limit), _p(out),
        weight_dtype_code(out.dtype), out.stride(0), _p(ws), ws.numel(), int(stages), _stream(dev)))
    return out


_FUSED_CACHE: dict = {}


def fused_experts_fp8(hidden: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, topk_weights: torch.Tensor,
                      topk_ids: torch.Tensor, scales: tuple, *, limit: float = 10.0,
                      expert_map: torch.Tensor | None = None) -> torch.Tensor:
    """apply(hidden, w13, w2, topk_weights, topk_ids, scales) for block-scaled e4m3 experts: scales =
    (w13_scale, w2_scale) (vLLM's w1_scale / w2_scale with block_shape [128, 128]). The descriptor is cached per
    weight tensor."""
    w13_scale, w2_scale = scales
    key = (w13.data_ptr(), w2.data_ptr(), w13_scale.data_ptr(), w2_scale.data_ptr())
    ex = _FUSED_CACHE.get(key)
    if ex is None:
        ex = Fp8Experts(w13, w13_scale, w2, w2_scale)
        _FUSED_CACHE[key] = ex
    T = hidden.shape[0]
    return moe_forward_ids(ex, hidden, topk_ids.reshape(T, -1), topk_weights.reshape(T, -1), limit=limit,
                           expert_map=expert_map, out_dtype=hidden.dtype)
