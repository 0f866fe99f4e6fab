"""The reference's call contracts for the routed-MoE path, backed by libmi355moe.so.

  Exl3MoEMethod        vLLM FusedMoE quant method shape: create_weights / process_weights_after_loading / apply
                       (code/fork/docs/prod_exl3_reference.py:2048-2343)
  apply_exl3_experts   the shipped routed-expert apply (prod_exl3_reference.py:1788-1823): x [T, K], topk ids and
                       weights -> routed output in x's dtype
  fused_experts        functional form apply(hidden, w13, w2, topk_weights, topk_ids, scales)
  exl3_moe             exllamav3_ext.exl3_moe's 29 positional arguments (code/fork/docs/ref/xl_exl3_moe.cu:93-130,
                       caller prod_exl3_reference.py:1490-1537): out (fp32) is accumulated into

Errors raise (ValueError for contract violations found on the host, _lib.MoeError for a rejected or failed call);
there is no silent fallback to another implementation.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, ops
from .layer import MCG_MARKER, Exl3Experts, tables_desc

SWIGLU_LIMIT_DEFAULT = 10.0      # prod_exl3_reference.py:53


def _experts_of(layer: torch.nn.Module) -> Exl3Experts:
    ex = getattr(layer, "_mi355_experts", None)
    if ex is None:
        raise RuntimeError("EXL3 experts were not built after weight load (process_weights_after_loading)")
    return ex


def apply_exl3_experts(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       layer: torch.nn.Module, *, limit: float = SWIGLU_LIMIT_DEFAULT, e4m3: bool = False) -> torch.Tensor:
    """Routed-expert output [.., T, K] in x's dtype (prod_exl3_reference.py:1788-1823). topk_ids are global ids;
    layer.expert_map (optional, global -> local or -1) selects this rank's experts. e4m3: the trellis-sourced e4m3
    numerics (code/fork/overlay/glm53_moe_e4m3.py:484-592 run() in place of the fp16 paths)."""
    experts = _experts_of(layer)
    tokens, hidden = x.shape[-2], x.shape[-1]
    x2d = x.reshape(tokens, hidden)
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    ids = topk_ids.reshape(tokens, -1)
    w = topk_weights.reshape(tokens, -1)
    emap = getattr(layer, "expert_map", None)
    fwd = ops.moe_forward_ids_e4m3 if e4m3 else ops.moe_forward_ids
    out = fwd(experts, x2d, ids, w, limit=limit, expert_map=emap, out_dtype=x.dtype)
    return out.reshape(x.shape)


def _fused_key(ts) -> tuple:
    """Identity of the weight tensors for the descriptor cache: storage address, shape, strides, dtype, device and
    torch's version counter (bumped by every in-place write, so a reload through copy_ builds a new descriptor)."""
    return tuple((t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, str(t.device), t._version) for t in ts)


def fused_experts(hidden: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, topk_weights: torch.Tensor,
                  topk_ids: torch.Tensor, scales: tuple, *, limit: float = SWIGLU_LIMIT_DEFAULT,
                  expert_map: torch.Tensor | None = None) -> torch.Tensor:
    """apply(hidden, w13, w2, topk_weights, topk_ids, scales): w13 = w13_trellis [n, 2, K/16, N/16, 64],
    w2 = w2_trellis [n, N/16, K/16, 64], scales = (w13_suh, w13_svh, w2_suh, w2_svh). The experts object (pointer
    tables, shared-suh flag) is cached per weight tensors (address, shape, strides, dtype, version), at most
    _FUSED_CACHE_MAX layers, least recently used dropped first; weights rewritten in a way that does not move the
    passed tensor's version counter (through .data, or outside torch) need clear_fused_cache()."""
    w13_suh, w13_svh, w2_suh, w2_svh = scales
    key = _fused_key((w13, w2, w13_suh, w13_svh, w2_suh, w2_svh))
    ex = _FUSED_CACHE.pop(key, None)
    if ex is None:
        ex = Exl3Experts(w13, w13_suh, w13_svh, w2, w2_suh, w2_svh)
    _FUSED_CACHE[key] = ex                        # most recently used last
    while len(_FUSED_CACHE) > _FUSED_CACHE_MAX:
        _FUSED_CACHE.pop(next(iter(_FUSED_CACHE)))
    T = hidden.shape[0]
    return ops.moe_forward_ids(ex, hidden, topk_ids.reshape(T, -1), topk_weights.reshape(T, -1), limit=limit,
                               expert_map=expert_map, out_dtype=hidden.dtype)


_FUSED_CACHE: dict = {}
_FUSED_CACHE_MAX = 128            # layers; a served model has one entry per MoE layer


def clear_fused_cache() -> None:
    """Drop every cached experts object of fused_experts (and the references it holds to weight tensors)."""
    _FUSED_CACHE.clear()


class Exl3MoEMethod:
    """FusedMoE quant method for EXL3 4-bit trellis routed experts (prod_exl3_reference.py:2030-2343)."""

    def __init__(self, bits: int = 4, swiglu_limit: float | None = None, e4m3: bool = False,
                 max_num_tokens: int | None = None, topk: int = 8, tp_rank: int = 0, tp_size: int = 1):
        if bits != 4:
            raise ValueError("only 4-bit EXL3 trellis tiles are supported")
        self.bits = bits
        self.swiglu_limit = swiglu_limit
        self.e4m3 = e4m3                  # the overlay's e4m3 expert numerics instead of the fp16 paths
        # with max_num_tokens the device workspace is sized once after weight load for every call up to that many
        # tokens (top-k picks each), so later calls never reallocate it (the reference's Scratch, sized at
        # registration, code/fork/tf_exl3_moe.py:391-418)
        self.max_num_tokens = max_num_tokens
        self.topk = topk
        self.tp_rank, self.tp_size = tp_rank, tp_size    # this rank's slice of N (gate/up columns, down rows)

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype=None, device=None, **_) -> None:
        if hidden_size % 16 or intermediate_size_per_partition % 16:
            raise ValueError("EXL3 trellis tiles are 16-wide; "
                             f"hidden={hidden_size} intermediate_local={intermediate_size_per_partition}")
        n, K, N = num_experts, hidden_size, intermediate_size_per_partition
        kw = dict(device=device)
        P = torch.nn.Parameter
        shapes = {
            "w13_trellis": ((n, 2, K // 16, N // 16, 16 * self.bits), torch.int16),
            "w13_suh": ((n, 2, K), torch.float16), "w13_svh": ((n, 2, N), torch.float16),
            "w13_mcg": ((n, 2, 1), torch.int32),
            "w2_trellis": ((n, N // 16, K // 16, 16 * self.bits), torch.int16),
            "w2_suh": ((n, N), torch.float16), "w2_svh": ((n, K), torch.float16), "w2_mcg": ((n, 1), torch.int32),
        }
        for name, (shape, dt) in shapes.items():
            param = P(torch.empty(shape, dtype=dt, **kw), requires_grad=False)
            layer.register_parameter(name, param)
            param.weight_loader = self.weight_loader
            param._mi355_owner = layer
        layer._exl3_hidden_size = K
        layer._exl3_intermediate_local = N
        layer._exl3_bits = self.bits

    def weight_loader(self, param: torch.nn.Parameter, loaded_weight: torch.Tensor, weight_name: str,
                      shard_id: str = "w1", expert_id: int = 0, return_success: bool = False):
        """One checkpoint tensor of one expert (global id) into the stacked parameters, sliced for this rank
        (prod_exl3_reference.py:2164-2221): shard_id w1 / w3 = gate / up (column slice), w2 = down (row slice).
        Non-local experts (layer.expert_map, global -> local or -1) are skipped."""
        from .loader import load_into
        layer = param._mi355_owner
        ok = load_into(layer, loaded_weight, weight_name, shard_id, expert_id, self.tp_rank, self.tp_size,
                       getattr(layer, "expert_map", None))
        return ok if return_success else None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        for name in ("w13_mcg", "w2_mcg"):
            m = getattr(layer, name, None)
            if m is not None and not bool(torch.all(m == MCG_MARKER)):
                raise RuntimeError(f"{name}: every entry must be the mcg codebook marker {MCG_MARKER} (0xCBAC1FED "
                                   "as int32); these weights use another trellis codebook")
        layer._mi355_experts = Exl3Experts.from_module(layer)
        if self.max_num_tokens:
            ops.reserve(layer._mi355_experts, self.max_num_tokens, self.topk)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              shared_experts=None, shared_experts_input=None) -> torch.Tensor:
        del shared_experts, shared_experts_input
        limit = self.swiglu_limit or SWIGLU_LIMIT_DEFAULT
        return apply_exl3_experts(x, topk_ids, topk_weights, layer, limit=float(limit), e4m3=self.e4m3)


def exl3_moe(hidden, out, expert_count, token_sorted, weight_sorted, temp_state_g, temp_state_u,
             temp_intermediate_g, temp_intermediate_u, act_function, K_gate, K_up, K_down, gate_trellis_ptrs,
             gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs,
             down_suh_ptrs, down_svh_ptrs, gate_mcg, gate_mul1, up_mcg, up_mul1, down_mcg, down_mul1, act_limit,
             num_active=None):
    """exllamav3_ext.exl3_moe (arg0..arg28 [, arg29 num_active]): out += routed output of the pre-sorted pairs.
    The temps are not written (they only set R = temp_state_g.size(1), the most rows an expert may have)."""
    del num_active, temp_state_u, temp_intermediate_u
    for t, name, dt in ((hidden, "hidden", torch.float16), (out, "out", torch.float32),
                        (expert_count, "expert_count", torch.int64), (token_sorted, "token_sorted", torch.int64),
                        (weight_sorted, "weight_sorted", torch.float16)):
        if t.dtype != dt or not t.is_contiguous() or not t.is_cuda:
            raise ValueError(f"exl3_moe: {name} must be a contiguous CUDA {dt} tensor")
    if hidden.dim() != 2 or out.shape != hidden.shape:
        raise ValueError("exl3_moe: hidden fp16 [B, K] and out fp32 [B, K]")
    B, K = hidden.shape
    n = expert_count.numel() - 1
    N = temp_intermediate_g.shape[-1]
    R = temp_state_g.shape[1]
    P = token_sorted.numel()
    if weight_sorted.numel() != P:
        raise ValueError("exl3_moe: token_sorted and weight_sorted differ in length")
    tabs = {"gate_trellis": gate_trellis_ptrs, "gate_suh": gate_suh_ptrs, "gate_svh": gate_svh_ptrs,
            "up_trellis": up_trellis_ptrs, "up_suh": up_suh_ptrs, "up_svh": up_svh_ptrs,
            "down_trellis": down_trellis_ptrs, "down_suh": down_suh_ptrs, "down_svh": down_svh_ptrs}
    desc = tables_desc(n, K, N, tabs)
    L = _lib.lib()
    nb = L.mi355moe_exl3_moe_workspace_bytes(ctypes.byref(desc), P)
    if nb < 0:
        raise ValueError("exl3_moe: unsupported shape")
    dev = hidden.device
    ws = ops.workspace(dev, nb)
    _lib.check("mi355moe_exl3_moe", L.mi355moe_exl3_moe(
        ctypes.byref(desc), ops._p(hidden), B, ops._p(out), ops._p(expert_count), ops._p(token_sorted),
        ops._p(weight_sorted), P, R, int(act_function), int(K_gate), int(K_up), int(K_down), int(bool(gate_mcg)),
        int(bool(gate_mul1)), int(bool(up_mcg)), int(bool(up_mul1)), int(bool(down_mcg)), int(bool(down_mul1)),
        float(act_limit), ops._p(ws), ws.numel(), ops._stream(dev)))
