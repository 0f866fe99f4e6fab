"""Torch-level wrappers of the C ABI (device tensors in, device tensors out, current stream).

Every function validates its tensors on the host, then calls one C entry point, which checks its arguments again
before enqueuing anything. No function synchronizes with the host or allocates per call except for its outputs
(the persistent workspace is allocated once per device, reserved up front with `reserve`, or replaced by a larger one
when a call outgrows it; a replaced workspace is kept alive for the graphs captured on it).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .layer import Exl3Experts

_WS: dict = {}           # device -> the workspace calls use
_RETIRED: dict = {}      # device -> superseded workspaces, kept alive for graphs captured on them


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _need_cuda(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("mi355moe: every tensor must be on the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"mi355moe: tensors on {t.device} and {dev}")
    return dev


def act_dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float16:
        return _lib.F16
    if dt == torch.bfloat16:
        return _lib.BF16
    raise ValueError(f"activations must be fp16 or bf16, got {dt}")


def weight_dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return _lib.F32
    return act_dtype_code(dt)


def ids_dtype_code(dt: torch.dtype) -> int:
    if dt == torch.int32:
        return _lib.I32
    if dt == torch.int64:
        return _lib.I64
    raise ValueError(f"router ids must be int32 or int64, got {dt}")


def _capturing(dev: torch.device) -> bool:
    """True while the current stream of a GPU device is being captured into a graph."""
    return dev.type == "cuda" and torch.cuda.is_current_stream_capturing()


def workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The persistent zero-initialised workspace of `dev`, at least `nbytes`. Calls keep its counters at zero; calls
    that share it must be stream-ordered.

    When a call needs more than the current workspace, a larger one replaces it for later calls and the old one is
    retired but never freed: a HIP graph captured earlier keeps replaying into the memory it captured, which no other
    tensor can be given. Growing during a graph capture raises instead (the capture would record the new buffer's
    zero fill); size the workspace beforehand with reserve_workspace / reserve, or by one eager call of the largest
    shape."""
    key = (dev.type, dev.index)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if _capturing(dev):
            have = 0 if ws is None else ws.numel()
            raise RuntimeError(f"mi355moe: this call needs a {int(nbytes)}-byte workspace on {dev} but {have} bytes "
                               "are reserved, and it cannot grow during graph capture; call "
                               "mi355moe.ops.reserve(...) or run one eager call of this shape before capturing")
        if ws is not None:
            _RETIRED.setdefault(key, []).append(ws)
        ws = torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def reserve_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Size the workspace of `dev` to at least `nbytes` now (at load time, before any capture)."""
    return workspace(torch.device(dev), int(nbytes))


def workspace_bytes(experts: Exl3Experts, tokens: int, topk: int = 8, router_experts: int | None = None) -> int:
    """The largest workspace any entry point of this module needs for calls of up to `tokens` tokens over `experts`
    (decode and grouped tiers, the trellis-sourced e4m3 variant, and with router_experts the whole-layer call)."""
    L = _lib.lib()
    d = ctypes.byref(experts.desc)
    need = 0
    for path in (_lib.PATH_AUTO, _lib.PATH_DECODE, _lib.PATH_PREFILL):
        if path == _lib.PATH_PREFILL and not experts.shared_suh:
            continue
        need = max(need, L.mi355moe_moe_workspace_bytes_path(d, tokens, topk, path))
    if experts.shared_suh and experts.K <= 4096:
        need = max(need, L.mi355moe_e4m3_moe_workspace_bytes(d, tokens, topk))
    if router_experts is not None:
        need = max(need, L.mi355moe_moe_layer_workspace_bytes(d, tokens, topk, router_experts))
    if need < 0:
        raise ValueError("mi355moe: the workspace size query rejected the shape")
    return int(need)


def reserve(experts: Exl3Experts, max_tokens: int, topk: int = 8, router_experts: int | None = None) -> torch.Tensor:
    """Reserve the workspace for every call of up to max_tokens tokens over `experts` once, as the reference sizes
    its persistent scratch at registration (code/fork/tf_exl3_moe.py:391-418): later calls within that size never
    reallocate, so graphs may be captured at any point after this."""
    top = max(1, int(max_tokens))
    # every size: the decode plan's split-K partials come and go with T (they exist only while the segments are too
    # few to fill the chip), so the need is not monotone in T
    return workspace(experts.device, max(workspace_bytes(experts, t, topk, router_experts) for t in range(1, top + 1)))


def dequant(trellis: torch.Tensor) -> torch.Tensor:
    """W_q fp16 [K, N] from a 4-bit trellis int16 [K/16, N/16, 64] (exl3_format_ref.py:88-97)."""
    dev = _need_cuda(trellis)
    if trellis.dtype != torch.int16 or trellis.dim() != 3 or trellis.shape[-1] != 64:
        raise ValueError("trellis must be int16 [K/16, N/16, 64]")
    t = trellis.contiguous()
    kt, nt = t.shape[0], t.shape[1]
    out = torch.empty(kt * 16, nt * 16, dtype=torch.float16, device=dev)
    _lib.check("mi355moe_exl3_dequant", _lib.lib().mi355moe_exl3_dequant(_p(t), kt, nt, _p(out), _stream(dev)))
    return out


def sigmoid(g: torch.Tensor, variant: int = 0) -> torch.Tensor:
    """The SwiGLU epilogues' sigmoid of fp32 g (any shape): variant 0 = the decode epilogue's
    1 / (1 + (float)exp(-(double)g)) (E3's formula, exl3_fat_moe.cu:366-369), 1 = the grouped prefill epilogues'."""
    dev = _need_cuda(g)
    if g.dtype != torch.float32:
        raise ValueError("g must be float32")
    t = g.contiguous()
    out = torch.empty_like(t)
    _lib.check("mi355moe_sigmoid", _lib.lib().mi355moe_sigmoid(_p(t), t.numel(), int(variant), _p(out), _stream(dev)))
    return out


def router_logits(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """fp32 [T, E] holding bf16(x bf16 [T, K] @ w bf16 [E, K]^T): the exact (float64) dot products rounded to bf16
    through fp32, what F.linear(x, w).to(torch.float32) returns (code/fork/docs/BF16_GEMV.md:27,38)."""
    dev = _need_cuda(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("router_logits: bf16 x [T, K] and bf16 W [E, K]")
    if x.stride(1) != 1:
        raise ValueError("router_logits: x needs unit column stride")
    w = w.contiguous()
    T, K = x.shape
    E = w.shape[0]
    out = torch.empty(T, E, dtype=torch.float32, device=dev)
    _lib.check("mi355moe_router_logits", _lib.lib().mi355moe_router_logits(_p(x), T, K, x.stride(0), _p(w), E,
                                                                           _p(out), _stream(dev)))
    return out


def router_topk(logits: torch.Tensor, topk: int, bias: torch.Tensor | None = None, routed_scale: float = 1.0,
                renormalize: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """(ids int32 [T, topk], weights fp32 [T, topk]) of vLLM grouped_topk with sigmoid scoring and one group."""
    dev = _need_cuda(logits, bias)
    lg = logits.float().contiguous()
    T, E = lg.shape
    b = None if bias is None else bias.float().contiguous()
    if b is not None and b.numel() != E:
        raise ValueError("bias must have one entry per expert")
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    wts = torch.empty(T, topk, dtype=torch.float32, device=dev)
    _lib.check("mi355moe_router_topk", _lib.lib().mi355moe_router_topk(
        _p(lg), T, E, _p(b), topk, float(routed_scale), int(bool(renormalize)), _p(ids), _p(wts), _stream(dev)))
    return ids, wts


def route(ids: torch.Tensor, weights: torch.Tensor, n: int, R: int = 1 << 30, seg_rows: int = 16,
          expert_map: torch.Tensor | None = None) -> dict:
    """The token -> expert permutation tables (stage entry; see mi355moe_route in include/mi355moe.h)."""
    dev = _need_cuda(ids, weights, expert_map)
    T, topk = ids.shape
    P = T * topk
    ids_c, w_c = ids.contiguous(), weights.contiguous()
    s_cap = min(P, n) + (P + seg_rows - 1) // seg_rows
    i32 = dict(dtype=torch.int32, device=dev)
    out = {"tok": torch.empty(P, **i32), "w16": torch.empty(P, dtype=torch.float16, device=dev),
           "pe": torch.empty(P, **i32), "inv": torch.empty(P, **i32), "seg_expert": torch.full((s_cap,), -1, **i32),
           "seg_row0": torch.zeros(s_cap, **i32), "seg_rows": torch.zeros(s_cap, **i32),
           "nseg": torch.zeros(1, **i32), "counts": torch.zeros(n + 1, **i32)}
    L = _lib.lib()
    ws = workspace(dev, L.mi355moe_route_workspace_bytes(P, n))
    em = None
    if expert_map is not None:
        em = expert_map.to(torch.int64).contiguous()
    _lib.check("mi355moe_route", L.mi355moe_route(
        _p(ids_c), ids_dtype_code(ids.dtype), _p(w_c), weight_dtype_code(weights.dtype), T, topk, _p(em),
        0 if em is None else em.numel(), n, R, seg_rows, _p(out["tok"]), _p(out["w16"]), _p(out["pe"]),
        _p(out["inv"]), _p(out["seg_expert"]), _p(out["seg_row0"]), _p(out["seg_rows"]), s_cap, _p(out["nseg"]),
        _p(out["counts"]), _p(ws), ws.numel(), _stream(dev)))
    return out


def rot_in(x: torch.Tensor, tok: torch.Tensor, pe: torch.Tensor, suh_table: torch.Tensor) -> torch.Tensor:
    """fp16 [P, K]: row pos = fp16(H(fp16(x[tok[pos]] * suh[pe[pos]])) * r) (rows with pe < 0 are NaN)."""
    dev = _need_cuda(x, tok, pe, suh_table)
    if x.stride(1) != 1:
        raise ValueError("rot_in: x needs unit column stride")
    P, K = tok.numel(), x.shape[1]
    out = torch.full((P, K), float("nan"), dtype=torch.float16, device=dev)
    _lib.check("mi355moe_rot_in", _lib.lib().mi355moe_rot_in(
        _p(x), act_dtype_code(x.dtype), x.stride(0), K, _p(tok.int().contiguous()), _p(pe.int().contiguous()), P,
        _p(suh_table.contiguous()), _p(out), _stream(dev)))
    return out


def moe_forward_ids(experts: Exl3Experts, x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                    limit: float = 10.0, expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None, stages: int = _lib.STAGE_ALL,
                    path: int = _lib.PATH_AUTO, accumulate: bool = False,
                    bf16_contrib: bool = False, persistent: bool = False) -> torch.Tensor:
    """Routed-expert output [T, K] (x's dtype unless out/out_dtype say otherwise), written, or with accumulate added
    to out's values (the shared-expert fold: out holds the shared experts' output; fp32 sum, one rounding).
    path: _lib.PATH_AUTO (decode kernels for few pairs, the grouped MFMA prefill kernels for many), or forced.
    stages: a subset of the call's launches (_lib.STAGE_*), for timing one kernel; the default runs them all.
    bf16_contrib: the grouped path keeps its per-pair down accumulators in bf16 (half the contribution traffic;
    code/fork/docs/OPT_MOE.md:13). persistent: the grouped path's gate/up and down tiles in one launch, taken in
    ticket order with per-segment dataflow counts (code/fork/kernels/moe_e4m3.cu:867-897), whatever the call's size
    (calls running both stages take it by themselves); results bit-identical to the separate launches."""
    if accumulate and out is None:
        raise ValueError("accumulate needs out")
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
        raise ValueError("out must be [T, K] with unit column stride")
    L = _lib.lib()
    nb = L.mi355moe_moe_workspace_bytes_path(ctypes.byref(experts.desc), T, topk, int(path))
    if nb < 0:
        raise ValueError("mi355moe_moe_workspace_bytes rejected the shape")
    ws = workspace(dev, nb)
    em = None if expert_map is None else expert_map.to(torch.int64).contiguous()
    opts = ((_lib.OPT_ACCUMULATE if accumulate else 0) | (_lib.OPT_BF16_CONTRIB if bf16_contrib else 0) |
            (_lib.OPT_PERSISTENT if persistent else 0))
    _lib.check("mi355moe_moe_forward_ids", L.mi355moe_moe_forward_ids_opt(
        ctypes.byref(experts.desc), _p(x), act_dtype_code(x.dtype), x.stride(0), T, _p(ids),
        ids_dtype_code(ids.dtype), _p(w), weight_dtype_code(w.dtype), topk, _p(em), 0 if em is None else em.numel(),
        float(limit), _p(out), weight_dtype_code(out.dtype), out.stride(0), _p(ws), ws.numel(), int(path),
        int(stages), opts, _stream(dev)))
    return out


def sched_item(ticket: int, segments: int, lag: int, gateup_items: int, down_items: int) -> tuple[int, int, int]:
    """(kind, segment, block) of item `ticket` of the one-launch schedule (kind 0 gate/up, 1 down, -1 past the last
    item): the library's own item order, evaluated on the host (code/fork/kernels/moe_e4m3.cu:931-959)."""
    k, s, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check("mi355moe_sched_item", _lib.lib().mi355moe_sched_item(int(ticket), int(segments), int(lag),
                                                                     int(gateup_items), int(down_items),
                                                                     ctypes.byref(k), ctypes.byref(s),
                                                                     ctypes.byref(b)))
    return k.value, s.value, b.value


def moe_forward_ids_split(experts: Exl3Experts, x: torch.Tensor, topk_ids: torch.Tensor,
                          topk_weights: torch.Tensor, thin_cap: int, limit: float = 10.0,
                          expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None,
                          out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The thin/fat split of a prefill-size call (code/fork/docs/prod_exl3_reference.py:1659-1679 with the cap of
    code/fork/glm53_prefill_cap.py): experts routed at most thin_cap rows on the decode kernels, the rest on the
    grouped kernels, one slot-order combine; output [T, K] written. thin_cap = 0: all experts grouped."""
    dev = _need_cuda(x, topk_ids, topk_weights, expert_map)
    if dev != experts.device:
        raise ValueError(f"activations on {dev}, experts on {experts.device}")
    if x.dim() != 2 or x.shape[1] != experts.K or x.stride(1) != 1:
        raise ValueError(f"x must be [T, {experts.K}] with unit column stride")
    T = x.shape[0]
    ids = topk_ids.reshape(T, -1).contiguous()
    w = topk_weights.reshape(T, -1).contiguous()
    topk = ids.shape[1]
    if out is None:
        out = torch.empty(T, experts.K, dtype=out_dtype or x.dtype, device=dev)
    L = _lib.lib()
    nb = L.mi355moe_moe_split_workspace_bytes(ctypes.byref(experts.desc), T, topk, int(thin_cap))
    if nb < 0:
        raise ValueError("mi355moe_moe_split_workspace_bytes rejected the shape")
    ws = workspace(dev, nb)
    em = None if expert_map is None else expert_map.to(torch.int64).contiguous()
    _lib.check("mi355moe_moe_forward_ids_split", L.mi355moe_moe_forward_ids_split(
        ctypes.byref(experts.desc), _p(x), act_dtype_code(x.dtype), x.stride(0), T, _p(ids),
        ids_dtype_code(ids.dtype), _p(w), weight_dtype_code(w.dtype), topk, _p(em), 0 if em is None else em.numel(),
        float(limit), _p(out), weight_dtype_code(out.dtype), out.stride(0), int(thin_cap), _p(ws), ws.numel(),
        _stream(dev)))
    return out


def moe_forward_ids_e4m3(experts: Exl3Experts, x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                         limit: float = 10.0, expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None,
                         out_dtype: torch.dtype | None = None, stages: int = _lib.STAGE_ALL,
                         accumulate: bool = False, bf16_contrib: bool = False, down16: bool = False,
                         persistent: bool = False) -> torch.Tensor:
    """The trellis-sourced e4m3 variant of the routed experts (code/fork/overlay/glm53_moe_e4m3.py:484-592 run(),
    numerics of spec_ffn :666-674): activations quantized per row to e4m3 after the input rotation, EXL3 weights
    rounded to e4m3, fp32 sums; output [T, K] written like moe_forward_ids. The layer needs gate and up sharing one
    suh and hidden <= 4096. accumulate / bf16_contrib: the ACC=bf16 and FOLD_SHARED knobs (code/fork/docs/
    OPT_MOE.md:9-21) as in moe_forward_ids. down16: the down projection on fp16 operands (DOWN16, spec_proj16
    :660-664) instead of e4m3. persistent: the one-launch ticket-ordered gate/up -> down schedule (SCHED mode
    "fused", code/fork/kernels/moe_e4m3.cu:867-897) whatever the call's size (calls running both stages take it by
    themselves); bit-identical to the separate launches."""
    if accumulate and out is None:
        raise ValueError("accumulate needs out")
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
        raise ValueError("out must be [T, K] with unit column stride")
    L = _lib.lib()
    nb = L.mi355moe_e4m3_moe_workspace_bytes(ctypes.byref(experts.desc), T, topk)
    if nb < 0:
        raise ValueError("mi355moe_e4m3_moe_workspace_bytes rejected the shape")
    ws = workspace(dev, nb)
    em = None if expert_map is None else expert_map.to(torch.int64).contiguous()
    if accumulate or bf16_contrib or down16 or persistent:
        opts = (_lib.OPT_E4M3 | (_lib.OPT_ACCUMULATE if accumulate else 0) |
                (_lib.OPT_BF16_CONTRIB if bf16_contrib else 0) | (_lib.OPT_DOWN16 if down16 else 0) |
                (_lib.OPT_PERSISTENT if persistent else 0))
        _lib.check("mi355moe_moe_forward_ids_opt", L.mi355moe_moe_forward_ids_opt(
            ctypes.byref(experts.desc), _p(x), act_dtype_code(x.dtype), x.stride(0), T, _p(ids),
            ids_dtype_code(ids.dtype), _p(w), weight_dtype_code(w.dtype), topk, _p(em),
            0 if em is None else em.numel(), float(limit), _p(out), weight_dtype_code(out.dtype), out.stride(0),
            _p(ws), ws.numel(), _lib.PATH_PREFILL, int(stages), opts, _stream(dev)))
        return out
    _lib.check("mi355moe_e4m3_moe_forward_ids", L.mi355moe_e4m3_moe_forward_ids(
        ctypes.byref(experts.desc), _p(x), act_dtype_code(x.dtype), x.stride(0), T, _p(ids),
        ids_dtype_code(ids.dtype), _p(w), weight_dtype_code(w.dtype), topk, _p(em), 0 if em is None else em.numel(),
        float(limit), _p(out), weight_dtype_code(out.dtype), out.stride(0), _p(ws), ws.numel(), int(stages),
        _stream(dev)))
    return out


def moe_layer(experts: Exl3Experts, x: torch.Tensor, router_w: torch.Tensor | None = None,
              logits: torch.Tensor | None = None, topk: int = 8, bias: torch.Tensor | None = None,
              routed_scale: float = 1.0, renormalize: bool = True, limit: float = 10.0,
              out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
              return_picks: bool = False, picks_out: tuple | None = None):
    """Routed-expert output [T, K] of one MoE layer from its hidden states: router logits (from router_w bf16
    [E, K], or the given fp32 logits [T, E]), sigmoid + bias top-k, permutation, expert GEMMs and combine in one
    call (small calls run router, top-k and permutation as one launch). With return_picks, also (ids int32, weights
    fp32), both [T, topk], written into picks_out when given."""
    if (router_w is None) == (logits is None):
        raise ValueError("give exactly one of router_w and logits")
    dev = _need_cuda(x, router_w, logits, bias)
    if dev != experts.device:
        raise ValueError(f"activations on {dev}, experts on {experts.device}")
    if x.dim() != 2 or x.shape[1] != experts.K or x.stride(1) != 1:
        raise ValueError(f"x must be [T, {experts.K}] with unit column stride")
    T = x.shape[0]
    if router_w is not None:
        if x.dtype != torch.bfloat16 or router_w.dtype != torch.bfloat16:
            raise ValueError("the router GEMV takes bf16 x and bf16 router_w")
        rw = router_w.contiguous()
        E = rw.shape[0]
        lg = None
    else:
        lg = logits.float().contiguous()
        E = lg.shape[1]
        rw = None
    b = None if bias is None else bias.float().contiguous()
    if b is not None and b.numel() != E:
        raise ValueError("bias must have one entry per expert")
    if out is None:
        out = torch.empty(T, experts.K, dtype=out_dtype or x.dtype, device=dev)
    if out.shape != (T, experts.K) or out.stride(1) != 1:
        raise ValueError("out must be [T, K] with unit column stride")
    ids = wts = None
    if picks_out is not None:
        ids, wts = picks_out
        if (ids.shape != (T, topk) or ids.dtype != torch.int32 or not ids.is_contiguous() or wts.shape != (T, topk)
                or wts.dtype != torch.float32 or not wts.is_contiguous()):
            raise ValueError("picks_out must be contiguous (int32 [T, topk], fp32 [T, topk])")
    elif return_picks:
        ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
        wts = torch.empty(T, topk, dtype=torch.float32, device=dev)
    L = _lib.lib()
    nb = L.mi355moe_moe_layer_workspace_bytes(ctypes.byref(experts.desc), T, topk, E)
    if nb < 0:
        raise ValueError("mi355moe_moe_layer_workspace_bytes rejected the shape")
    ws = workspace(dev, nb)
    _lib.check("mi355moe_moe_layer", L.mi355moe_moe_layer(
        ctypes.byref(experts.desc), _p(x), act_dtype_code(x.dtype), x.stride(0), T, _p(rw), _p(lg), E, _p(b), topk,
        float(routed_scale), int(bool(renormalize)), float(limit), _p(out), weight_dtype_code(out.dtype),
        out.stride(0), _p(ids), _p(wts), _p(ws), ws.numel(), _stream(dev)))
    return (out, ids, wts) if (return_picks or picks_out is not None) else out
