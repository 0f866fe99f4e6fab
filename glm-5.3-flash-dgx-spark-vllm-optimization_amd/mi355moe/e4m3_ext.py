"""The e4m3 expert extension's stage functions as the reference's overlay drives them
(code/fork/overlay/glm53_moe_e4m3.py:450-592 plan() / run(); extension bindings code/fork/kernels/moe_e4m3.cu:
3085-3099), over the trellis-sourced e4m3 kernels of libmi355moe.so.

  tile_rows / version      segment height of the fused stage (this library's 256-row tiles) / 1
  seg_tables               (seg_expert, seg_row0, seg_rows, num_segs, num_rows) from int64 counts [n]
  gather2                  per routed pair: rotate, quantise per row to e4m3, write row pos[j]; zero `out` if given
  fused                    gate/up + down-input quantisation + down over the segments; out[token] += rows in row order
  plan / run               the overlay's routing tables and its fused-schedule run() on an EXL3 layer

The quantised rows are staged in this library's layout (fp16 holding the e4m3 values, k permuted within 16-element
groups), which takes two bytes per element: `a8` (uint8 [P, K] in the reference) keeps its signature role but the
rows live in a per-device staging buffer that gather2 fills and the next fused call on the same device reads, so the
two must be called in that order on one stream (as run() does). a8d, dsc and sync are likewise accepted and unused
(the down inputs and their scales live in the workspace; a16 only gives the intermediate size), and lag / grid /
variant are schedule knobs of the reference's kernel with no counterpart here.
"""
from __future__ import annotations

import torch

from . import _lib, ops

_STAGE: dict = {}          # device -> fp16 staging buffer of the quantised rows (grown, old ones kept alive)
_STAGE_OLD: dict = {}


def tile_rows() -> int:
    return int(_lib.lib().mi355moe_e4m3_tile_rows())


def version() -> int:
    return 1


def _staging(dev: torch.device, rows: int, K: int) -> torch.Tensor:
    key = (dev.type, dev.index)
    buf = _STAGE.get(key)
    if buf is None or buf.numel() < rows * K:
        if ops._capturing(dev):
            raise RuntimeError("mi355moe e4m3 staging buffer cannot grow during graph capture; run one eager call of "
                               "this size first")
        if buf is not None:
            _STAGE_OLD.setdefault(key, []).append(buf)
        buf = torch.empty(max(rows * K, 1 << 20), dtype=torch.float16, device=dev)
        _STAGE[key] = buf
    return buf


def seg_tables(counts: torch.Tensor, tile: int, rows_cap: int) -> list:
    """[seg_expert, seg_row0, seg_rows, num_segs, num_rows] (int32, device) of rows grouped by expert: expert e's
    rows start at the exclusive scan of counts, ceil(counts[e] / tile) segments each; max_segs = ceil(rows_cap /
    tile) + n entries (moe_e4m3.cu:3066-3083)."""
    if not counts.is_cuda or counts.dtype != torch.int64 or counts.dim() != 1 or not counts.is_contiguous():
        raise ValueError("counts must be a contiguous int64 CUDA vector")
    n = counts.numel()
    max_segs = (rows_cap + tile - 1) // tile + n
    i32 = dict(dtype=torch.int32, device=counts.device)
    se, sr0, sr = torch.zeros(max_segs, **i32), torch.zeros(max_segs, **i32), torch.zeros(max_segs, **i32)
    ns, nr = torch.empty(1, **i32), torch.empty(1, **i32)
    _lib.check("mi355moe_e4m3_seg_tables", _lib.lib().mi355moe_e4m3_seg_tables(
        ops._p(counts), n, int(tile), int(rows_cap), ops._p(se), ops._p(sr0), ops._p(sr), max_segs, ops._p(ns),
        ops._p(nr), ops._stream(counts.device)))
    return [se, sr0, sr, ns, nr]


def gather2(xh: torch.Tensor, local: torch.Tensor, pos: torch.Tensor, gate_suh: torch.Tensor, a8: torch.Tensor,
            asc: torch.Tensor, out: torch.Tensor | None, topk: int, n_exp: int) -> None:
    """Routed pair j = (token j // topk) with local expert local[j] (skipped unless 0 <= local < n_exp): v =
    H(fp16(x) * suh) * r, s = amax / 448, the e4m3 row written as row pos[j], asc[pos[j]] = s; out zeroed if given."""
    del a8
    if xh.dim() != 2 or xh.stride(1) != 1:
        raise ValueError("xh must be [T, K] with unit column stride")
    for name, t, dt in (("local", local, torch.int32), ("pos", pos, torch.int32), ("gate_suh", gate_suh, torch.int64),
                        ("asc", asc, torch.float32)):
        if not t.is_cuda or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name}: expected a contiguous CUDA {dt} tensor")
    T, K = xh.shape
    P = T * int(topk)
    stage = _staging(xh.device, P, K)
    od = _lib.F32
    if out is not None:
        od = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}.get(out.dtype)
        if od is None or out.shape != (T, K) or out.stride(1) != 1:
            raise ValueError("out must be fp32 or bf16 [T, K] with unit column stride")
    _lib.check("mi355moe_e4m3_gather2", _lib.lib().mi355moe_e4m3_gather2(
        ops._p(xh), ops.act_dtype_code(xh.dtype), xh.stride(0), T, K, ops._p(local), ops._p(pos), int(topk),
        int(n_exp), ops._p(gate_suh), ops._p(stage), ops._p(asc), ops._p(out), od,
        0 if out is None else out.stride(0), ops._stream(xh.device)))


def fused(a8, asc, a8d, dsc, a16, out, gate_ptrs, up_ptrs, gate_svh, up_svh, down_ptrs, down_suh, down_svh, row_token,
          row_weight, seg_expert, seg_row0, seg_rows, num_segs, sync, limit, lag=12, grid=0, variant=0, *,
          intermediate: int | None = None) -> None:
    """Gate/up, the down input's per-row e4m3 quantisation and the down GEMM of every segment's rows (the rows gather2
    staged), then out[token] += the token's rows in row order weighted by row_weight (fp32; out fp32 or bf16). The
    intermediate size is a16's second dimension (the reference passes its fp16 [rows_cap, N] buffer), or
    `intermediate`."""
    del a8, a8d, dsc, sync, lag, grid, variant
    N = int(intermediate) if intermediate else (int(a16.shape[1]) if a16 is not None else 0)
    if N <= 0:
        raise ValueError("fused(): pass a16 ([rows_cap, N]) or intermediate=N")
    rows_cap = int(row_token.numel())
    T, K = out.shape
    dev = out.device
    stage = _staging(dev, rows_cap, K)
    od = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}.get(out.dtype)
    if od is None or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 or bf16 [T, K] tensor")
    for name, t in (("asc", asc), ("row_token", row_token), ("seg_expert", seg_expert), ("num_segs", num_segs)):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name}: expected a contiguous CUDA tensor")
    rw = row_weight.to(torch.float32).contiguous()
    L = _lib.lib()
    ws = ops.workspace(dev, L.mi355moe_e4m3_fused_workspace_bytes(rows_cap, K, N, T))
    _lib.check("mi355moe_e4m3_fused", L.mi355moe_e4m3_fused(
        ops._p(stage), ops._p(asc), ops._p(out), od, T, out.stride(0), K, N, gate_ptrs.numel(), ops._p(gate_ptrs),
        ops._p(up_ptrs), ops._p(gate_svh), ops._p(up_svh), ops._p(down_ptrs), ops._p(down_suh), ops._p(down_svh),
        ops._p(row_token.to(torch.int64)), ops._p(rw), rows_cap, ops._p(seg_expert), ops._p(seg_row0),
        ops._p(seg_rows), seg_expert.numel(), ops._p(num_segs), float(limit), ops._p(ws), ws.numel(),
        ops._stream(dev)))


def plan(ids: torch.Tensor, weights: torch.Tensor, n_exp: int, expert_map: torch.Tensor | None = None) -> dict:
    """Routing tables on the device, no host synchronisation (glm53_moe_e4m3.py:450-477): rows = routed (token, slot)
    pairs sorted by local expert (stable), non-local / invalid pairs last and never computed."""
    T, topk = int(ids.shape[0]), int(ids.shape[1])
    P = T * topk
    dev = ids.device
    flat = ids.reshape(-1).to(torch.long)
    if expert_map is not None:
        em = expert_map.to(torch.long)
        safe = flat.clamp(0, em.numel() - 1)
        mapped = em[safe]
        bad = (flat < 0) | (flat >= em.numel()) | (mapped < 0) | (mapped >= n_exp)
        local = torch.where(bad, torch.full_like(flat, n_exp), mapped)
    else:
        local = torch.where((flat < 0) | (flat >= n_exp), torch.full_like(flat, n_exp), flat)
    order = torch.argsort(local, stable=True)
    counts = torch.zeros(n_exp + 1, dtype=torch.long, device=dev)
    counts.scatter_add_(0, local, torch.ones_like(local))
    pos = torch.empty(P, dtype=torch.int32, device=dev)
    pos[order] = torch.arange(P, dtype=torch.int32, device=dev)
    t = {"T": T, "topk": topk, "P": P, "n_exp": n_exp, "local": local.to(torch.int32), "pos": pos,
         "row_token": torch.div(order, topk, rounding_mode="floor"),
         "row_weight": weights.reshape(-1).to(torch.float32).index_select(0, order),
         "row_expert": local.index_select(0, order).to(torch.int32)}
    se, sr0, sr, ns, nr = seg_tables(counts[:n_exp].contiguous(), tile_rows(), P)
    t.update(seg_expert=se, seg_row0=sr0, seg_rows=sr, num_segs=ns, num_rows=nr)
    return t


def run(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts, limit: float,
        expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """The routed experts of one EXL3 layer in e4m3 numerics for every token of x2d, the overlay's fused schedule
    (glm53_moe_e4m3.py:480-592): plan, gather2 (zeroing out), fused. Returns fp32 [T, K] (or adds into `out`, fp32 or
    bf16, without zeroing it). experts: an mi355moe.Exl3Experts."""
    T = int(x2d.shape[0])
    ids2 = ids.reshape(T, -1)
    t = plan(ids2, weights.reshape(T, -1), experts.n, expert_map)
    ptrs = experts.tables
    asc = torch.empty(t["P"], dtype=torch.float32, device=x2d.device)
    xc = x2d.contiguous()
    if out is None:
        out = torch.empty(T, experts.K, dtype=torch.float32, device=x2d.device)
        gather2(xc, t["local"], t["pos"], ptrs["gate_suh"], None, asc, out, t["topk"], experts.n)
    else:
        gather2(xc, t["local"], t["pos"], ptrs["gate_suh"], None, asc, None, t["topk"], experts.n)
    fused(None, asc, None, None, None, out, ptrs["gate_trellis"], ptrs["up_trellis"], ptrs["gate_svh"],
          ptrs["up_svh"], ptrs["down_trellis"], ptrs["down_suh"], ptrs["down_svh"], t["row_token"], t["row_weight"],
          t["seg_expert"], t["seg_row0"], t["seg_rows"], t["num_segs"], None, limit, intermediate=experts.N)
    return out
