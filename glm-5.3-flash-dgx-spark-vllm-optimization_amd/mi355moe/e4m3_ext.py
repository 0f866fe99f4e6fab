"""The e4m3 expert extension's stage functions, as the reference's overlay drives them (code/fork/overlay/
glm53_moe_e4m3.py:450-592 plan() / run(); extension bindings code/fork/kernels/moe_e4m3.cu:3081-3096), over the
trellis-sourced e4m3 kernels of libmi355moe.so.

Every buffer belongs to the caller and holds the extension's format (include/mi355moe.h):
  a8 uint8 [rows, K], a8d uint8 [rows, N]   e4m3 codes, the columns of each 16-group in the order
                                            0,1,8,9,2,3,10,11,4,5,12,13,6,7,14,15 (the extension's perm_cols)
  asc, dsc float32 [rows]                   row scales (value = code * scale)
  a16 float16 [rows, N]                     the SwiGLU output, plain column order
so a stage may be replaced by the reference's own (or read by its tests) at any point of the chain. The kernels'
fp16 staging copies of the code rows live in the library's scratch workspace for the duration of one call only.

  tile_rows / version      segment height of the GEMM stages (this library's 256-row tiles) / 2
  seg_tables               (seg_expert, seg_row0, seg_rows, num_segs, num_rows) from int64 counts [n]
  gather / gather2         per routed pair: rotate, quantise per row to e4m3, write row pos[j] (gather2: and zero out)
  gather_tok               one quantised row per token (every expert shares its w13 suh), out zeroed if given
  gateup / actq / down     the chunked schedule's stages (segments of chunk c of nchunks)
  fused                    gateup + actq + down of every segment; a8d / dsc / a16 written when given
  plan / run               the overlay's routing tables (on the device) and its schedule on an Exl3Experts layer

The per-call knobs of the reference's persistent kernel (lag, grid, sync) are accepted unused: fused() takes the
library's one-launch schedule by itself where it pays (its lag from the environment variable MI355MOE_SCHED_LAG).
"""
from __future__ import annotations

import torch

from . import _lib, ops
from .layer import _check_aligned

TOKEN_ROWS = _lib.E4M3_TOKEN_ROWS       # fused variant bit: a8 / asc hold one row per token (gather_tok)
DOWN16 = _lib.E4M3_DOWN16               # fused variant bit: the down projection on fp16 operands
LEAN_MAINLOOP = _lib.E4M3_LEAN_MAINLOOP  # fused variant bit of the reference's leaner main loop: same results


def tile_rows() -> int:
    return int(_lib.lib().mi355moe_e4m3_tile_rows())


def version() -> int:
    return 2


def _dev_tensor(name: str, t: torch.Tensor, dtype: torch.dtype, dim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous CUDA {dtype} tensor")
    if dim is not None and t.dim() != dim:
        raise ValueError(f"{name}: expected {dim} dimensions, got {t.dim()}")
    if t.data_ptr() % 16:
        raise ValueError(f"{name}: the buffer must start on a 16-byte boundary")


def _ptr_table(name: str, t: torch.Tensor, n: int) -> None:
    if not t.is_cuda or t.dtype != torch.int64 or t.dim() != 1 or t.numel() < n or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous int64 CUDA vector of >= {n} device addresses")
    _check_aligned(name, t, n)


def _segs(seg_expert, seg_row0, seg_rows, num_segs) -> int:
    for name, t in (("seg_row0", seg_row0), ("seg_rows", seg_rows), ("num_segs", num_segs)):
        _dev_tensor(name, t, torch.int32)
    if seg_expert is not None:
        _dev_tensor("seg_expert", seg_expert, torch.int32)
        if seg_expert.numel() > seg_row0.numel() or seg_expert.numel() > seg_rows.numel():
            raise ValueError("segment tables of different lengths")
        return seg_expert.numel()
    return min(seg_row0.numel(), seg_rows.numel())


def _stage_ws(dev: torch.device, rows: int, K: int, N: int, tokens: int) -> torch.Tensor:
    nb = _lib.lib().mi355moe_e4m3_stage_workspace_bytes(rows, K, N, tokens)
    if nb < 0:
        raise ValueError("mi355moe_e4m3_stage_workspace_bytes rejected the shape")
    return ops.workspace(dev, nb)


def seg_tables(counts: torch.Tensor, tile: int, rows_cap: int) -> list:
    """[seg_expert, seg_row0, seg_rows, num_segs, num_rows] (int32, device) of rows grouped by expert: expert e's rows
    start at the exclusive scan of counts, ceil(counts[e] / tile) segments each; max_segs = ceil(rows_cap / tile) + n
    entries (moe_e4m3.cu:3062-3083). tile <= tile_rows()."""
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


def _out_args(out: torch.Tensor | None, T: int):
    if out is None:
        return None, _lib.F32, 0
    od = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}.get(out.dtype)
    if od is None or out.dim() != 2 or out.shape[0] != T or out.stride(1) != 1 or out.stride(0) < out.shape[1]:
        raise ValueError("out must be fp32 or bf16 [T, K] with unit column stride")
    return out, od, out.stride(0)


def _x_args(x: torch.Tensor) -> None:
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [T, K] with unit column stride")


def gather2(x: torch.Tensor, local: torch.Tensor, pos: torch.Tensor, suh_ptrs: torch.Tensor, a8: torch.Tensor,
            asc: torch.Tensor, out: torch.Tensor | None, topk: int, n_exp: int) -> None:
    """Routed pair j = (token j // topk, slot j % topk) with local expert local[j] (skipped unless 0 <= local <
    n_exp): v = H(fp16(x) * suh) * r, s = amax / 448, the e4m3 codes into a8 row pos[j], asc[pos[j]] = s
    (moe_e4m3.cu:2493-2534); out (fp32 or bf16 [T, K]) zeroed when given."""
    _x_args(x)
    T, K = x.shape
    _dev_tensor("local", local, torch.int32)
    _dev_tensor("pos", pos, torch.int32)
    _dev_tensor("a8", a8, torch.uint8, 2)
    _dev_tensor("asc", asc, torch.float32)
    _ptr_table("suh_ptrs", suh_ptrs, int(n_exp))
    if a8.shape[1] != K or asc.numel() < a8.shape[0] or local.numel() < T * topk or pos.numel() < T * topk:
        raise ValueError("gather2: a8 uint8 [rows, K], asc [>= rows], local / pos [>= T * topk]")
    out, od, ostr = _out_args(out, T)
    _lib.check("mi355moe_e4m3_gather2", _lib.lib().mi355moe_e4m3_gather2(
        ops._p(x), ops.act_dtype_code(x.dtype), x.stride(0), T, K, ops._p(local), ops._p(pos), int(topk), int(n_exp),
        ops._p(suh_ptrs), ops._p(a8), a8.shape[0], ops._p(asc), ops._p(out), od, ostr, ops._stream(x.device)))


def gather(x: torch.Tensor, local: torch.Tensor, pos: torch.Tensor, suh_ptrs: torch.Tensor, a8: torch.Tensor,
           asc: torch.Tensor, topk: int, n_exp: int, variant: int = 0) -> None:
    """gather2 without the zeroing of an output (moe_e4m3.cu:2457-2491; variant 0 only, the others are the
    reference's debug builds)."""
    if variant != 0:
        raise ValueError(f"gather: unknown variant {variant}")
    gather2(x, local, pos, suh_ptrs, a8, asc, None, topk, n_exp)


def gather_tok(x: torch.Tensor, suh_ptrs: torch.Tensor, a8: torch.Tensor, asc: torch.Tensor,
               out: torch.Tensor | None) -> None:
    """One quantised row per token with the suh of expert 0 (every expert's, when the layer shares one w13 suh):
    a8 row t, asc[t] (moe_e4m3.cu:2536-2571); out zeroed when given."""
    _x_args(x)
    T, K = x.shape
    _dev_tensor("a8", a8, torch.uint8, 2)
    _dev_tensor("asc", asc, torch.float32)
    _ptr_table("suh_ptrs", suh_ptrs, 1)
    if a8.shape[1] != K or a8.shape[0] < T or asc.numel() < T:
        raise ValueError("gather_tok: a8 uint8 [>= T, K], asc [>= T]")
    out, od, ostr = _out_args(out, T)
    _lib.check("mi355moe_e4m3_gather_tok", _lib.lib().mi355moe_e4m3_gather_tok(
        ops._p(x), ops.act_dtype_code(x.dtype), x.stride(0), T, K, ops._p(suh_ptrs), ops._p(a8), a8.shape[0],
        ops._p(asc), ops._p(out), od, ostr, ops._stream(x.device)))


def gateup(a8, asc, gate_ptrs, up_ptrs, gate_svh, up_svh, a16, seg_expert, seg_row0, seg_rows, num_segs, limit,
           variant=0, chunk=0, nchunks=1, grid=0) -> None:
    """a16 rows of the segments of chunk `chunk` of `nchunks` = fp16(silu(min(g, L)) * clamp(u, -L, L)) from the a8
    rows (moe_e4m3.cu:2641-2676; variant 0 only)."""
    del grid
    if variant != 0:
        raise ValueError(f"gateup: unknown variant {variant}")
    _dev_tensor("a8", a8, torch.uint8, 2)
    _dev_tensor("asc", asc, torch.float32)
    _dev_tensor("a16", a16, torch.float16, 2)
    rows, K = a8.shape
    N = a16.shape[1]
    if a16.shape[0] != rows or asc.numel() < rows:
        raise ValueError("gateup: a8 [rows, K], asc [>= rows], a16 [rows, N]")
    n = gate_ptrs.numel()
    for name, t in (("gate_ptrs", gate_ptrs), ("up_ptrs", up_ptrs), ("gate_svh", gate_svh), ("up_svh", up_svh)):
        _ptr_table(name, t, n)
    S = _segs(seg_expert, seg_row0, seg_rows, num_segs)
    dev = a8.device
    ws = _stage_ws(dev, rows, K, N, 0)
    _lib.check("mi355moe_e4m3_gateup", _lib.lib().mi355moe_e4m3_gateup(
        ops._p(a8), ops._p(asc), rows, K, N, n, ops._p(gate_ptrs), ops._p(up_ptrs), ops._p(gate_svh), ops._p(up_svh),
        ops._p(a16), ops._p(seg_expert), ops._p(seg_row0), ops._p(seg_rows), S, ops._p(num_segs), float(limit),
        int(chunk), int(nchunks), ops._p(ws), ws.numel(), ops._stream(dev)))


def actq(a16, row_expert, suh_ptrs, a8d, dsc, seg_row0, seg_rows, num_segs, chunk=0, nchunks=1) -> None:
    """The down inputs of the chunk's rows: v = H(float(a16[r]) * suh_d[row_expert[r]]) * r quantised per row into
    a8d row r and dsc[r] (moe_e4m3.cu:2573-2600)."""
    _dev_tensor("a16", a16, torch.float16, 2)
    _dev_tensor("row_expert", row_expert, torch.int32)
    _dev_tensor("a8d", a8d, torch.uint8, 2)
    _dev_tensor("dsc", dsc, torch.float32)
    rows, N = a16.shape
    if a8d.shape != (rows, N) or dsc.numel() < rows or row_expert.numel() < rows:
        raise ValueError("actq: a16 [rows, N], a8d [rows, N], dsc / row_expert [>= rows]")
    n = suh_ptrs.numel()
    _ptr_table("suh_ptrs", suh_ptrs, n)
    S = _segs(None, seg_row0, seg_rows, num_segs)
    ws = _stage_ws(a16.device, rows, 256, N, 0)
    _lib.check("mi355moe_e4m3_actq", _lib.lib().mi355moe_e4m3_actq(
        ops._p(a16), rows, N, ops._p(row_expert), n, ops._p(suh_ptrs), ops._p(a8d), ops._p(dsc), ops._p(seg_row0),
        ops._p(seg_rows), S, ops._p(num_segs), int(chunk), int(nchunks), ops._p(ws), ws.numel(),
        ops._stream(a16.device)))


def down(a8d, dsc, down_ptrs, down_svh, out, row_token, row_weight, seg_expert, seg_row0, seg_rows, num_segs,
         variant=0, chunk=0, nchunks=1, grid=0) -> None:
    """out (fp32 [T, K]) += every token's rows of the chunk's segments, ((H(acc_d * dsc) * r) * svh_d) * row_weight,
    summed in row order (moe_e4m3.cu:2678-2719; variant 0 only)."""
    del grid
    if variant != 0:
        raise ValueError(f"down: unknown variant {variant}")
    _dev_tensor("a8d", a8d, torch.uint8, 2)
    _dev_tensor("dsc", dsc, torch.float32)
    _dev_tensor("row_token", row_token, torch.int64)
    _dev_tensor("row_weight", row_weight, torch.float32)
    if not out.is_cuda or out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be fp32 [T, K] with unit column stride")
    rows, N = a8d.shape
    T, K = out.shape
    if dsc.numel() < rows or row_token.numel() < rows or row_weight.numel() < rows:
        raise ValueError("down: dsc / row_token / row_weight [>= rows]")
    n = down_ptrs.numel()
    _ptr_table("down_ptrs", down_ptrs, n)
    _ptr_table("down_svh", down_svh, n)
    S = _segs(seg_expert, seg_row0, seg_rows, num_segs)
    ws = _stage_ws(out.device, rows, K, N, T)
    _lib.check("mi355moe_e4m3_down", _lib.lib().mi355moe_e4m3_down(
        ops._p(a8d), ops._p(dsc), rows, K, N, n, ops._p(down_ptrs), ops._p(down_svh), ops._p(out), T, out.stride(0),
        ops._p(row_token), ops._p(row_weight), ops._p(seg_expert), ops._p(seg_row0), ops._p(seg_rows), S,
        ops._p(num_segs), int(chunk), int(nchunks), ops._p(ws), ws.numel(), ops._stream(out.device)))


def fused(a8, asc, a8d, dsc, a16, out, gate_ptrs, up_ptrs, gate_svh, up_svh, down_ptrs, down_suh, down_svh, row_token,
          row_weight, seg_expert, seg_row0, seg_rows, num_segs, sync, limit, lag=12, grid=0, variant=0, *,
          intermediate: int | None = None) -> None:
    """Gate/up, the down input's per-row quantisation and the down GEMM of every segment, then out[token] += the
    token's rows in row order (moe_e4m3.cu:2721-2725; out fp32 or bf16). a8d / dsc and a16 receive the intermediates
    when given (a16 also gives the intermediate size, else `intermediate`). variant: TOKEN_ROWS (a8 / asc from
    gather_tok), DOWN16 (fp16 down operands; a8d / dsc not written), LEAN_MAINLOOP (accepted). Calls on the 256-row
    tiles with DOWN16 run gate/up and down as one ticket-ordered launch by themselves (lag: the environment variable
    MI355MOE_SCHED_LAG); the reference's per-call sync, lag and grid are accepted unused."""
    del sync, lag, grid
    N = int(intermediate) if intermediate else (int(a16.shape[1]) if a16 is not None else 0)
    if N <= 0:
        raise ValueError("fused(): pass a16 ([rows_cap, N]) or intermediate=N")
    _dev_tensor("a8", a8, torch.uint8, 2)
    _dev_tensor("asc", asc, torch.float32)
    _dev_tensor("row_token", row_token, torch.int64)
    _dev_tensor("row_weight", row_weight, torch.float32)
    if (a8d is None) != (dsc is None):
        raise ValueError("fused(): pass both a8d and dsc, or neither")
    rows = row_token.numel()
    T, K = out.shape
    tok_rows = bool(int(variant) & TOKEN_ROWS)
    if a8.shape[1] != K or a8.shape[0] < (T if tok_rows else rows) or asc.numel() < a8.shape[0]:
        raise ValueError("fused(): a8 uint8 [rows (or tokens with TOKEN_ROWS), K], asc [>= a8 rows]")
    if a8d is not None:
        _dev_tensor("a8d", a8d, torch.uint8, 2)
        _dev_tensor("dsc", dsc, torch.float32)
        if a8d.shape[0] < rows or a8d.shape[1] != N or dsc.numel() < rows:
            raise ValueError("fused(): a8d uint8 [rows, N], dsc [>= rows]")
    if a16 is not None:
        _dev_tensor("a16", a16, torch.float16, 2)
        if a16.shape[0] < rows or a16.shape[1] != N:
            raise ValueError("fused(): a16 fp16 [rows, N]")
    if row_weight.numel() < rows:
        raise ValueError("fused(): row_weight [>= rows]")
    out, od, ostr = _out_args(out, T)
    n = gate_ptrs.numel()
    for name, t in (("gate_ptrs", gate_ptrs), ("up_ptrs", up_ptrs), ("gate_svh", gate_svh), ("up_svh", up_svh),
                    ("down_ptrs", down_ptrs), ("down_suh", down_suh), ("down_svh", down_svh)):
        _ptr_table(name, t, n)
    S = _segs(seg_expert, seg_row0, seg_rows, num_segs)
    dev = out.device
    ws = _stage_ws(dev, rows, K, N, T)
    _lib.check("mi355moe_e4m3_fused", _lib.lib().mi355moe_e4m3_fused(
        ops._p(a8), ops._p(asc), a8.shape[0], ops._p(a8d), ops._p(dsc), ops._p(a16), ops._p(out), od, T, ostr, K, N, n,
        ops._p(gate_ptrs), ops._p(up_ptrs), ops._p(gate_svh), ops._p(up_svh), ops._p(down_ptrs), ops._p(down_suh),
        ops._p(down_svh), ops._p(row_token), ops._p(row_weight), rows, ops._p(seg_expert), ops._p(seg_row0),
        ops._p(seg_rows), S, ops._p(num_segs), float(limit), int(variant), ops._p(ws), ws.numel(), ops._stream(dev)))


def plan(ids: torch.Tensor, weights: torch.Tensor, n_exp: int, expert_map: torch.Tensor | None = None) -> dict:
    """The overlay's routing tables (glm53_moe_e4m3.py:450-477) from this library's device permutation, no host
    synchronisation: local ids by map_topk_to_local (n_exp for a pair with no local expert), the pairs grouped by
    local id in pair order with those pairs last (rows), and the segment tables over the local experts' rows."""
    T, topk = int(ids.shape[0]), int(ids.shape[1])
    P = T * topk
    dev = ids.device
    idc = ids.contiguous()
    wts = weights.reshape(T, topk).contiguous()
    em = None if expert_map is None else expert_map.to(torch.int64).contiguous()
    i32 = dict(dtype=torch.int32, device=dev)
    t = {"T": T, "topk": topk, "P": P, "n_exp": n_exp, "local": torch.empty(P, **i32), "pos": torch.empty(P, **i32),
         "row_token": torch.empty(P, dtype=torch.int64, device=dev),
         "row_weight": torch.empty(P, dtype=torch.float32, device=dev), "row_expert": torch.empty(P, **i32)}
    counts = torch.empty(n_exp + 1, dtype=torch.int64, device=dev)
    L = _lib.lib()
    ws = ops.workspace(dev, L.mi355moe_route_rows_workspace_bytes(P, n_exp))
    _lib.check("mi355moe_route_rows", L.mi355moe_route_rows(
        ops._p(idc), ops.ids_dtype_code(idc.dtype), ops._p(wts), ops.weight_dtype_code(wts.dtype), T, topk,
        ops._p(em), 0 if em is None else em.numel(), n_exp, ops._p(t["local"]), ops._p(t["pos"]),
        ops._p(t["row_token"]), ops._p(t["row_weight"]), ops._p(t["row_expert"]), ops._p(counts), ops._p(ws),
        ws.numel(), ops._stream(dev)))
    se, sr0, sr, ns, nr = seg_tables(counts[:n_exp], tile_rows(), P)
    t.update(counts=counts, seg_expert=se, seg_row0=sr0, seg_rows=sr, num_segs=ns, num_rows=nr)
    return t


def run(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts, limit: float,
        expert_map: torch.Tensor | None = None, out: torch.Tensor | None = None, keep: dict | None = None,
        sched: dict | None = None) -> torch.Tensor:
    """The routed experts of one EXL3 layer in e4m3 numerics for every token of x2d, through the overlay's own stage
    sequence (glm53_moe_e4m3.py:480-592): plan; gather_tok when every expert shares one w13 suh (else gather2),
    zeroing a new fp32 output; then fused, or with sched {"mode": "chunked", "nchunks": c} gateup, actq and down per
    chunk. Returns fp32 [T, K] (or adds into `out`, fp32 or bf16, without zeroing it). keep: a dict that receives
    the tables and the intermediate buffers (a8 as the per-row view the GEMMs read). experts: an mi355moe.Exl3Experts.
    sched {"down16": True} selects the fp16 down projection (fused only)."""
    sc = {"mode": "fused", "nchunks": 1, "down16": False}
    sc.update(sched or {})
    T = int(x2d.shape[0])
    dev = x2d.device
    t = plan(ids.reshape(T, -1), weights.reshape(T, -1), experts.n, expert_map)
    P, K, N = t["P"], experts.K, experts.N
    ptrs = experts.tables
    xc = x2d.contiguous()
    tok_rows = sc["mode"] == "fused" and bool(experts.uniform_suh)
    a8 = torch.empty(T if tok_rows else P, K, dtype=torch.uint8, device=dev)
    asc = torch.empty(a8.shape[0], dtype=torch.float32, device=dev)
    a8d = torch.empty(P, N, dtype=torch.uint8, device=dev)
    dsc = torch.empty(P, dtype=torch.float32, device=dev)
    a16 = torch.empty(P, N, dtype=torch.float16, device=dev)
    zero = out is None
    if zero:
        out = torch.empty(T, K, dtype=torch.float32, device=dev)
    if tok_rows:
        gather_tok(xc, ptrs["gate_suh"], a8, asc, out if zero else None)
    else:
        gather2(xc, t["local"], t["pos"], ptrs["gate_suh"], a8, asc, out if zero else None, t["topk"], experts.n)
    if sc["mode"] == "fused":
        variant = (TOKEN_ROWS if tok_rows else 0) | (DOWN16 if sc["down16"] else 0)
        fused(a8, asc, None if sc["down16"] else a8d, None if sc["down16"] else dsc, a16, out, ptrs["gate_trellis"],
              ptrs["up_trellis"], ptrs["gate_svh"], ptrs["up_svh"], ptrs["down_trellis"], ptrs["down_suh"],
              ptrs["down_svh"], t["row_token"], t["row_weight"], t["seg_expert"], t["seg_row0"], t["seg_rows"],
              t["num_segs"], None, limit, variant=variant)
    elif sc["mode"] == "chunked":
        if sc["down16"] or out.dtype != torch.float32:
            raise ValueError("the chunked schedule runs the e4m3 down into an fp32 output")
        nc = int(sc["nchunks"])
        for c in range(nc):
            gateup(a8, asc, ptrs["gate_trellis"], ptrs["up_trellis"], ptrs["gate_svh"], ptrs["up_svh"], a16,
                   t["seg_expert"], t["seg_row0"], t["seg_rows"], t["num_segs"], limit, 0, c, nc)
            actq(a16, t["row_expert"], ptrs["down_suh"], a8d, dsc, t["seg_row0"], t["seg_rows"], t["num_segs"], c, nc)
            down(a8d, dsc, ptrs["down_trellis"], ptrs["down_svh"], out, t["row_token"], t["row_weight"],
                 t["seg_expert"], t["seg_row0"], t["seg_rows"], t["num_segs"], 0, c, nc)
    else:
        raise ValueError(f"unknown schedule mode {sc['mode']!r}")
    if keep is not None:
        keep.update(t)
        rows_a8 = a8.index_select(0, t["row_token"]) if tok_rows else a8
        rows_asc = asc.index_select(0, t["row_token"]) if tok_rows else asc
        keep.update(a8=rows_a8, asc=rows_asc, a8d=a8d, dsc=dsc, a16=a16, tok_rows=tok_rows)
    return out
