"""The grouped fat-expert tier (E3) as the reference's production module drives it: the three stage entry points
on device-side row tables, the table builder and the apply that chains them.

  exl3_fat_moe_gather / _gateup / _down   the stage contract of code/fork/docs/ref/mia_exl3-fat-kernel/
                                          exl3_fat_moe.cuh:20-56 (same argument order and meaning)
  exl3_fat_moe_tile_rows_gateup / _down   the segment height the tables must be built with (this library's 256-row
                                          MFMA tiles, both stages)
  build_grouped_fat_tables                code/fork/docs/prod_exl3_reference.py:1316-1361: fat experts (count > cap)
                                          back to back in expert order, one segment per tile_rows rows, all on the
                                          device from capacity-sized tensors (no host synchronisation)
  apply_exl3_grouped_fat                  prod_exl3_reference.py:1364-1435: out (fp32) += the fat experts' output

h13 / h2 hold rows in this library's staging order (k permuted within 16-element groups): they are intermediates
from one stage to the next, not rotated activations in plain order. The down stage sums each token's rows in row
order and adds them to out (deterministic); its scratch comes from the device workspace (mi355moe.ops.workspace).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, ops


def exl3_fat_moe_tile_rows_gateup() -> int:
    return int(_lib.lib().mi355moe_e3_tile_rows())


def exl3_fat_moe_tile_rows_down() -> int:
    return int(_lib.lib().mi355moe_e3_tile_rows())


def _cuda_contig(name: str, t: torch.Tensor, dtype: torch.dtype | None = None) -> None:
    if not t.is_cuda or not t.is_contiguous() or (dtype is not None and t.dtype != dtype):
        raise ValueError(f"{name}: expected a contiguous CUDA tensor" + (f" of {dtype}" if dtype else ""))


def exl3_fat_moe_gather(x: torch.Tensor, row_token: torch.Tensor, row_expert: torch.Tensor, suh_ptrs: torch.Tensor,
                        h13: torch.Tensor, num_rows: torch.Tensor) -> None:
    """h13[row] = the rotated input x[row_token[row]] with expert row_expert[row]'s suh, rows < num_rows[0]."""
    for name, t, dt in (("row_token", row_token, torch.int64), ("row_expert", row_expert, torch.int32),
                        ("suh_ptrs", suh_ptrs, torch.int64), ("h13", h13, torch.float16),
                        ("num_rows", num_rows, torch.int32)):
        _cuda_contig(name, t, dt)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [tokens, K] with unit column stride")
    rows_cap, K = h13.shape
    if x.shape[1] != K or row_token.numel() < rows_cap or row_expert.numel() < rows_cap:
        raise ValueError("gather: x [tokens, K], row tables >= rows_cap, h13 [rows_cap, K]")
    _lib.check("mi355moe_e3_gather", _lib.lib().mi355moe_e3_gather(
        ops._p(x), ops.act_dtype_code(x.dtype), x.stride(0), x.shape[0], K, ops._p(row_token), ops._p(row_expert),
        rows_cap, suh_ptrs.numel(), ops._p(suh_ptrs), ops._p(h13), ops._p(num_rows), ops._stream(x.device)))


def exl3_fat_moe_gateup(h13: torch.Tensor, gate_ptrs: torch.Tensor, up_ptrs: torch.Tensor, gate_svh_ptrs: torch.Tensor,
                        up_svh_ptrs: torch.Tensor, down_suh_ptrs: torch.Tensor, h2: torch.Tensor,
                        seg_expert: torch.Tensor, seg_row0: torch.Tensor, seg_rows: torch.Tensor,
                        num_segs: torch.Tensor, act_limit: float) -> None:
    """h2 = the rotated down input of every segment's rows (gate/up GEMM, limit before SiLU, SwiGLU)."""
    for name, t in (("gate_ptrs", gate_ptrs), ("up_ptrs", up_ptrs), ("gate_svh_ptrs", gate_svh_ptrs),
                    ("up_svh_ptrs", up_svh_ptrs), ("down_suh_ptrs", down_suh_ptrs)):
        _cuda_contig(name, t, torch.int64)
    for name, t in (("seg_expert", seg_expert), ("seg_row0", seg_row0), ("seg_rows", seg_rows),
                    ("num_segs", num_segs)):
        _cuda_contig(name, t, torch.int32)
    _cuda_contig("h13", h13, torch.float16)
    _cuda_contig("h2", h2, torch.float16)
    rows_cap, K = h13.shape
    N = h2.shape[1]
    if h2.shape[0] < rows_cap or seg_row0.numel() < seg_expert.numel() or seg_rows.numel() < seg_expert.numel():
        raise ValueError("gateup: h2 [rows_cap, N] and segment tables of one length")
    _lib.check("mi355moe_e3_gateup", _lib.lib().mi355moe_e3_gateup(
        ops._p(h13), rows_cap, K, N, gate_ptrs.numel(), ops._p(gate_ptrs), ops._p(up_ptrs), ops._p(gate_svh_ptrs),
        ops._p(up_svh_ptrs), ops._p(down_suh_ptrs), ops._p(h2), ops._p(seg_expert), ops._p(seg_row0),
        ops._p(seg_rows), seg_expert.numel(), ops._p(num_segs), float(act_limit), ops._stream(h13.device)))


def exl3_fat_moe_down(h2: torch.Tensor, down_ptrs: torch.Tensor, down_svh_ptrs: torch.Tensor, out: torch.Tensor,
                      row_token: torch.Tensor, row_weight: torch.Tensor, seg_expert: torch.Tensor,
                      seg_row0: torch.Tensor, seg_rows: torch.Tensor, num_segs: torch.Tensor) -> None:
    """out[token] += the weighted down output of the token's rows (fp32 out, accumulated in row order)."""
    for name, t, dt in (("down_ptrs", down_ptrs, torch.int64), ("down_svh_ptrs", down_svh_ptrs, torch.int64),
                        ("out", out, torch.float32), ("row_token", row_token, torch.int64),
                        ("row_weight", row_weight, torch.float16), ("seg_expert", seg_expert, torch.int32),
                        ("seg_row0", seg_row0, torch.int32), ("seg_rows", seg_rows, torch.int32),
                        ("num_segs", num_segs, torch.int32), ("h2", h2, torch.float16)):
        _cuda_contig(name, t, dt)
    rows_cap, N = h2.shape
    tokens, K = out.shape
    if row_token.numel() < rows_cap or row_weight.numel() < rows_cap:
        raise ValueError("down: row tables must cover rows_cap rows")
    L = _lib.lib()
    nb = L.mi355moe_e3_down_workspace_bytes(rows_cap, K, tokens)
    ws = ops.workspace(out.device, nb)
    _lib.check("mi355moe_e3_down", L.mi355moe_e3_down(
        ops._p(h2), rows_cap, K, N, down_ptrs.numel(), ops._p(down_ptrs), ops._p(down_svh_ptrs), ops._p(out), tokens,
        out.stride(0), ops._p(row_token), ops._p(row_weight), ops._p(seg_expert), ops._p(seg_row0), ops._p(seg_rows),
        seg_expert.numel(), ops._p(num_segs), ops._p(ws), ws.numel(), ops._stream(out.device)))


def _excl_cumsum(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    inc = torch.cumsum(v, 0)
    return inc - v, inc


def build_grouped_fat_tables(counts: torch.Tensor, cap: int, token_sorted: torch.Tensor,
                             weight_sorted: torch.Tensor, rows_cap: int, tile_rows: int) -> dict:
    """Row and segment tables of the fat experts (code/fork/docs/prod_exl3_reference.py:1316-1361). counts int64 [n]
    (the sentinel bucket excluded): experts with more than cap rows are laid out back to back in expert order; row r
    of the fat-row buffer is sorted position sorted_off[e] + (r - row_off[e]) of its expert e; segment s covers
    tile_rows rows of one expert. Capacity-sized device tensors, no host synchronisation."""
    n = int(counts.numel())
    dev = counts.device
    fat = torch.where(counts > cap, counts, torch.zeros_like(counts))
    row_off, row_cum = _excl_cumsum(fat)
    sorted_off, _ = _excl_cumsum(counts)
    tiles = (fat + tile_rows - 1) // tile_rows
    tile_off, tile_cum = _excl_cumsum(tiles)
    max_segs = (rows_cap + tile_rows - 1) // tile_rows + n
    seg = torch.arange(max_segs, device=dev)
    se = torch.searchsorted(tile_cum, seg, right=True).clamp_(max=n - 1)
    local_tile = seg - tile_off[se]
    r = torch.arange(rows_cap, device=dev)
    re = torch.searchsorted(row_cum, r, right=True).clamp_(max=n - 1)
    src = (sorted_off[re] + (r - row_off[re])).clamp_(max=max(rows_cap - 1, 0))
    return {"seg_expert": se.to(torch.int32),
            "seg_row0": (row_off[se] + local_tile * tile_rows).to(torch.int32),
            "seg_rows": torch.clamp(fat[se] - local_tile * tile_rows, min=0, max=tile_rows).to(torch.int32),
            "num_segs": tile_cum[-1:].to(torch.int32), "num_rows": row_cum[-1:].to(torch.int32),
            "row_expert": re.to(torch.int32),
            "row_token": token_sorted.index_select(0, src), "row_weight": weight_sorted.index_select(0, src)}


def apply_exl3_grouped_fat(xh: torch.Tensor, out: torch.Tensor, counts: torch.Tensor, token_sorted: torch.Tensor,
                           weight_sorted: torch.Tensor, layer, cap: int, limit: float) -> None:
    """out (fp32 [T, K]) += every fat expert's routed output, three launches and no host synchronisation
    (code/fork/docs/prod_exl3_reference.py:1364-1435). `layer` carries the pointer tables as production's
    `_exl3_ptrs` dict, or is an mi355moe.Exl3Experts (its `tables`)."""
    ptrs = getattr(layer, "_exl3_ptrs", None) or getattr(layer, "tables")
    N = int(getattr(layer, "N", 0) or getattr(layer, "_exl3_intermediate_local"))
    dev = ptrs["gate_trellis"].device
    if xh.device != dev or out.device != dev or counts.device != dev:
        raise RuntimeError(f"EXL3 grouped tier: activations on {xh.device}, experts on {dev}")
    if not (xh.is_contiguous() and out.is_contiguous() and out.dtype == torch.float32):
        raise RuntimeError("EXL3 grouped tier needs contiguous fp16/bf16 input and fp32 output")
    rows_cap, K = int(token_sorted.numel()), int(xh.shape[1])
    tile = exl3_fat_moe_tile_rows_gateup()
    tg = build_grouped_fat_tables(counts, cap, token_sorted.contiguous(), weight_sorted.contiguous(), rows_cap, tile)
    h13 = torch.empty(rows_cap, K, dtype=torch.float16, device=dev)
    h2 = torch.empty(rows_cap, N, dtype=torch.float16, device=dev)
    exl3_fat_moe_gather(xh, tg["row_token"], tg["row_expert"], ptrs["gate_suh"], h13, tg["num_rows"])
    exl3_fat_moe_gateup(h13, ptrs["gate_trellis"], ptrs["up_trellis"], ptrs["gate_svh"], ptrs["up_svh"],
                        ptrs["down_suh"], h2, tg["seg_expert"], tg["seg_row0"], tg["seg_rows"], tg["num_segs"],
                        float(limit))
    exl3_fat_moe_down(h2, ptrs["down_trellis"], ptrs["down_svh"], out, tg["row_token"], tg["row_weight"],
                      tg["seg_expert"], tg["seg_row0"], tg["seg_rows"], tg["num_segs"])
