"""The grouped fat-expert tier (E3) as the reference's production module drives it: the three stage entry points
on device-side row tables, the table builder and the apply that chains them.

  exl3_fat_moe_gather / _gateup / _down   the stage contract of code/fork/docs/ref/mia_exl3-fat-kernel/
                                          exl3_fat_moe.cuh:20-56 (same argument order and meaning)
  exl3_fat_moe_tile_rows_gateup / _down   the segment height the tables must be built with (this library's 256-row
                                          MFMA tiles, both stages)
  build_grouped_fat_tables                the table contract of code/fork/docs/prod_exl3_reference.py:1316-1361,
                                          built by this library's device kernels (mi355moe_e3_fat_tables)
  apply_exl3_grouped_fat                  the contract of prod_exl3_reference.py:1364-1435: out (fp32) += the fat
                                          experts' output, tables then the three stages, no host synchronisation

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


def build_grouped_fat_tables(counts: torch.Tensor, cap: int, token_sorted: torch.Tensor,
                             weight_sorted: torch.Tensor, rows_cap: int, tile_rows: int) -> dict:
    """The fat experts' row and segment tables, built on the device by mi355moe_e3_fat_tables (the table contract of
    code/fork/docs/prod_exl3_reference.py:1316-1361). counts int64 [n] (sentinel bucket excluded) of the pairs
    sorted by expert (token_sorted int64, weight_sorted fp16, rows_cap entries): the experts with more than cap
    pairs, back to back in expert order; segments of at most tile_rows rows. Returns the device tensors seg_expert /
    seg_row0 / seg_rows (int32 [ceil(rows_cap / tile_rows) + n]), num_segs / num_rows (int32 [1]), row_expert (int32
    [rows_cap], -1 past num_rows), row_token (int64) and row_weight (fp16); nothing is read back to the host."""
    if not counts.is_cuda or counts.dtype != torch.int64 or counts.dim() != 1:
        raise ValueError("counts must be an int64 CUDA vector of per-expert pair counts")
    n = int(counts.numel())
    dev = counts.device
    cnt = counts.contiguous()
    tok = token_sorted.to(torch.int64).contiguous()
    wts = weight_sorted.to(torch.float16).contiguous()
    if tok.numel() < rows_cap or wts.numel() < rows_cap:
        raise ValueError("token_sorted / weight_sorted must hold rows_cap entries")
    max_segs = (rows_cap + tile_rows - 1) // tile_rows + n
    i32 = dict(dtype=torch.int32, device=dev)
    t = {"seg_expert": torch.empty(max_segs, **i32), "seg_row0": torch.empty(max_segs, **i32),
         "seg_rows": torch.empty(max_segs, **i32), "num_segs": torch.empty(1, **i32),
         "num_rows": torch.empty(1, **i32), "row_expert": torch.empty(max(rows_cap, 1), **i32),
         "row_token": torch.empty(max(rows_cap, 1), dtype=torch.int64, device=dev),
         "row_weight": torch.empty(max(rows_cap, 1), dtype=torch.float16, device=dev)}
    scratch = torch.empty(2 * n, **i32)
    _lib.check("mi355moe_e3_fat_tables", _lib.lib().mi355moe_e3_fat_tables(
        ops._p(cnt), n, int(cap), ops._p(tok), ops._p(wts), int(rows_cap), int(tile_rows), ops._p(t["seg_expert"]),
        ops._p(t["seg_row0"]), ops._p(t["seg_rows"]), max_segs, ops._p(t["num_segs"]), ops._p(t["num_rows"]),
        ops._p(t["row_expert"]), ops._p(t["row_token"]), ops._p(t["row_weight"]), ops._p(scratch), ops._stream(dev)))
    return t


def apply_exl3_grouped_fat(xh: torch.Tensor, out: torch.Tensor, counts: torch.Tensor, token_sorted: torch.Tensor,
                           weight_sorted: torch.Tensor, layer, cap: int, limit: float) -> None:
    """Adds every fat expert's (more than cap pairs) routed output to out (fp32 [T, K]): device tables, then the
    gather, gate/up and down stages; no host synchronisation (the contract of code/fork/docs/
    prod_exl3_reference.py:1364-1435). `layer` carries the pointer tables as production's `_exl3_ptrs` dict, or is an
    mi355moe.Exl3Experts (its `tables`)."""
    ptrs = getattr(layer, "_exl3_ptrs", None) or getattr(layer, "tables")
    N = int(getattr(layer, "N", 0) or getattr(layer, "_exl3_intermediate_local"))
    dev = ptrs["gate_trellis"].device
    for name, t in (("xh", xh), ("out", out), ("counts", counts)):
        if t.device != dev:
            raise RuntimeError(f"grouped fat tier: {name} is on {t.device} but the experts' tables are on {dev}")
    if out.dtype != torch.float32 or not out.is_contiguous() or not xh.is_contiguous():
        raise RuntimeError("grouped fat tier: out must be contiguous fp32 and xh contiguous fp16 / bf16")
    rows, K = int(token_sorted.numel()), int(xh.shape[1])
    tabs = build_grouped_fat_tables(counts, cap, token_sorted, weight_sorted, rows,
                                    exl3_fat_moe_tile_rows_gateup())
    h13 = torch.empty(rows, K, dtype=torch.float16, device=dev)
    h2 = torch.empty(rows, N, dtype=torch.float16, device=dev)
    segs = (tabs["seg_expert"], tabs["seg_row0"], tabs["seg_rows"], tabs["num_segs"])
    exl3_fat_moe_gather(xh, tabs["row_token"], tabs["row_expert"], ptrs["gate_suh"], h13, tabs["num_rows"])
    exl3_fat_moe_gateup(h13, ptrs["gate_trellis"], ptrs["up_trellis"], ptrs["gate_svh"], ptrs["up_svh"],
                        ptrs["down_suh"], h2, *segs, float(limit))
    exl3_fat_moe_down(h2, ptrs["down_trellis"], ptrs["down_svh"], out, tabs["row_token"], tabs["row_weight"], *segs)
