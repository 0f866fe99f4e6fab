"""e4m3 expert variant on the CPU (oracle; test infrastructure only).

The arithmetic lives in oracle/csrc/fp8.c (its header cites the reference file:line of every step); this module
loads it through oracle/moe.py's library and exposes:
  encode / decode      OCP float8 E4M3FN, round to nearest even, saturating at 448 (orc_e4m3_from_f32 / _to_f32)
  quant_rows           per-row dynamic quantisation: s = amax / 448 (1 if 0), q = e4m3(clamp(v / s))
                       (code/fork/kernels/moe_e4m3.cu:152-176, code/fork/overlay/glm53_moe_e4m3.py:648-652)
  block_quant          e4m3 weights with one fp32 scale per 128x128 block (the synthetic block-scaled experts)
  forward(..., mode)   routed output of one layer of block-scaled e4m3 experts: "kernel" = fp32 sums per 128-block
                       (the kernels' rounding points up to the order inside a block), "f64" = float64 sums from the
                       same quantised operands
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import moe

E4M3_MAX = 448.0


class _Fp8Layer(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int),
                ("w13", ctypes.c_void_p), ("w13s", ctypes.c_void_p), ("w2", ctypes.c_void_p), ("w2s", ctypes.c_void_p)]


_READY = False


def _lib() -> ctypes.CDLL:
    global _READY
    L = moe.lib()
    if not _READY:
        L.orc_e4m3_from_f32.restype = ctypes.c_uint8
        L.orc_e4m3_from_f32.argtypes = [ctypes.c_float]
        L.orc_e4m3_to_f32.restype = ctypes.c_float
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_quant_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_fp8_moe_forward.restype = ctypes.c_int
        L.orc_fp8_moe_forward.argtypes = [ctypes.POINTER(_Fp8Layer), ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        _READY = True
    return L


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def decode_table() -> np.ndarray:
    """float32 value of every e4m3 code [256] (NaN for 0x7F / 0xFF)."""
    L = _lib()
    return np.array([L.orc_e4m3_to_f32(b) for b in range(256)], np.float32)


def encode(v: np.ndarray) -> np.ndarray:
    """e4m3 codes (uint8) of float32 values, round to nearest even, saturating at +-448."""
    L = _lib()
    flat = np.ascontiguousarray(v, np.float32).ravel()
    out = np.fromiter((L.orc_e4m3_from_f32(float(f)) for f in flat), np.uint8, count=flat.size)
    return out.reshape(np.shape(v))


def decode(q: np.ndarray) -> np.ndarray:
    return decode_table()[np.asarray(q, np.uint8)]


def quant_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(q uint8 [rows, K], s float32 [rows]) of float32 rows."""
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.uint8)
    s = np.empty(rows, np.float32)
    _lib().orc_quant_rows(_p(x), rows, K, _p(q), _p(s))
    return q, s


def block_quant(w: np.ndarray, block: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """e4m3 codes and fp32 block scales of float32 matrices [..., R, C]: s = amax(block) / 448 (1 if 0), codes of
    clamp(w / s) -- the dequantised weight is decode(q) * s."""
    *lead, R, C = w.shape
    wb = w.reshape(*lead, R // block, block, C // block, block).astype(np.float32)
    amax = np.abs(wb).max(axis=(-3, -1))
    s = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
    v = np.clip(wb / s[..., :, None, :, None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    q = encode_fast(v).reshape(w.shape)
    return q, s


def encode_fast(v: np.ndarray) -> np.ndarray:
    """encode() for large arrays: nearest code by table search with ties to the even code (same result)."""
    tab = decode_table()
    codes = np.arange(256, dtype=np.uint8)
    ok = ~np.isnan(tab)
    vals, cds = tab[ok].astype(np.float64), codes[ok]
    order = np.argsort(vals, kind="stable")
    vals, cds = vals[order], cds[order]
    # drop -0 (keep +0 as the code for zero; the sign of a zero result follows the input below)
    keep = ~((vals == 0) & (cds == 0x80))
    vals, cds = vals[keep], cds[keep]
    x = np.clip(np.asarray(v, np.float64), -E4M3_MAX, E4M3_MAX)
    i = np.clip(np.searchsorted(vals, x), 1, len(vals) - 1)
    lo, hi = vals[i - 1], vals[i]
    dlo, dhi = x - lo, hi - x
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((cds[i] & 1) == 0))
    out = np.where(pick_hi, cds[i], cds[i - 1]).astype(np.uint8)
    zero = (out == 0) & np.signbit(x)
    return np.where(zero, np.uint8(0x80), out).astype(np.uint8)


def forward(layer: dict, x: np.ndarray, pair_token: np.ndarray, pair_expert: np.ndarray, pair_w: np.ndarray,
            limit: float, mode: str = "kernel", threads: int = 0) -> np.ndarray:
    """Routed output [T, K] (float32 for "kernel", float64 for "f64"), summed per token in pair order.
    layer: w13 uint8 [n, 2N, K], w13_scale float32 [n, 2N/128, K/128], w2 uint8 [n, K, N], w2_scale float32
    [n, K/128, N/128]; x float32 [T, K]."""
    w13 = np.ascontiguousarray(layer["w13"], np.uint8)
    w13s = np.ascontiguousarray(layer["w13_scale"], np.float32)
    w2 = np.ascontiguousarray(layer["w2"], np.uint8)
    w2s = np.ascontiguousarray(layer["w2_scale"], np.float32)
    n, N2, K = w13.shape
    N = N2 // 2
    L = _Fp8Layer(n, K, N, _p(w13), _p(w13s), _p(w2), _p(w2s))
    xx = np.ascontiguousarray(x, np.float32)
    T = xx.shape[0]
    tok = np.ascontiguousarray(pair_token, np.int32)
    ex = np.ascontiguousarray(pair_expert, np.int32)
    w = np.ascontiguousarray(pair_w, np.float32)
    m = {"kernel": 0, "f64": 1}[mode]
    if m == 1:
        out = np.zeros((T, K), np.float64)
        rc = _lib().orc_fp8_moe_forward(ctypes.byref(L), T, _p(xx), tok.size, _p(tok), _p(ex), _p(w), float(limit),
                                        m, None, _p(out), int(threads))
    else:
        out = np.zeros((T, K), np.float32)
        rc = _lib().orc_fp8_moe_forward(ctypes.byref(L), T, _p(xx), tok.size, _p(tok), _p(ex), _p(w), float(limit),
                                        m, _p(out), None, int(threads))
    if rc != 0:
        raise RuntimeError(f"orc_fp8_moe_forward failed: {rc}")
    return out


def pairs_fp32(local_ids: np.ndarray, weights: np.ndarray, n: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(token, local expert or -1, fp32 weight) per routed pair in (token, slot) order."""
    T, k = local_ids.shape
    tok = np.repeat(np.arange(T, dtype=np.int32), k)
    ex = local_ids.reshape(-1).astype(np.int64)
    ex = np.where((ex >= 0) & (ex < n), ex, -1).astype(np.int32)
    return tok, ex, np.asarray(weights, np.float32).reshape(-1)
