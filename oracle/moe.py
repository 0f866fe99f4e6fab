"""Routed-MoE forward of one EXL3 layer on the CPU (oracle; test infrastructure only).

The arithmetic lives in oracle/csrc/oracle.c (see its header for the reference file:line of every step); this
module loads it with ctypes and exposes:
  codebook_c / unpack_c   the C restatement of the EXL3 decode (cross-checked against oracle/exl3.py)
  forward(..., mode)      mode "decode"  : the decode kernels' rounding points (exl3_moe semantics: limit after SiLU)
                          mode "e3"      : the E3 prefill kernels' rounding points (limit before SiLU)
                          mode "f64"     : float64 reference, limit after SiLU (code/fork/tests/test_e2e_vs_f64.py:52-75)
                          mode "f64_pre" : float64 reference, limit before SiLU (code/fork/docs/prod_exl3_reference.py:961-1006)
                          mode "decode_x": "decode" with every weight fp16(lo) + fp16(hi) unrounded (the decode GEMV
                                           feeds both codebook halves to the matrix cores)
                          mode "tf_parity": the reference's default decode numerics (TF_PARITY=1,
                                           code/fork/kernels/exl3.cu:31-32, :351-496): fp16 roundings of the GEMV
                                           sums, fp16 svh / SiLU / limit / suh_d products, correctly rounded fp16
                                           exp and reciprocal in the SiLU
  silu_h / gateup_epilogue_tf / down_epilogue_tf   the "tf_parity" epilogues on their own
  pairs_from_routing      (token, local expert, fp16 weight) per routed pair, invalid ids skipped
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_LIB = None
MODES = {"decode": 0, "e3": 1, "f64": 2, "f64_pre": 3, "decode_x": 4, "tf_parity": 5}


class _Layer(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int),
                ("w13_trellis", ctypes.c_void_p), ("w13_suh", ctypes.c_void_p), ("w13_svh", ctypes.c_void_p),
                ("w2_trellis", ctypes.c_void_p), ("w2_suh", ctypes.c_void_p), ("w2_svh", ctypes.c_void_p)]


def build() -> str:
    """Compile the C oracle with its Makefile (needs gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        L.orc_h2f.restype = ctypes.c_float
        L.orc_h2f.argtypes = [ctypes.c_uint16]
        L.orc_f2h.restype = ctypes.c_uint16
        L.orc_f2h.argtypes = [ctypes.c_float]
        L.orc_d2h.restype = ctypes.c_uint16
        L.orc_d2h.argtypes = [ctypes.c_double]
        L.orc_codebook.argtypes = [ctypes.c_void_p]
        L.orc_codebook_exact.argtypes = [ctypes.c_void_p]
        L.orc_unpack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.orc_fwht128.argtypes = [ctypes.c_void_p]
        L.orc_rot_in.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.orc_expf_via_double.restype = ctypes.c_float
        L.orc_silu_h.restype = ctypes.c_float
        L.orc_silu_h.argtypes = [ctypes.c_float]
        L.orc_gateup_epilogue_tf.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
        L.orc_down_epilogue_tf.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint16, ctypes.c_int,
                                           ctypes.c_void_p]
        L.orc_gateup_epilogue.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                                                  ctypes.c_void_p]
        L.orc_down_epilogue.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint16, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_void_p]
        L.orc_expf_via_double.argtypes = [ctypes.c_float]
        L.orc_sigmoid_bits.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.orc_moe_forward.restype = ctypes.c_int
        L.orc_moe_forward.argtypes = [ctypes.POINTER(_Layer), ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        _LIB = L
    return _LIB


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def codebook_c() -> np.ndarray:
    out = np.empty(65536, np.uint16)
    lib().orc_codebook(_p(out))
    return out.view(np.float16)


def codebook_exact_c() -> np.ndarray:
    out = np.empty(65536, np.float32)
    lib().orc_codebook_exact(_p(out))
    return out


def unpack_c(trellis: np.ndarray) -> np.ndarray:
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    kt, nt = t.shape[0], t.shape[1]
    out = np.empty((kt * 16, nt * 16), np.uint16)
    lib().orc_unpack(_p(t), kt, nt, _p(out))
    return out.view(np.float16)


def fwht128_c(v: np.ndarray) -> np.ndarray:
    b = np.array(v, dtype=np.float32, copy=True).reshape(-1, 128)
    for r in range(b.shape[0]):
        row = np.ascontiguousarray(b[r])
        lib().orc_fwht128(_p(row))
        b[r] = row
    return b.reshape(np.shape(v))


def rot_in_c(x16: np.ndarray, suh16: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x16, np.float16)
    s = np.ascontiguousarray(np.broadcast_to(suh16, x.shape), np.float16)
    out = np.empty_like(x)
    xr, sr, orr = x.reshape(-1, x.shape[-1]), s.reshape(-1, x.shape[-1]), out.reshape(-1, x.shape[-1])
    for r in range(xr.shape[0]):
        lib().orc_rot_in(_p(xr[r:r + 1].view(np.uint16)), _p(sr[r:r + 1].view(np.uint16)), x.shape[-1],
                         _p(orr[r:r + 1].view(np.uint16)))
    return out


def silu_h(x16: np.ndarray) -> np.ndarray:
    """fp16 SiLU of the reference's default numerics, elementwise over fp16 values."""
    x = np.asarray(x16, np.float16).ravel()
    f = lib().orc_silu_h
    return np.array([f(float(v)) for v in x], np.float32).astype(np.float16).reshape(np.shape(x16))


def gateup_epilogue_tf(zg: np.ndarray, zu: np.ndarray, svh_g: np.ndarray, svh_u: np.ndarray, suh_d: np.ndarray,
                       limit: float) -> np.ndarray:
    """One pair row: fp32 GEMV sums zg / zu [N] -> the down GEMV's fp16 input [N] (exl3.cu:371-436, TF_PARITY=1)."""
    zg = np.ascontiguousarray(zg, np.float32)
    zu = np.ascontiguousarray(zu, np.float32)
    args = [np.ascontiguousarray(a, np.float16) for a in (svh_g, svh_u, suh_d)]
    N = zg.size
    if N % 128 or zu.size != N or any(a.size != N for a in args):
        raise ValueError("gateup_epilogue_tf: rows of one length, a multiple of 128")
    out = np.zeros(N, np.float16)
    lib().orc_gateup_epilogue_tf(_p(zg), _p(zu), *[_p(a) for a in args], N, float(limit), _p(out))
    return out


def down_epilogue_tf(zd: np.ndarray, svh_d: np.ndarray, w16) -> np.ndarray:
    """One pair row: fp32 down GEMV sums zd [K] -> the pair's fp32 contribution (exl3.cu:455-496, TF_PARITY=1)."""
    zd = np.ascontiguousarray(zd, np.float32)
    sv = np.ascontiguousarray(svh_d, np.float16)
    K = zd.size
    if K % 128 or sv.size != K:
        raise ValueError("down_epilogue_tf: rows of one length, a multiple of 128")
    out = np.zeros(K, np.float32)
    w = int(np.asarray(w16, np.float16).view(np.uint16))
    lib().orc_down_epilogue_tf(_p(zd), _p(sv), w, K, _p(out))
    return out


def gateup_epilogue(zg: np.ndarray, zu: np.ndarray, svh_g: np.ndarray, svh_u: np.ndarray, suh_d: np.ndarray,
                    limit: float, mode: str) -> np.ndarray:
    """One pair row of the kernel modes ("decode" / "decode_x": SiLU then the limit; "e3": the limit then SiLU):
    fp32 sums zg / zu [N] -> the down input fp16 [N] (orc_gateup_epilogue, the epilogue forward() runs)."""
    zg = np.array(zg, np.float32, copy=True)
    zu = np.array(zu, np.float32, copy=True)
    args = [np.ascontiguousarray(a, np.float16) for a in (svh_g, svh_u, suh_d)]
    N = zg.size
    if N % 128 or zu.size != N or any(a.size != N for a in args) or mode not in ("decode", "decode_x", "e3"):
        raise ValueError("gateup_epilogue: rows of one length (a multiple of 128), mode decode / decode_x / e3")
    out = np.zeros(N, np.float16)
    lib().orc_gateup_epilogue(_p(zg), _p(zu), *[_p(a) for a in args], N, float(limit), int(mode == "e3"), _p(out))
    return out


def down_epilogue(zd: np.ndarray, svh_d: np.ndarray, w16, mode: str) -> np.ndarray:
    """One pair row of the kernel modes: fp32 down sums zd [K] -> the pair's fp32 contribution (orc_down_epilogue)."""
    zd = np.array(zd, np.float32, copy=True)
    sv = np.ascontiguousarray(svh_d, np.float16)
    K = zd.size
    if K % 128 or sv.size != K or mode not in ("decode", "decode_x", "e3"):
        raise ValueError("down_epilogue: rows of one length (a multiple of 128), mode decode / decode_x / e3")
    out = np.zeros(K, np.float32)
    w = int(np.asarray(w16, np.float16).view(np.uint16))
    lib().orc_down_epilogue(_p(zd), _p(sv), w, K, int(mode == "e3"), _p(out))
    return out


def sigmoid_bits(first: int, n: int, threads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """(g, sigmoid(g)) float32 for the n floats whose bit patterns are first, first + 1, ...: the epilogues' sigmoid
    1 / (1 + (float)exp(-(double)g)) with IEEE float32 add and division, exp from the host's libm
    (exl3_fat_moe.cu:366-369)."""
    if n < 0 or first < 0 or first + n > 1 << 32:
        raise ValueError("sigmoid_bits: a range of 32-bit patterns")
    g = np.empty(n, np.float32)
    s = np.empty(n, np.float32)
    lib().orc_sigmoid_bits(int(first), int(n), _p(g), _p(s), int(threads))
    return g, s


def pairs_from_routing(local: np.ndarray, weights: np.ndarray, n: int, topk: int):
    """(token, expert, fp16 weight) of every routed pair j = t*topk + k in pair order; the sentinel (local id n)
    and invalid ids keep expert -1 so the forward skips them."""
    local = np.asarray(local, np.int64).reshape(-1)
    P = local.size
    tok = (np.arange(P) // topk).astype(np.int32)
    ex = np.where(local < n, local, -1).astype(np.int32)
    w16 = np.asarray(weights, np.float32).reshape(-1).astype(np.float16)
    return tok, ex, w16


def forward(layer: dict, x16: np.ndarray, pair_token: np.ndarray, pair_expert: np.ndarray, pair_w16: np.ndarray,
            limit: float, mode: str = "decode", threads: int = 0) -> np.ndarray:
    """Routed output [T, K] (float32 for the kernel and tf_parity modes, float64 for the f64 modes), summed per
    token in pair order. layer: numpy arrays w13_trellis int16 [n,2,K/16,N/16,64], w13_suh/w13_svh fp16 [n,2,K]/[n,2,N],
    w2_trellis int16 [n,N/16,K/16,64], w2_suh fp16 [n,N], w2_svh fp16 [n,K]."""
    arrs = {k: np.ascontiguousarray(layer[k]) for k in
            ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh", "w2_svh")}
    n, _, kt, nt, _ = arrs["w13_trellis"].shape
    K, N = kt * 16, nt * 16
    L = _Layer(n, K, N, *[_p(arrs[k]) for k in ("w13_trellis", "w13_suh", "w13_svh", "w2_trellis", "w2_suh",
                                                  "w2_svh")])
    x = np.ascontiguousarray(x16, np.float16)
    T = x.shape[0]
    tok = np.ascontiguousarray(pair_token, np.int32)
    ex = np.ascontiguousarray(pair_expert, np.int32)
    w = np.ascontiguousarray(pair_w16, np.float16)
    m = MODES[mode]
    if m in (2, 3):
        out = np.zeros((T, K), np.float64)
        rc = lib().orc_moe_forward(ctypes.byref(L), T, _p(x), tok.size, _p(tok), _p(ex), _p(w), float(limit), m,
                                   None, _p(out), int(threads))
    else:
        out = np.zeros((T, K), np.float32)
        rc = lib().orc_moe_forward(ctypes.byref(L), T, _p(x), tok.size, _p(tok), _p(ex), _p(w), float(limit), m,
                                   _p(out), None, int(threads))
    if rc != 0:
        raise RuntimeError(f"orc_moe_forward failed: {rc}")
    return out
