"""EXL3 4-bit trellis format, numpy restatement (oracle; test infrastructure only).

Follows code/fork/kernels/exl3_format_ref.py:13-27 (the closed form) and :47-131 (codebook, tile positions,
states, unpack, Hadamard, rotate). A linear layer with K inputs and N outputs is trellis int16 [K/16, N/16, 64]
(16x16 tiles, row-major over tiles), suh fp16 [K], svh fp16 [N]; the layer computes
y = ((((x * suh) @ H_K) @ W_q) @ H_N) * svh with H the 128-point Sylvester Hadamard scaled by 1/sqrt(128).
"""
from __future__ import annotations

import functools

import numpy as np

MCG = 0xCBAC1FED            # exl3_format_ref.py:41; code/fork/docs/prod_exl3_reference.py:50
MASK = 0x8FFF8FFF           # exl3_format_ref.py:42
FLIP = 0x3B603B60           # exl3_format_ref.py:43
MCG_MARKER = -877912083     # the int32 view of MCG, prod_exl3_reference.py:51
HAD = 128
HAD_R = np.float32(0.088388347648)   # 1/sqrt(128) as fp32, code/fork/kernels/exl3.cu:37-39


@functools.lru_cache(maxsize=1)
def codebook() -> np.ndarray:
    """fp16 value of every 16-bit state [65536] (exl3_format_ref.py:47-56): x = s*MCG mod 2^32,
    x = (x & MASK) ^ FLIP, value = fp16(lo) + fp16(hi) rounded once (the float64 sum is exact)."""
    s = np.arange(1 << 16, dtype=np.uint64)
    x = ((s * np.uint64(MCG)) & np.uint64(0xFFFFFFFF))
    x = (x & np.uint64(MASK)) ^ np.uint64(FLIP)
    lo = (x & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    return (lo + hi).astype(np.float16)


@functools.lru_cache(maxsize=1)
def codebook_exact() -> np.ndarray:
    """fp16(lo) + fp16(hi) of every state as float64 without the final fp16 rounding: the weight the decode GEMV's
    matrix cores see when they take both halves as operands (exactly representable in float32)."""
    s = np.arange(1 << 16, dtype=np.uint64)
    x = ((s * np.uint64(MCG)) & np.uint64(0xFFFFFFFF))
    x = (x & np.uint64(MASK)) ^ np.uint64(FLIP)
    lo = (x & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    return lo + hi


@functools.lru_cache(maxsize=1)
def tile_order() -> tuple[np.ndarray, np.ndarray]:
    """(row, col) inside its 16x16 tile of stream value p = 0..255 (exl3_format_ref.py:22-23, :59-67)."""
    p = np.arange(256)
    word, j = p >> 3, p & 7
    row = 2 * (word & 3) + (j & 1) + 8 * ((j >> 1) & 1)
    col = (word >> 2) + 8 * (j >> 2)
    return row, col


def tile_words(trellis: np.ndarray) -> np.ndarray:
    """int16 [..., 64] -> uint32 [..., 32]: the 64 int16 of a tile read as 32 little-endian 32-bit words."""
    t = np.ascontiguousarray(trellis)
    if t.dtype != np.int16 or t.shape[-1] != 64:
        raise ValueError(f"trellis must be int16 [..., 64] (4 bits), got {t.dtype} {t.shape}")
    u = t.view(np.uint16).astype(np.uint32)
    return u[..., 0::2] | (u[..., 1::2] << np.uint32(16))


def states(trellis: np.ndarray) -> np.ndarray:
    """16-bit state of every value [..., 256] (exl3_format_ref.py:70-85). Value p of a tile is the 16 stream bits
    that end at bit 4p+4 of the tile's circular 1024-bit stream, read MSB-first from each 32-bit word; word l holds
    stream bits 32l..32l+31, so value 8l+j is bits 28-4j..43-4j of the 64-bit pair (word l-1, word l)."""
    w = tile_words(trellis).astype(np.uint64)
    prev = np.roll(w, 1, axis=-1)                                  # word l-1, circular
    pair = (prev << np.uint64(32)) | w                             # [..., 32]
    shifts = (28 - 4 * np.arange(8)).astype(np.uint64)            # j = 0..7
    s = (pair[..., :, None] >> shifts) & np.uint64(0xFFFF)         # [..., 32, 8]
    return s.reshape(s.shape[:-2] + (256,)).astype(np.uint32)


def unpack(trellis: np.ndarray) -> np.ndarray:
    """W_q fp16 [K, N] from trellis int16 [K/16, N/16, 64] (exl3_format_ref.py:88-97)."""
    st = states(trellis)                                           # [kt, nt, 256]
    kt, nt = st.shape[0], st.shape[1]
    vals = codebook()[st]                                          # [kt, nt, 256]
    row, col = tile_order()
    w = np.empty((kt, nt, 16, 16), dtype=np.float16)
    w[:, :, row, col] = vals
    return np.ascontiguousarray(w.transpose(0, 2, 1, 3)).reshape(kt * 16, nt * 16)


@functools.lru_cache(maxsize=4)
def sylvester(n: int = HAD) -> np.ndarray:
    """n x n Sylvester Hadamard of +-1 (exl3_format_ref.py:100-106): H[i, j] = (-1)^popcount(i & j)."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def fwht128_f32(v: np.ndarray) -> np.ndarray:
    """fp32 Walsh-Hadamard of every 128-block of the last axis, butterfly strides 1, 2, ..., 64 in that order
    (exl3.cu:273-284; the order fixes every fp32 rounding). Returns a new float32 array."""
    v = np.array(v, dtype=np.float32, copy=True)
    if v.shape[-1] % HAD:
        raise ValueError("last axis must be a multiple of 128")
    shp = v.shape
    b = v.reshape(-1, HAD)
    idx = np.arange(HAD)
    s = 1
    while s < HAD:
        lo = idx[(idx & s) == 0]
        hi = lo + s
        a, c = b[:, lo].copy(), b[:, hi].copy()
        b[:, lo] = a + c
        b[:, hi] = a - c
        s <<= 1
    return b.reshape(shp)


def rotate_f64(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """H / sqrt(128) on every 128-block along ``axis`` in float64 (exl3_format_ref.py:109-116)."""
    h = sylvester() / np.sqrt(HAD)
    x = np.moveaxis(np.asarray(x, dtype=np.float64), axis, -1)
    shp = x.shape
    y = (x.reshape(shp[:-1] + (shp[-1] // HAD, HAD)) @ h).reshape(shp)
    return np.moveaxis(y, -1, axis)


def rot_in(x16: np.ndarray, suh16: np.ndarray) -> np.ndarray:
    """fp16(H(fp16(x * suh)) * r) row-wise (exl3.cu:321-349 with TF_PARITY; xl_hadamard_inner.cuh:91-131):
    the fp16 x fp16 product is exact in fp32 and rounded once to fp16; the butterfly runs in fp32."""
    p = (x16.astype(np.float32) * suh16.astype(np.float32)).astype(np.float16).astype(np.float32)
    return (fwht128_f32(p) * HAD_R).astype(np.float16)


def linear_f64(x: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray) -> np.ndarray:
    """y = ((((x*suh) H) W_q) H) * svh in float64 (exl3_format_ref.py:127-131)."""
    xh = rotate_f64(np.asarray(x, np.float64) * suh.astype(np.float64), -1)
    return rotate_f64(xh @ unpack(trellis).astype(np.float64), -1) * svh.astype(np.float64)
