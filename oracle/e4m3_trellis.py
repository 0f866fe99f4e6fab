"""Trellis-sourced e4m3 variant of the EXL3 experts on the CPU (oracle; test infrastructure only).

Restates code/fork/overlay/glm53_moe_e4m3.py:654-674 (spec_proj / spec_ffn with DOWN16 off) with the activation
quantiser of code/fork/kernels/moe_e4m3.cu:152-176 and :245-310 (gather2: fp32 product of the fp16 input and suh,
fp32 butterflies, r applied after the transform, s = amax / 448 by IEEE division, q = e4m3(clamp(v / s))):

  act_quant(x16, suh16)   (q values float32, s float32) per row
  weights_e4m3(trellis)   W_q of the 4-bit trellis (exl3.unpack) rounded to the nearest e4m3 value, float32
  forward(...)            routed output [T, K] in float64: per pair row q, s of the gate input (gate and up share
                          one suh), acc = q @ W8 summed in float64, g = H(acc * s) * svh (H scaled by 1/sqrt(128)),
                          a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (iff L != 0), the down input
                          v_d = fp32 butterflies of fp32(a16 * suh_d) times r, quantised per row as above, the down
                          GEMM likewise, y = H(acc_d * s_d) * svh_d, out[t] = sum of w * y in pair order.

  forward(..., down16=True)  the DOWN16 variant (spec_proj16, glm53_moe_e4m3.py:660-664): the down input
                          h = fp16(fp32 butterflies of fp32(a16 * suh_d) times r) times the fp16 W_q, float64 sums.

The extension's stage buffers (code/fork/kernels/moe_e4m3.cu:18-21 and :150-156, the k permutation of its e4m3 rows):
  STORAGE_PERM16          byte p of every 16-column group holds column STORAGE_PERM16[p]
  act_quant_codes(...)    the uint8 codes of act_quant in plain column order; to_storage / from_storage permute rows
  gateup_rows(...)        a16 from given quantised rows (q, s) of one expert: the stage's output in float64 sums
  down_rows(...)          y = H(qd @ W8 * sd) * svh_d of given quantised down rows, float64

Every step reuses a pinned piece: exl3.unpack (the codebook and tile order), exl3.fwht128_f32 (the butterfly
order), e4m3.encode_fast (OCP E4M3FN, pinned exhaustively against torch). The composition is checked in
tests/test_oracle_e4m3_trellis.py against closed-form properties and an independent torch statement of spec_ffn.
"""
from __future__ import annotations

import numpy as np

from . import e4m3, exl3

E4M3_MAX = np.float32(448.0)


# The extension's byte order inside each 16-column group of an e4m3 row (its mainloop's B-fragment k order).
STORAGE_PERM16 = np.array([0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15], np.int64)


def storage_columns(cols: int) -> np.ndarray:
    """The column held at each byte position of a stored row of `cols` e4m3 codes."""
    p = np.arange(cols)
    return (p // 16) * 16 + STORAGE_PERM16[p % 16]


def to_storage(rows: np.ndarray) -> np.ndarray:
    """Rows in plain column order -> the extension's stored order (last axis)."""
    return np.asarray(rows)[..., storage_columns(np.asarray(rows).shape[-1])]


def from_storage(rows: np.ndarray) -> np.ndarray:
    """Stored rows -> plain column order (last axis)."""
    rows = np.asarray(rows)
    out = np.empty_like(rows)
    out[..., storage_columns(rows.shape[-1])] = rows
    return out


def act_quant_codes(x16: np.ndarray, suh16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(uint8 e4m3 codes [rows, K] in plain column order, scales [rows] float32) of act_quant's rows."""
    q, s = act_quant(x16, suh16)
    return e4m3.encode_fast(q), s


def act_quant(x16: np.ndarray, suh16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(dequantisation-free e4m3 values q [rows, K] float32, row scales s [rows] float32) of
    v = fwht(fp32(x16) * fp32(suh16)) * r: s = amax|v| / 448 (1 if 0), q = e4m3(clamp(v / s, -448, 448))."""
    p = np.asarray(x16, np.float16).astype(np.float32) * np.asarray(suh16, np.float16).astype(np.float32)
    v = (exl3.fwht128_f32(p) * exl3.HAD_R).astype(np.float32)
    amax = np.abs(v).max(axis=-1).astype(np.float32)
    s = (amax / E4M3_MAX).astype(np.float32)
    s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
    r = np.clip((v / s[..., None]).astype(np.float32), -E4M3_MAX, E4M3_MAX)
    q = e4m3.decode(e4m3.encode_fast(r)).astype(np.float32)
    return q, s


def weights_e4m3(trellis: np.ndarray) -> np.ndarray:
    """The layer's W_q [K, N] (fp16 codebook sums) rounded to the nearest e4m3 values, as float32."""
    wq = exl3.unpack(trellis).astype(np.float32)
    return e4m3.decode(e4m3.encode_fast(wq)).astype(np.float32)


def _silu_act(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    if limit != 0.0:
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
    return g / (1.0 + np.exp(-g)) * u


def gateup_rows(q: np.ndarray, s: np.ndarray, trellis_g: np.ndarray, trellis_u: np.ndarray, svh_g: np.ndarray,
                svh_u: np.ndarray, limit: float) -> np.ndarray:
    """a16 fp16 [rows, N] of one expert from quantised gate/up input rows (values q, scales s): g = H(q @ W8_g * s)
    * svh_g (float64 sums of the exact e4m3 products), u likewise, fp16(silu(min(g, L)) * clamp(u, -L, L))
    (glm53_moe_e4m3.py:654-671, the gate/up stage of moe_e4m3.cu:4-9)."""
    s64 = np.asarray(s, np.float64)[:, None]
    q64 = np.asarray(q, np.float64)
    g = exl3.rotate_f64((q64 @ weights_e4m3(trellis_g).astype(np.float64)) * s64) * np.asarray(svh_g, np.float64)
    u = exl3.rotate_f64((q64 @ weights_e4m3(trellis_u).astype(np.float64)) * s64) * np.asarray(svh_u, np.float64)
    return _silu_act(g, u, limit).astype(np.float16)


def down_rows(qd: np.ndarray, sd: np.ndarray, trellis_d: np.ndarray, svh_d: np.ndarray) -> np.ndarray:
    """y float64 [rows, K] = H(qd @ W8_d * sd) * svh_d from quantised down input rows (moe_e4m3.cu:10)."""
    y = exl3.rotate_f64((np.asarray(qd, np.float64) @ weights_e4m3(trellis_d).astype(np.float64)) *
                        np.asarray(sd, np.float64)[:, None])
    return y * np.asarray(svh_d, np.float64)


def down16_rows(a16: np.ndarray, suh_d: np.ndarray, trellis_d: np.ndarray, svh_d: np.ndarray) -> np.ndarray:
    """The DOWN16 down projection (glm53_moe_e4m3.py:660-664): h = fp16(fwht(fp32(a16) * fp32(suh_d)) * r), y =
    H(h @ W_q) * svh_d with the fp16 W_q and float64 sums."""
    p = np.asarray(a16, np.float16).astype(np.float32) * np.asarray(suh_d, np.float16).astype(np.float32)
    h = (exl3.fwht128_f32(p) * exl3.HAD_R).astype(np.float32).astype(np.float16)
    y = exl3.rotate_f64(h.astype(np.float64) @ exl3.unpack(trellis_d).astype(np.float64))
    return y * np.asarray(svh_d, np.float64)


def forward(layer: dict, x16: np.ndarray, pair_token: np.ndarray, pair_expert: np.ndarray, pair_w: np.ndarray,
            limit: float, down16: bool = False) -> np.ndarray:
    """Routed output [T, K] float64. layer: numpy w13_trellis int16 [n,2,K/16,N/16,64], w13_suh fp16 [n,2,K] (gate
    and up equal), w13_svh fp16 [n,2,N], w2_trellis int16 [n,N/16,K/16,64], w2_suh fp16 [n,N], w2_svh fp16 [n,K];
    x16 fp16 [T, K]; pairs with expert < 0 are skipped. down16: the DOWN16 down projection."""
    x16 = np.asarray(x16, np.float16)
    T, K = x16.shape
    out = np.zeros((T, K), np.float64)
    tok = np.asarray(pair_token, np.int64)
    ex = np.asarray(pair_expert, np.int64)
    w = np.asarray(pair_w, np.float64)
    for e in np.unique(ex[ex >= 0]):
        rows = np.nonzero(ex == e)[0]
        q, s = act_quant(x16[tok[rows]], np.broadcast_to(layer["w13_suh"][e, 0], (rows.size, K)))
        a16 = gateup_rows(q, s, layer["w13_trellis"][e, 0], layer["w13_trellis"][e, 1], layer["w13_svh"][e, 0],
                          layer["w13_svh"][e, 1], limit)
        if down16:
            y = down16_rows(a16, np.broadcast_to(layer["w2_suh"][e], a16.shape), layer["w2_trellis"][e],
                            layer["w2_svh"][e])
        else:
            qd, sd = act_quant(a16, np.broadcast_to(layer["w2_suh"][e], a16.shape))
            y = down_rows(qd, sd, layer["w2_trellis"][e], layer["w2_svh"][e])
        np.add.at(out, tok[rows], w[rows, None] * y)
    return out
