"""Pins the EXL3 part of the oracle (oracle/exl3.py, oracle/csrc/oracle.c) against checks that do not restate it:
Python's own binary16 rounding, a bit-by-bit stream reader, the PTX m16n8k16 fragment layout, known constants,
and float64 matrix forms of the Hadamard and of the layer."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import exl3, moe


def _half_bits_py(x: float) -> int:
    """IEEE binary16 bits of x rounded to nearest even by CPython's own packer (struct 'e')."""
    return struct.unpack("<H", struct.pack("<e", x))[0]


def _half_value_py(bits: int) -> float:
    return struct.unpack("<e", struct.pack("<H", bits))[0]


def test_codebook_exhaustive_vs_python_integers():
    cb = exl3.codebook().view(np.uint16)
    for s in range(65536):
        x = (s * 0xCBAC1FED) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        v = _half_value_py(x & 0xFFFF) + _half_value_py(x >> 16)       # exact in Python float (double)
        assert cb[s] == _half_bits_py(v), s


def test_codebook_c_equals_numpy_and_known_answers():
    assert np.array_equal(moe.codebook_c().view(np.uint16), exl3.codebook().view(np.uint16))
    cbf = exl3.codebook().astype(np.float64)
    assert np.abs(cbf).max() == 3.94921875          # "max |v| 3.949", code/fork/kernels/moe_e4m3.cu:13-14
    assert np.int32(np.uint32(exl3.MCG)) == exl3.MCG_MARKER  # prod_exl3_reference.py:50-51
    assert abs(cbf.mean()) < 0.05 and 0.5 < cbf.std() < 2.0


def test_exact_codebook_sums_vs_python_integers():
    """The unrounded lo + hi sums (what the decode GEMV's matrix cores add): equal in C and numpy, exactly
    representable in float32, every one rounding to the pinned fp16 codebook, and equal to Python's own sums."""
    ex = exl3.codebook_exact()
    exc = moe.codebook_exact_c()
    assert np.array_equal(exc.astype(np.float64), ex)
    assert np.array_equal(ex.astype(np.float32).astype(np.float64), ex)
    assert np.array_equal(ex.astype(np.float16).view(np.uint16), exl3.codebook().view(np.uint16))
    for s in list(range(0, 65536, 97)) + [0, 1, 0x7FFF, 0x8000, 0xFFFF]:
        x = (s * 0xCBAC1FED) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        assert ex[s] == _half_value_py(x & 0xFFFF) + _half_value_py(x >> 16), s
    assert np.any(ex != exl3.codebook().astype(np.float64))          # the rounding is not a no-op


def test_tile_order_is_the_ptx_b_fragment_layout():
    # PTX ISA, mma.m16n8k16 (.f16): B is 16x8; lane L holds b0,b1 at rows 2*(L%4)+{0,1} and b2,b3 at rows
    # 2*(L%4)+8+{0,1}, column L/4. A tile's lane decodes two n8 halves: values j=0..3 -> first half,
    # j=4..7 -> second half (column + 8).
    row, col = exl3.tile_order()
    for p in range(256):
        L, j = divmod(p, 8)
        half, r = divmod(j, 4)
        exp_row = 2 * (L % 4) + (r % 2) + 8 * (r // 2)
        exp_col = L // 4 + 8 * half
        assert (row[p], col[p]) == (exp_row, exp_col)
    assert len(set(zip(row.tolist(), col.tolist()))) == 256


def _states_bitstream(tile: np.ndarray) -> list[int]:
    """States read bit by bit: the tile's 1024-bit circular stream is its 32 little-endian words, MSB first."""
    words = [int(tile[2 * i]) & 0xFFFF | ((int(tile[2 * i + 1]) & 0xFFFF) << 16) for i in range(32)]
    bits = "".join(format(w, "032b") for w in words)
    out = []
    for p in range(256):
        end = 4 * p + 4
        s = "".join(bits[(b + 1024) % 1024] for b in range(end - 16, end))
        out.append(int(s, 2))
    return out


def test_states_vs_bitstream_reader():
    rng = np.random.default_rng(7)
    t = rng.integers(-32768, 32768, size=(3, 2, 64), dtype=np.int16)
    st = exl3.states(t)
    for a in range(3):
        for b in range(2):
            assert st[a, b].tolist() == _states_bitstream(t[a, b])


def test_unpack_numpy_equals_c_and_brute_force():
    rng = np.random.default_rng(3)
    t = rng.integers(-32768, 32768, size=(8, 16, 64), dtype=np.int16)
    wn = exl3.unpack(t)
    wc = moe.unpack_c(t)
    assert np.array_equal(wn.view(np.uint16), wc.view(np.uint16))
    cb = exl3.codebook()
    row, col = exl3.tile_order()
    for a, b in [(0, 0), (7, 15), (3, 9)]:
        st = _states_bitstream(t[a, b])
        for p in range(256):
            assert wn[a * 16 + row[p], b * 16 + col[p]].view(np.uint16) == cb[st[p]].view(np.uint16)


def test_fwht_matches_sylvester_and_is_exact_on_integers():
    h = exl3.sylvester()
    assert np.array_equal(h @ h, 128 * np.eye(128))
    for i in (0, 1, 5, 77, 127):
        for j in (0, 3, 64, 127):
            assert h[i, j] == (-1) ** bin(i & j).count("1")
    rng = np.random.default_rng(1)
    iv = rng.integers(-1000, 1000, size=(4, 256)).astype(np.float32)      # sums stay exact in fp32
    got = exl3.fwht128_f32(iv).astype(np.float64)
    ref = (iv.astype(np.float64).reshape(4, 2, 128) @ h).reshape(4, 256)
    assert np.array_equal(got, ref)
    fv = rng.standard_normal((4, 256)).astype(np.float32)
    got = exl3.fwht128_f32(fv).astype(np.float64)
    ref = (fv.astype(np.float64).reshape(4, 2, 128) @ h).reshape(4, 256)
    assert np.max(np.abs(got - ref)) < 1e-4
    assert np.array_equal(exl3.fwht128_f32(fv), moe.fwht128_c(fv))


def test_fwht_butterfly_order_is_strides_1_to_64():
    # a plausible mistake (strides 64..1) gives the same math but other fp32 roundings; pin the order on values
    # whose sums round differently: evaluate the documented order with explicit Python fp32 steps
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(128) * np.float32(1e4)).astype(np.float32)
    w = [np.float32(a) for a in v]
    s = 1
    while s < 128:
        for i in range(0, 128, 2 * s):
            for k in range(i, i + s):
                a, b = w[k], w[k + s]
                w[k], w[k + s] = np.float32(a + b), np.float32(a - b)
        s *= 2
    assert np.array_equal(np.array(w, np.float32), exl3.fwht128_f32(v))


def test_rot_in_numpy_c_equal_and_close_to_f64():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 512)).astype(np.float16)
    s = (np.sign(rng.standard_normal(512)) * (1 + 0.25 * rng.random(512))).astype(np.float16)
    a = exl3.rot_in(x, s)
    b = moe.rot_in_c(x, s)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    p = (x.astype(np.float32) * s.astype(np.float32)).astype(np.float16).astype(np.float64)
    ref = exl3.rotate_f64(p, -1)
    assert np.max(np.abs(a.astype(np.float64) - ref)) <= 2e-3 * np.max(np.abs(ref))


def test_linear_f64_equals_explicit_dequantized_matrix():
    rng = np.random.default_rng(5)
    K, N = 256, 128
    t = rng.integers(-32768, 32768, size=(K // 16, N // 16, 64), dtype=np.int16)
    suh = rng.standard_normal(K).astype(np.float16)
    svh = rng.standard_normal(N).astype(np.float16)
    x = rng.standard_normal((3, K))
    h = exl3.sylvester() / np.sqrt(128)
    hk = np.kron(np.eye(K // 128), h)
    hn = np.kron(np.eye(N // 128), h)
    W = np.diag(suh.astype(np.float64)) @ hk @ exl3.unpack(t).astype(np.float64) @ hn @ np.diag(
        svh.astype(np.float64))
    assert np.allclose(exl3.linear_f64(x, t, suh, svh), x @ W, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("v", [0.0, -0.0, 1.0, 65504.0, 65519.9, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9, -3.14159, 0.1])
def test_c_fp16_rounding_matches_python(v):
    f = float(np.float32(v))
    assert moe.lib().orc_f2h(f) == _half_bits_py(f)


def test_c_fp16_rounding_overflow_and_random():
    assert moe.lib().orc_f2h(65520.0) == 0x7C00 and moe.lib().orc_f2h(-1e6) == 0xFC00
    rng = np.random.default_rng(9)
    for v in (rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 5, 3000)).astype(np.float32):
        f = float(v)
        if abs(f) < 65504:
            assert moe.lib().orc_f2h(f) == _half_bits_py(f), f
