"""OCP 8-bit floating point E4M3 ("float8_e4m3fn") encoder written from the format spec (TEST ORACLE).

Format (OCP 8-bit Floating Point Specification, v1.0, E4M3): 1 sign bit, 4
exponent bits with bias 7, 3 mantissa bits; no infinities; S.1111.111 is NaN,
so the largest finite magnitude is 1.75 * 2**8 = 448. Exponent field 0 holds
subnormals m/8 * 2**-6. Rounding is to nearest, ties to even.

The reference relies on torch's ``.to(torch.float8_e4m3fn)`` (quant.py:83, 98),
always after clamping to +-448; this encoder pins that cast independently.
"""

from __future__ import annotations

import numpy as np


def encode(x: np.ndarray) -> np.ndarray:
    """float32/float64 values already clamped to [-448, 448] -> uint8 e4m3fn codes."""
    x = np.asarray(x, dtype=np.float64)
    if np.any(np.abs(x) > 448.0) or np.any(~np.isfinite(x)):
        raise ValueError("encode expects finite values clamped to [-448, 448]")
    sign = (np.signbit(x)).astype(np.uint8) << 7
    a = np.abs(x)
    out = np.zeros(a.shape, dtype=np.uint8)
    # subnormal range: a < 2**-6 -> m = rint(a / 2**-9), m in 0..8 (8 == smallest normal 0x08)
    sub = a < 2.0 ** -6
    m_sub = np.rint(a[sub] * 2.0 ** 9).astype(np.int64)  # exact scaling by a power of two
    out[sub] = m_sub.astype(np.uint8)  # code (0<<3)|m, and m == 8 encodes exponent 1, mantissa 0
    nrm = ~sub
    an = a[nrm]
    e = np.floor(np.log2(an)).astype(np.int64)
    # guard log2 rounding at exact powers of two
    e = np.where(2.0 ** e > an, e - 1, e)
    e = np.where(2.0 ** (e + 1) <= an, e + 1, e)
    frac = an / 2.0 ** e  # in [1, 2), exact
    m = np.rint((frac - 1.0) * 8.0).astype(np.int64)  # 0..8, ties to even
    carry = m == 8
    m = np.where(carry, 0, m)
    e = np.where(carry, e + 1, e)
    code = ((e + 7) << 3) | m
    if np.any(code > 0x7E):
        raise AssertionError("value rounded past 448")
    out[nrm] = code.astype(np.uint8)
    return out | sign


def decode(code: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float64 values (NaN for 0x7F / 0xFF)."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return s * val
