"""CPU: the arithmetic identities the quantize kernels rely on, checked exhaustively in numpy.

1. RN32(RN64(x * RN64(1 / s))) == RN32(x / s): the kernels form the double reciprocal of the row scale
   once and multiply, instead of an fp32 division per element (quant.py:100 divides).
2. clamp(v, -127, 127) + 1.5 * 2^23 leaves clamp(rint(v), -127, 127) in the low byte of the float bits
   (torch.round is half-to-even; quant.py:100 rounds, then clamps).
"""

from __future__ import annotations

import numpy as np


def _all_bf16_values() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    return v[np.isfinite(v)]


def _scales(rng) -> np.ndarray:
    s = [np.float32(1.0), np.float32(2.0 ** -20), np.float32(1e-12) / np.float32(127.0),
         np.float32(1e-12) / np.float32(448.0)]
    # mantissas of all ones and of one, across binades
    for e in range(-40, 40, 3):
        s.append(np.float32(2.0 ** e) * np.float32(1.9999999))
        s.append(np.float32(2.0 ** e) * np.float32(1.0000001))
    # amax / 127 and amax / 448 for amax drawn from every binade of bf16 and fp32
    amax = np.concatenate([np.abs(_all_bf16_values()[::37]), rng.uniform(1e-6, 1e6, 2000).astype(np.float32)])
    amax = amax[amax > 1e-12]
    s.extend((amax / np.float32(127.0)).astype(np.float32))
    s.extend((amax[::7] / np.float32(448.0)).astype(np.float32))
    return np.array(s, dtype=np.float32)


def test_double_reciprocal_product_equals_fp32_division():
    rng = np.random.default_rng(0)
    xs = _all_bf16_values()
    # plus random fp32 bit patterns (fp32 activations)
    xf = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    xf = xf[np.isfinite(xf)]
    scales = _scales(rng)
    checked = 0
    with np.errstate(over="ignore", under="ignore"):
        for x in (xs, xf):
            for s in scales[::1 if x is xs else 5]:
                want = x / s                                     # fp32 / fp32: correctly rounded
                rd = 1.0 / np.float64(s)
                got = (x.astype(np.float64) * rd).astype(np.float32)
                ok = np.isfinite(want) & (np.abs(want) >= np.float32(2.0 ** -126))  # normal quotients
                assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32)), f"scale {s!r}"
                checked += int(ok.sum())
    assert checked > 100_000_000


def test_magic_add_rounds_half_to_even_then_clamps():
    v = np.arange(-200.0, 200.0, 0.125, dtype=np.float32)
    v = np.concatenate([v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(-np.inf)),
                        np.array([126.5, 127.5, 128.5, -126.5, -127.5, -128.5, 0.5, -0.5, 1.5, -1.5], np.float32)])
    want = np.clip(np.rint(v), -127, 127).astype(np.int8)        # np.rint is half-to-even, like torch.round
    c = np.clip(v, np.float32(-127.0), np.float32(127.0)).astype(np.float32)
    got = ((c + np.float32(12582912.0)).view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    assert np.array_equal(got, want)
