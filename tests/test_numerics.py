"""CPU: the arithmetic identities the quantize kernels rely on, checked exhaustively.

1. The FMA-refined quotient q' = RN(RN(x - q s) r + q), q = RN(x r), r = RN(1 / s), equals RN32(x / s)
   (quant.py:100 divides) for every bf16 x and random fp32 x over ~900 row scales, and rounds to the same
   integer everywhere; its FP8 form with the residual negated keeps the sign of every quotient, zeros
   included (tests/c/fma_division.c, compiled here with gcc and FMA from libm).
2. clamp(v, -127, 127) + 1.5 * 2^23 leaves clamp(rint(v), -127, 127) in the low byte of the float bits
   (torch.round is half-to-even; quant.py:100 rounds, then clamps).
3. With scale = RN(amax / 127) and |x| <= amax, RN(x / scale) rounds to at most 127: the int8 clamp never
   acts when the amax comes from the quantized values themselves.
4. The gated kernel's 32-bit column mapping: umulhi(k, floor((2^32 - 1) / hd) + 1) == k // hd for every
   row column k < 2^14 (the longest row) and every head width hd = 8, 16, ..., 2^14.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _all_bf16_values() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    return v[np.isfinite(v)]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_refined_quotient_equals_fp32_division(tmp_path):
    exe = tmp_path / "fma_division"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                    os.path.join(HERE, "c", "fma_division.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    words = out.stdout.split()
    assert out.returncode == 0 and words[0] == "checked" and words[2] == "mismatches", out.stdout
    assert int(words[1]) > 50_000_000 and int(words[3]) == 0, out.stdout


def test_int8_quotient_of_the_row_amax_stays_within_127():
    """|x| <= amax and scale = RN(amax / 127): RN(x / scale) <= 127 (1 + 2^-23), so rint gives <= 127."""
    amax = np.abs(_all_bf16_values())
    amax = np.maximum(amax[amax > 0], np.float32(1e-12)).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(over="ignore"):
        q = (amax / scale).astype(np.float32)                     # the largest quotient of each row
    q = q[np.isfinite(q)]
    assert q.size > 30_000
    assert float(q.max()) <= 127.0 * (1 + 2.0 ** -23) and np.all(np.rint(q) <= 127)


def test_magic_add_rounds_half_to_even_then_clamps():
    v = np.arange(-200.0, 200.0, 0.125, dtype=np.float32)
    v = np.concatenate([v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(-np.inf)),
                        np.array([126.5, 127.5, 128.5, -126.5, -127.5, -128.5, 0.5, -0.5, 1.5, -1.5], np.float32)])
    want = np.clip(np.rint(v), -127, 127).astype(np.int8)        # np.rint is half-to-even, like torch.round
    c = np.clip(v, np.float32(-127.0), np.float32(127.0)).astype(np.float32)
    got = ((c + np.float32(12582912.0)).view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    assert np.array_equal(got, want)


def test_gate_column_division_by_multiply_high():
    k = np.arange(1 << 14, dtype=np.uint64)
    for hd in range(8, (1 << 14) + 1, 8):
        m = np.uint64((0xFFFFFFFF // hd + 1) & 0xFFFFFFFF)
        assert m != 0
        q = (k * m) >> np.uint64(32)
        assert np.array_equal(q, k // np.uint64(hd)), hd
