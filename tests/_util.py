"""Helpers shared by the tests (seeded inputs, error metrics)."""

from __future__ import annotations

import torch


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Norm-wise relative error, the metric of the reference's tests/test_quant.py:11-12."""
    return float((a.float() - b.float()).norm() / b.float().norm())


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|ordinal(a) - ordinal(b)| of two bf16 tensors (same sign region assumed per element)."""
    def ordinal(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (ordinal(a) - ordinal(b)).abs()


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def rand_i8(g: torch.Generator, *shape) -> torch.Tensor:
    """Uniform int8 in [-127, 127] (the range the quantizer produces)."""
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int16).to(torch.int8)


def rand_fp8(g: torch.Generator, *shape) -> torch.Tensor:
    """e4m3fn values spread over the full range by quantizing N(0,1) rows (max 448)."""
    x = torch.randn(*shape, generator=g)
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
    return (x / (amax / 448.0)).clamp(-448, 448).to(torch.float8_e4m3fn)
