"""Quantized SwiGLU MLP on fused gfx950 kernels (the reference's _TrtllmMLP with QuantLinear).

Reference chain (d3trt/model/trtllm_stack.py:131-134, core.py:214-215):

    result = hidden + down_proj(silu(gate) * up),  gate, up = gate_up_proj(norm(hidden)).chunk(2)

Here the chain is four launches, each one HBM pass:

    1. rmsnorm_quantize   norm + per-token quant of the block input; clears the row-amax buffer
    2. gemm (SWIGLU)      gate_up GEMM; epilogue dequantizes gate and up, applies SwiGLU with the
                          eager chain's bf16 rounding points, stores h and atomically maxes |h| per row
    3. quantize_rows_amax per-token requant of h with the amax gathered in 2
    4. gemm (RESIDUAL)    down GEMM; epilogue dequantizes and adds the residual in bf16

gate_up weights are stored interleaved in blocks of 32 rows so that a gate
column and its up column sit in the same lane of one wave (see
kernels.interleave_gate_up); the math per output column is unchanged.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn

from . import _lib
from . import kernels as K
from .quant import QuantLinear, quantize_weight


class QuantMLP(nn.Module):
    """gate_up / down W8A8 projections with a fused SwiGLU epilogue."""

    def __init__(self, hidden_size: int, intermediate_size: int, *, mode: str, dtype: torch.dtype,
                 device: Any):
        super().__init__()
        if intermediate_size % 32:
            raise ValueError("intermediate_size must be a multiple of 32 for the fused SwiGLU layout")
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.mode = mode
        self.dtype = dtype
        # gate_up_proj.weight holds rows interleaved in blocks of 32 (gate, up, gate, up, ...)
        self.gate_up_proj = QuantLinear(hidden_size, 2 * intermediate_size, mode=mode, dtype=dtype, device=device)
        self.down_proj = QuantLinear(intermediate_size, hidden_size, mode=mode, dtype=dtype, device=device)

    @torch.no_grad()
    def load_full(self, gate_up: torch.Tensor, down: torch.Tensor) -> None:
        """Load the reference's ``cat([gate, up], 0)`` weight (trtllm_stack.py:366-368) and ``down``.

        Quantization is per output row, so quantizing then permuting the rows
        equals permuting then quantizing.
        """
        gu = self.gate_up_proj
        if tuple(gate_up.shape) != (gu.out_features, gu.in_features):
            raise ValueError(
                f"gate_up shape mismatch: module {(gu.out_features, gu.in_features)} vs {tuple(gate_up.shape)}"
            )
        q, s = quantize_weight(gate_up.to(gu.weight.device), self.mode)
        gu.set_weight_rows(K.interleave_gate_up(q.view(torch.uint8)).view(q.dtype))
        gu.weight_scale.copy_(K.interleave_gate_up(s))
        self.down_proj.load_full(down)

    def _swiglu_requant(self, q1: torch.Tensor, s1: torch.Tensor, amax: torch.Tensor):
        gu = self.gate_up_proj
        M = s1.shape[0]
        h = torch.empty(M, self.intermediate_size, dtype=self.dtype, device=s1.device)
        K.gemm(self.mode, q1, s1.reshape(-1), gu.weight, gu.weight_scale, epilogue=_lib.EPI_SWIGLU,
               out_dtype=self.dtype, out=h, row_amax=amax)
        q2, s2 = K.quantize_rows_amax(h, amax, self.mode, kblock=self.down_proj.kblock)
        return h, q2, s2

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """``down(silu(gate) * up)`` of ``x`` (trtllm_stack.py:131-134), [..., H] -> [..., H]."""
        shape = x.shape[:-1]
        flat = x.reshape(-1, self.hidden_size)
        q1, s1 = K.quantize_rows(flat, self.mode, kblock=self.gate_up_proj.kblock)
        amax = torch.zeros(flat.shape[0], dtype=torch.float32, device=x.device)
        _, q2, s2 = self._swiglu_requant(q1, s1, amax)
        d = self.down_proj
        out = K.gemm(self.mode, q2, s2.reshape(-1), d.weight, d.weight_scale, epilogue=_lib.EPI_DEQUANT,
                     out_dtype=self.dtype)
        self._mark()
        return out.reshape(*shape, self.hidden_size)

    def block(self, hidden: torch.Tensor, norm_weight: torch.Tensor, eps: float, *,
              zero_centered: bool = True) -> torch.Tensor:
        """``hidden + mlp(rmsnorm(hidden))`` (core.py:214-215) in four fused launches."""
        shape = hidden.shape
        flat = hidden.reshape(-1, self.hidden_size)
        if not flat.is_contiguous():
            flat = flat.contiguous()
        M = flat.shape[0]
        amax = torch.empty(M, dtype=torch.float32, device=hidden.device)  # cleared by the norm kernel
        q1, s1, _ = K.rmsnorm_quantize(flat, norm_weight, eps, self.mode, zero_centered=zero_centered,
                                       clear_amax=amax, kblock=self.gate_up_proj.kblock)
        _, q2, s2 = self._swiglu_requant(q1, s1, amax)
        d = self.down_proj
        out = K.gemm(self.mode, q2, s2.reshape(-1), d.weight, d.weight_scale, epilogue=_lib.EPI_RESIDUAL,
                     out_dtype=self.dtype, residual=flat)
        self._mark()
        return out.reshape(shape)

    def _mark(self) -> None:
        name = "hip-i8" if self.mode == "int8" else "hip-f8"
        self.gate_up_proj.kernel = name
        self.down_proj.kernel = name
