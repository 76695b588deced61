"""torch-CPU restatement of the reference's W8A8 Linear arithmetic (TEST ORACLE).

Every function here runs on CPU tensors only and follows a cited line range of
the reference (paths relative to the reference checkout). It is the checker
the HIP path is measured against; the product package never imports it.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

MODES = ("auto", "none", "fp8", "int8")  # d3trt/model/quant.py:28
FP8 = torch.float8_e4m3fn                # quant.py:30 (OCP E4M3, max 448, no inf)
FP8_MAX = 448.0                          # quant.py:31
INT8_MAX = 127.0                         # quant.py:32
EPS = 1e-12                              # quant.py:34 (activation/weight amax floor)


def _cpu(t: torch.Tensor) -> torch.Tensor:
    if t.device.type != "cpu":
        raise ValueError("the oracle runs on CPU tensors only")
    return t


# ---------------------------------------------------------------------------
# quantization (quant.py:77-100)
# ---------------------------------------------------------------------------
def quantize_weight(weight: torch.Tensor, mode: str) -> tuple[torch.Tensor, torch.Tensor]:
    """[N, K] float -> ([N, K] int8/fp8, [N] fp32 per-output-channel scale).

    Follows d3trt/model/quant.py:77-89: amax per row floored at 1e-12,
    scale = amax / 127 (or / 448), q = clamp(round(w / scale)) for int8 and
    clamp(w / scale) cast to e4m3fn (round-to-nearest-even) for fp8.
    """
    w = _cpu(weight).float()
    amax = w.abs().amax(dim=1).clamp_min(EPS)
    if mode == "fp8":
        scale = amax / FP8_MAX
        q = (w / scale[:, None]).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    elif mode == "int8":
        scale = amax / INT8_MAX
        q = (w / scale[:, None]).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8)
    else:
        raise ValueError(f"cannot quantize weights to {mode!r}")
    return q.contiguous(), scale.contiguous()


def quantize_rows(x: torch.Tensor, mode: str) -> tuple[torch.Tensor, torch.Tensor]:
    """[M, K] activations -> (q [M, K], [M, 1] fp32 per-token scale).

    Follows d3trt/model/quant.py:92-100. Note the two fp32 divisions
    (amax / 127, then x / scale) and torch.round's half-to-even rounding.
    """
    xf = _cpu(x).float()
    amax = xf.abs().amax(dim=1, keepdim=True).clamp_min(EPS)
    if mode == "fp8":
        scale = amax / FP8_MAX
        return (xf / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8), scale
    scale = amax / INT8_MAX
    return (xf / scale).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8), scale


def quantize_rows_with_amax(x: torch.Tensor, amax: torch.Tensor, mode: str):
    """quantize_rows with the row amax supplied (it must equal max|x_r|).

    Used for the requantization after SwiGLU, where the amax is gathered while
    the rows are produced; the arithmetic after the amax is quant.py:95-100.
    """
    xf = _cpu(x).float()
    amax = _cpu(amax).float().reshape(-1, 1).clamp_min(EPS)
    if mode == "fp8":
        scale = amax / FP8_MAX
        return (xf / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8), scale
    scale = amax / INT8_MAX
    return (xf / scale).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8), scale


# ---------------------------------------------------------------------------
# accumulation
# ---------------------------------------------------------------------------
_LIB: Optional[ctypes.CDLL] = None


def _lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libd3oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing; run oracle/build.py")
        lib = ctypes.CDLL(path)
        lib.oracle_igemm_i8.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ]
        lib.oracle_igemm_i8.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def int_accumulate_bruteforce(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Exact int64 ``q @ w.T`` for int8 q [M, K] and w [N, K] (C brute force)."""
    q = _cpu(q).contiguous()
    w = _cpu(w).contiguous()
    if q.dtype != torch.int8 or w.dtype != torch.int8 or q.shape[1] != w.shape[1]:
        raise ValueError("int_accumulate_bruteforce wants int8 [M, K] and [N, K]")
    M, K = q.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=torch.int64)
    rc = _lib().oracle_igemm_i8(q.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K, K, K)
    if rc != 0:
        raise RuntimeError(f"oracle_igemm_i8 failed ({rc})")
    return out


def int_accumulate(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Exact int64 ``q @ w.T`` for int8 operands via a float64 GEMM.

    Every product is an integer of magnitude <= 127*127 and every partial sum
    of K <= 2**39 such terms stays below 2**53, so float64 additions are exact
    in any summation order; the result equals the int64 brute force (pinned by
    the oracle tests).
    """
    q = _cpu(q)
    w = _cpu(w)
    if q.dtype != torch.int8 or w.dtype != torch.int8:
        raise ValueError("int_accumulate wants int8 operands")
    return (q.double() @ w.double().t()).to(torch.int64)


def fp32_accumulate(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The reference emulation's accumulator, ``q.float() @ w.float().t()`` (quant.py:161)."""
    return _cpu(q).float() @ _cpu(w).float().t()


def fp8_accumulate(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """float64 ``q @ w.T`` of e4m3fn operands (products exact; sum rounded once at the end)."""
    return (_cpu(q).double() @ _cpu(w).double().t()).float()


def dequant(acc: torch.Tensor, scale_tok: torch.Tensor, scale_ch: torch.Tensor,
            dtype: torch.dtype) -> torch.Tensor:
    """``(acc.float() * scale_tok) * scale_ch`` rounded to ``dtype``.

    quant.py:197 (int8: int32 acc converted to fp32, then the token scale, then
    the channel scale, evaluated left to right) and quant.py:162 (emulation).
    """
    accf = acc.float() if acc.dtype != torch.float32 else acc
    return (accf * scale_tok.reshape(-1, 1).float() * scale_ch.reshape(1, -1).float()).to(dtype)


def int8_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, dtype: torch.dtype):
    """QuantLinear._int8 (quant.py:190-197) with the exact integer accumulator.

    Returns (out [M, N] dtype, acc int64 [M, N], q [M, K], scale [M, 1]).
    Zero padding rows (quant.py:194, 200-205) only append rows and are dropped
    again, so they do not change the first M rows.
    """
    q, s = quantize_rows(x, "int8")
    acc = int_accumulate(q, wq)
    return dequant(acc, s, ws, dtype), acc, q, s


def fp8_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, dtype: torch.dtype):
    """QuantLinear._fp8 rowwise (quant.py:164-179): e4m3 quant, fp32-accurate GEMM,
    ``(acc * s_tok) * s_ch`` to ``dtype``. Returns (out, acc fp32, q, scale)."""
    q, s = quantize_rows(x, "fp8")
    acc = fp8_accumulate(q, wq)
    return dequant(acc, s, ws, dtype), acc, q, s


def emulated_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, mode: str,
                    dtype: torch.dtype) -> torch.Tensor:
    """QuantLinear._emulated (quant.py:158-162) verbatim in semantics: fp32 accumulate."""
    q, s = quantize_rows(x, mode)
    acc = fp32_accumulate(q, wq)
    return (acc * s * ws[None, :]).to(dtype)


def linear_forward(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, mode: str,
                   dtype: torch.dtype) -> torch.Tensor:
    """QuantLinear.forward (quant.py:148-155): flatten [..., K] -> [M, K], run, reshape."""
    shape = x.shape[:-1]
    flat = x.reshape(-1, x.shape[-1])
    if mode == "int8":
        out = int8_linear(flat, wq, ws, dtype)[0]
    else:
        out = fp8_linear(flat, wq, ws, dtype)[0]
    return out.reshape(*shape, wq.shape[0])


# ---------------------------------------------------------------------------
# the chain around the linears
# ---------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, zero_centered: bool = True):
    """Qwen3_5RMSNorm (transformers models/qwen3_5/modeling_qwen3_5.py:720-734).

    ``bf16( (fp32(x) * rsqrt(mean(fp32(x)**2) + eps)) * (1 + fp32(w)) )``; with
    ``zero_centered=False`` the gain is ``w`` itself. This is the semantics of
    the reference's TRT-LLM ``RMSNorm(use_gemma=True)`` (trtllm_stack.py:217-228).
    """
    xf = _cpu(x).float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    gain = (1.0 + weight.float()) if zero_centered else weight.float()
    return (normed * gain).to(x.dtype)


def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """_TrtllmMLP.forward's activation (trtllm_stack.py:132-134).

    ``gate, up = gate_up.chunk(2, -1)``; ``F.silu(gate) * up`` on bf16 tensors:
    silu is computed in fp32 and rounded to bf16, then the product is rounded.
    """
    gate, up = _cpu(gate_up).chunk(2, dim=-1)
    return F.silu(gate) * up


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float,
                  head_dim: int) -> torch.Tensor:
    """``delta.norm(core, z)`` of D3Core._delta (core.py:390): Qwen3_5RMSNormGated (transformers
    modeling_qwen3_5.py:175-184) on rows of ``head_dim``, the module built in the model dtype
    (trtllm_stack.py:198), reshaped back to x's shape."""
    shape = x.shape
    h = _cpu(x).reshape(-1, head_dim)
    g = _cpu(z).reshape(-1, head_dim)
    input_dtype = h.dtype
    hs = h.to(torch.float32)
    variance = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(variance + eps)
    hs = _cpu(weight) * hs.to(input_dtype)
    hs = hs * F.silu(g.to(torch.float32))
    return hs.to(input_dtype).reshape(shape)


def split_query_gate(q_proj_out: torch.Tensor, head_dim: int):
    """D3Core._attention's split of the q_proj output (core.py:231-232): rows viewed as
    [heads, 2 * head_dim], chunked into query and gate halves, the gate reshaped to [..., heads * head_dim]."""
    t = _cpu(q_proj_out)
    shape = t.shape[:-1]
    query, gate = torch.chunk(t.view(*shape, -1, head_dim * 2), 2, dim=-1)
    return query, gate.reshape(*shape, -1)


def gated_input(out: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """The o_proj input of a gated attention layer, ``out * torch.sigmoid(gate)`` (core.py:297), in the
    tensors' dtype: torch rounds the sigmoid to that dtype, then the product."""
    return _cpu(out) * torch.sigmoid(_cpu(gate))


def mlp_block(x: torch.Tensor, norm_w: torch.Tensor, eps: float,
              wgu_q: torch.Tensor, wgu_s: torch.Tensor,
              wd_q: torch.Tensor, wd_s: torch.Tensor, mode: str,
              zero_centered: bool = True) -> dict:
    """The quantized MLP block: norm -> quant -> gate_up -> SwiGLU -> requant -> down -> +x.

    core.py:214-215 (``hidden + mlp(post_attention_layernorm(hidden))``) with
    _TrtllmMLP.forward (trtllm_stack.py:131-134) and QuantLinear for both
    projections. ``wgu_q`` is the reference's ``cat([gate, up], 0)`` layout
    (trtllm_stack.py:366-368). Returns every intermediate for staged parity.
    """
    normed = rmsnorm(x, norm_w, eps, zero_centered)
    lin = int8_linear if mode == "int8" else fp8_linear
    gu, acc1, q1, s1 = lin(normed, wgu_q, wgu_s, x.dtype)
    h = swiglu(gu)
    down, acc2, q2, s2 = lin(h, wd_q, wd_s, x.dtype)
    out = x + down
    return dict(normed=normed, q1=q1, s1=s1, acc1=acc1, gate_up=gu, h=h,
                q2=q2, s2=s2, acc2=acc2, down=down, out=out)


def stack_layer(x: torch.Tensor, w_in: torch.Tensor, w_post: torch.Tensor,
                wqkv_q: torch.Tensor, wqkv_s: torch.Tensor, wo_q: torch.Tensor, wo_s: torch.Tensor,
                wgu_q: torch.Tensor, wgu_s: torch.Tensor, wd_q: torch.Tensor, wd_s: torch.Tensor,
                mode: str, eps: float = 1e-6) -> dict:
    """One backbone layer with the token mixer replaced by identity on the query block.

    D3Core._layer (core.py:205-215): ``h = x + o_proj(mix(qkv_proj(input_layernorm(x))))``,
    ``out = h + mlp(post_attention_layernorm(h))``, every projection a W8A8 QuantLinear; ``mix``
    keeps the first ``hidden`` columns of the fused [q | k | v] output. Returns the intermediates.
    """
    H = x.shape[1]
    lin = int8_linear if mode == "int8" else fp8_linear
    normed = rmsnorm(x, w_in, eps)
    qkv = lin(normed, wqkv_q, wqkv_s, x.dtype)[0]
    o = lin(qkv[:, :H], wo_q, wo_s, x.dtype)[0]
    h = x + o
    mlp = mlp_block(h, w_post, eps, wgu_q, wgu_s, wd_q, wd_s, mode)
    return dict(normed=normed, qkv=qkv, o=o, h=h, out=mlp["out"], mlp=mlp)


# ---------------------------------------------------------------------------
# synthetic inputs
# ---------------------------------------------------------------------------
def outlier_activations(gen: torch.Generator, M: int, K: int, frac: float = 0.01,
                        factor: float = 20.0) -> torch.Tensor:
    """bf16 [M, K] ~ N(0, 1) with round(frac*K) channels scaled by ``factor``.

    Draw order: x = randn(M, K), then idx = randperm(K)[:round(frac*K)].
    """
    x = torch.randn(M, K, generator=gen)
    n_out = int(round(frac * K))
    if n_out:
        idx = torch.randperm(K, generator=gen)[:n_out]
        x[:, idx] *= factor
    return x.to(torch.bfloat16)


def gaussian_weight(gen: torch.Generator, N: int, K: int, std: float = 0.02) -> torch.Tensor:
    """bf16 [N, K] ~ N(0, std^2)."""
    return (std * torch.randn(N, K, generator=gen)).to(torch.bfloat16)


def numpy_f32(t: torch.Tensor) -> np.ndarray:
    return _cpu(t).float().numpy()
