"""W8A8 quantized Linear for MI355X (gfx950): the reference's quant module API on HIP kernels.

Drop-in for d3trt/model/quant.py. Same names, signatures, buffers, attribute
names and error types:

* ``fp8``  - OCP E4M3 (``torch.float8_e4m3fn``) weights with a per-output-channel
  fp32 scale, activations quantized per token at run time, GEMM on
  ``v_mfma_scale_f32_32x32x64_f8f6f4`` with fp32 accumulation.
* ``int8`` - the same scheme in INT8 on ``v_mfma_i32_32x32x32_i8`` with exact
  int32 accumulation.

All arithmetic (quantization, GEMM, dequantization) runs in the hand-written
kernels of libd3w8a8.so. A CPU tensor raises instead of falling back: the
reference's CPU emulation (quant.py:158-162) is not part of this package.
``QuantLinear.kernel`` reports ``"hip-i8"`` / ``"hip-f8"`` once the module has run.
"""

from __future__ import annotations

from typing import Any, Sequence

import torch
import torch.nn as nn

from . import _lib
from . import kernels as K

MODES = ("auto", "none", "fp8", "int8")  # quant.py:28

_FP8 = torch.float8_e4m3fn
_FP8_MAX = 448.0
_INT8_MAX = 127.0
_EPS = 1e-12
_ARCH = "gfx950"


def fp8_supported(device: Any) -> bool:
    """True on a gfx950 GPU (quant.py:37-40 checks sm_89+; OCP FP8 MFMA is a gfx950 feature)."""
    dev = torch.device(device)
    if dev.type != "cuda" or not torch.cuda.is_available():
        return False
    arch = getattr(torch.cuda.get_device_properties(dev), "gcnArchName", "")
    return arch.split(":")[0] == _ARCH


def resolve_mode(mode: str, device: Any, weight_bytes: int | None = None) -> str:
    """Turn ``auto`` into a concrete mode (quant.py:43-69).

    ``auto`` keeps bf16 when the weights fit with 20% headroom, else picks fp8
    on gfx950 and int8 elsewhere. Explicit ``fp8`` on a GPU without OCP FP8
    MFMA is an error, not a silent downgrade.
    """
    if mode not in MODES:
        raise ValueError(f"unknown quant mode {mode!r}; expected one of {MODES}")
    dev = torch.device(device)
    if mode == "fp8" and dev.type == "cuda" and not fp8_supported(dev):
        name = torch.cuda.get_device_name(dev)
        arch = getattr(torch.cuda.get_device_properties(dev), "gcnArchName", "?")
        raise ValueError(f"fp8 needs {_ARCH} (OCP E4M3 MFMA); {name} is {arch}. Use --quant int8.")
    if mode != "auto":
        return mode
    if dev.type != "cuda":
        return "none"
    if weight_bytes:
        free, _ = torch.cuda.mem_get_info(dev)
        if free >= weight_bytes * 1.2:
            return "none"
    return "fp8" if fp8_supported(dev) else "int8"


def quantizable(in_features: int, out_features: int) -> bool:
    """Shape gate of quant.py:72-74 (both GEMM dims divisible by 16)."""
    return in_features % 16 == 0 and out_features % 16 == 0


def quantize_weight(weight: torch.Tensor, mode: str, *, kblock: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """[N, K] float -> ([N, K] fp8/int8, [N] float32 per-channel scale) (quant.py:77-89).

    Per output channel: scale = max(max|w_n|, 1e-12) / 127 (or / 448); the
    quantization is the same per-row kernel as :func:`quantize_rows`. ``kblock=True`` returns the
    codes K-blocked, [K // 64, N, 64] (QuantLinear's storage).
    """
    if mode not in ("fp8", "int8"):
        raise ValueError(f"cannot quantize weights to {mode!r}")
    w = weight
    if w.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        w = w.float()
    q, s = K.quantize_rows(w, mode, kblock=kblock)
    return q, s.reshape(-1)


def _weight_rows_in_state_dict(module: "QuantLinear", state_dict: dict, prefix: str, local_metadata: dict):
    """state_dict() hook: a K-blocked weight leaves as the reference's row-major [out, in]."""
    key = prefix + "weight"
    if module.weight_kblock and key in state_dict:
        state_dict[key] = K.unblock(state_dict[key])
    return state_dict


def _weight_from_state_dict(module: "QuantLinear", state_dict: dict, prefix: str, local_metadata: dict,
                            strict: bool, missing_keys: list, unexpected_keys: list, error_msgs: list) -> None:
    """load_state_dict() pre-hook: a row-major [out, in] weight is K-blocked into the module's storage."""
    key = prefix + "weight"
    w = state_dict.get(key)
    if module.weight_kblock and isinstance(w, torch.Tensor) and tuple(w.shape) == (module.out_features,
                                                                                   module.in_features):
        state_dict[key] = K.to_kblock(w)


def quantize_rows(x: torch.Tensor, mode: str, *, kblock: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """[M, K] activations -> (quantized [M, K], [M, 1] float32 per-token scale) (quant.py:92-100).

    ``kblock=True`` returns the quantized rows K-blocked, [K // 64, M, 64] (the layout the GEMM tiles
    load fastest; :func:`d3trt_amd.kernels.unblock` turns it back into [M, K]).
    """
    if mode not in ("fp8", "int8"):
        # the reference treats every non-fp8 mode as int8 here (quant.py:99-100)
        mode = "int8"
    x2 = x
    if x2.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        x2 = x2.float()
    return K.quantize_rows(x2, mode, kblock=kblock)


class QuantLinear(nn.Module):
    """A bias-free W8A8 linear that stands in for a TRT-LLM ``Linear`` (TP=1) (quant.py:103-197)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        mode: str,
        dtype: torch.dtype,
        device: Any,
    ):
        super().__init__()
        if mode not in ("fp8", "int8"):
            raise ValueError(f"QuantLinear needs fp8 or int8, got {mode!r}")
        if not quantizable(in_features, out_features):
            raise ValueError(f"{out_features}x{in_features} is not a quantizable GEMM shape")
        self.in_features = in_features
        self.out_features = out_features
        self.mode = mode
        self.dtype = dtype
        self.tp_size = 1
        storage = _FP8 if mode == "fp8" else torch.int8
        # The weight codes are stored the way the GEMM loads them fastest: K-blocked,
        # [in // 64, out, 64] with byte (n, k) at ((k // 64) * out + n) * 64 + k % 64, where in % 64 == 0
        # (row-major [out, in] otherwise). state_dict() and load_state_dict() exchange the reference's
        # [out, in]; weight_rows() / set_weight_rows() read and write that form.
        self.weight_kblock = in_features % 64 == 0
        wshape = (in_features // 64, out_features, 64) if self.weight_kblock else (out_features, in_features)
        self.register_buffer("weight", torch.empty(*wshape, dtype=storage, device=device))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float32, device=device))
        self._register_state_dict_hook(_weight_rows_in_state_dict)
        self._register_load_state_dict_pre_hook(_weight_from_state_dict, with_module=True)
        # "hip-i8" / "hip-f8" after the first call
        self.kernel: str | None = None
        # the activations pass from the quantize kernel to the GEMM K-blocked (whole 128-byte lines per
        # GEMM load) where K allows it; the result is the same as through row-major rows
        self.kblock = in_features % 64 == 0

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, mode={self.mode}"

    def weight_rows(self) -> torch.Tensor:
        """The weight codes as the reference holds them, row-major [out, in] (a copy when K-blocked)."""
        return K.unblock(self.weight) if self.weight_kblock else self.weight

    @torch.no_grad()
    def set_weight_rows(self, q: torch.Tensor) -> None:
        """Store row-major [out, in] weight codes (the reference's layout) into the weight buffer."""
        if tuple(q.shape) != (self.out_features, self.in_features) or q.dtype != self.weight.dtype:
            raise ValueError(f"weight codes must be {self.weight.dtype} [{self.out_features}, {self.in_features}], "
                             f"got {q.dtype} {tuple(q.shape)}")
        q = q.to(self.weight.device)
        self.weight.copy_(K.to_kblock(q) if self.weight_kblock else q)

    @torch.no_grad()
    def load_full(self, full: torch.Tensor) -> None:
        """Quantize a full-precision [out, in] weight into the buffers (quant.py:137-146)."""
        if tuple(full.shape) != (self.out_features, self.in_features):
            raise ValueError(
                f"linear shape mismatch: module {(self.out_features, self.in_features)} "
                f"vs checkpoint {tuple(full.shape)}"
            )
        q, scale = quantize_weight(full.to(self.weight.device), self.mode, kblock=self.weight_kblock)
        self.weight.copy_(q)
        self.weight_scale.copy_(scale)

    def _kernel_name(self) -> str:
        return "hip-i8" if self.mode == "int8" else "hip-f8"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[..., in] -> [..., out] in ``self.dtype`` (quant.py:148-155): quantize rows, GEMM, dequant."""
        shape = x.shape[:-1]
        flat = x.reshape(-1, self.in_features)
        q, scale = quantize_rows(flat, self.mode, kblock=self.kblock)
        out = K.gemm(self.mode, q, scale.reshape(-1), self.weight, self.weight_scale,
                     epilogue=_lib.EPI_DEQUANT, out_dtype=self.dtype)
        self.kernel = self._kernel_name()
        return out.reshape(*shape, self.out_features)

    def forward_gated(self, x: torch.Tensor, gate: torch.Tensor, *, gate_head_dim: int = 0) -> torch.Tensor:
        """``forward(x * torch.sigmoid(gate))`` with the product fused into the quantization: the gated
        attention output projection, ``attn.o_proj(out * torch.sigmoid(gate))`` (core.py:297).

        ``gate`` has x's shape, or (``gate_head_dim=head_dim``) is the q_proj output, [..., 2 * in], whose
        rows hold per head [query | gate] (core.py:231); the gate half is then read in place.
        """
        shape = x.shape[:-1]
        flat = x.reshape(-1, self.in_features)
        g = gate.reshape(flat.shape[0], -1)
        q, scale, _ = K.gate_quantize(flat, g, self.mode, gate_head_dim=gate_head_dim, kblock=self.kblock)
        out = K.gemm(self.mode, q, scale.reshape(-1), self.weight, self.weight_scale,
                     epilogue=_lib.EPI_DEQUANT, out_dtype=self.dtype)
        self.kernel = self._kernel_name()
        return out.reshape(*shape, self.out_features)

    def forward_gated_norm(self, x: torch.Tensor, z: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                           head_dim: int) -> torch.Tensor:
        """``forward(norm(x, z))`` with the gated RMSNorm over heads of ``head_dim`` fused into the
        quantization: the GDN output projection, ``delta.out_proj(delta.norm(core, z))``
        (core.py:390-391; the norm is Qwen3_5RMSNormGated with weight ``norm_weight``)."""
        shape = x.shape[:-1]
        flat = x.reshape(-1, self.in_features)
        q, scale, _ = K.gdn_norm_quantize(flat, z.reshape(flat.shape), norm_weight, eps, head_dim, self.mode,
                                          kblock=self.kblock)
        out = K.gemm(self.mode, q, scale.reshape(-1), self.weight, self.weight_scale,
                     epilogue=_lib.EPI_DEQUANT, out_dtype=self.dtype)
        self.kernel = self._kernel_name()
        return out.reshape(*shape, self.out_features)

    def forward_ragged(self, x: torch.Tensor, lengths: Sequence[int]) -> torch.Tensor:
        """A right-padded question batch [B, W, in] with ``lengths[b]`` valid rows per block.

        Only the sum(lengths) valid rows are quantized and multiplied, in one
        GEMM launch; their outputs land at their padded positions and padded
        rows of the [B, W, out] result are zero. Valid rows are bit-identical
        to :meth:`forward` on each block separately.
        """
        B, W, _ = x.shape
        out = torch.empty(B, W, self.out_features, dtype=self.dtype, device=x.device)
        out2 = out.view(B * W, self.out_features)
        q, s, row_map = K.quantize_rows_ragged(x, lengths, self.mode, out=out2, kblock=self.kblock)
        if row_map.numel():
            K.gemm(self.mode, q, s.reshape(-1), self.weight, self.weight_scale, epilogue=_lib.EPI_DEQUANT,
                   out_dtype=self.dtype, out=out2, row_map=row_map)
        self.kernel = self._kernel_name()
        return out


def make_linear(
    in_features: int,
    out_features: int,
    *,
    quant: str,
    dtype: torch.dtype,
    mapping: Any,
    tensor_parallel_mode: Any,
    device: Any,
) -> nn.Module:
    """:class:`QuantLinear` for quantizable fp8/int8 projections (quant.py:214-236).

    Anything else is the dense bf16 branch, which the reference hands to
    TRT-LLM's ``Linear``; here it is a bias-free ``torch.nn.Linear`` (TP=1;
    ``mapping`` and ``tensor_parallel_mode`` are accepted and ignored, as
    QuantLinear ignores them in the reference).
    """
    del mapping, tensor_parallel_mode
    if quant in ("fp8", "int8") and quantizable(in_features, out_features):
        return QuantLinear(in_features, out_features, mode=quant, dtype=dtype, device=device)
    layer = nn.Linear(in_features, out_features, bias=False, dtype=dtype, device=device)
    layer.tp_size = 1
    return layer


def summarize(modules: Any) -> dict[str, Any]:
    """Bytes held by quantized and unquantized linear weights, and kernels used (quant.py:239-255)."""
    quantized = dense = 0
    kernels: dict[str, int] = {}
    for module in modules:
        if isinstance(module, QuantLinear):
            quantized += module.weight.numel() * module.weight.element_size()
            key = module.kernel or "unused"
            kernels[key] = kernels.get(key, 0) + 1
        elif hasattr(module, "weight") and isinstance(getattr(module, "weight"), torch.Tensor):
            if module.weight.dim() == 2:
                dense += module.weight.numel() * module.weight.element_size()
    return {
        "quantized_gib": round(quantized / 1024**3, 3),
        "dense_linear_gib": round(dense / 1024**3, 3),
        "kernels": kernels,
    }
