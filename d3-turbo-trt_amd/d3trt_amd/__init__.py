"""d3trt_amd: the W8A8 quantized Linear path of d3-trt as gfx950 (MI355X) HIP kernels.

Public API mirrors d3trt/model/quant.py (``MODES``, ``fp8_supported``,
``resolve_mode``, ``quantizable``, ``quantize_weight``, ``quantize_rows``,
``QuantLinear``, ``make_linear``, ``summarize``) plus the fused MLP block
(:class:`QuantMLP`), the backbone projection stack (:class:`LinearStack`), packed
question passes over variable-length blocks (:class:`QuestionScheduler`), per-layer
streaming of bf16 safetensors checkpoints (:func:`stream_into_stack`,
:func:`convert_checkpoint`) and pre-quantized weight files (:func:`save_quantized`,
:func:`load_quantized`).
The arithmetic lives in libd3w8a8.so (C ABI: include/d3w8a8.h); ``kernels``
holds the thin torch wrappers over it.
"""

from .quant import (  # noqa: F401
    MODES,
    QuantLinear,
    fp8_supported,
    make_linear,
    quantizable,
    quantize_rows,
    quantize_weight,
    resolve_mode,
    summarize,
)
from .mlp import QuantMLP  # noqa: F401
from .stack import LinearStack  # noqa: F401
from .weights import load_quantized, save_quantized  # noqa: F401
from .schedule import QuestionScheduler, plan_batches  # noqa: F401
from .checkpoint import ShardedCheckpoint, convert_checkpoint, load_converted_stack, stream_into_stack  # noqa: F401
from ._lib import LIB_PATH, LibraryMissing, version  # noqa: F401

__all__ = [
    "MODES", "QuantLinear", "QuantMLP", "LinearStack", "fp8_supported", "make_linear", "quantizable", "quantize_rows",
    "quantize_weight", "resolve_mode", "summarize", "LIB_PATH", "LibraryMissing", "version", "save_quantized",
    "load_quantized", "QuestionScheduler", "plan_batches", "ShardedCheckpoint", "stream_into_stack",
    "convert_checkpoint", "load_converted_stack",
]
