"""Pre-quantized weight files: the W8A8 buffers of QuantLinear / QuantMLP modules in safetensors.

The reference quantizes every projection at load time from the bf16 checkpoint
(QuantLinear.load_full, d3trt/model/quant.py:137-146, fed by the per-layer reader of
d3trt/model/weights.py:60-78) and has no quantized checkpoint format
(docs/TENSORRT.md:123-124). Here a module is stored as the buffers the kernels read: the
quantized weight ([out, in], int8 or float8_e4m3fn) and its fp32 per-output-channel scales.
Loading copies them back, with no re-quantization. A QuantMLP's gate_up weight is stored in
the row order its fused SwiGLU epilogue reads (blocks of 32 gate rows, then 32 up rows),
which the metadata records.

File layout: tensors ``<name>.weight`` / ``<name>.weight_scale`` for a linear,
``<name>.gate_up_proj.*`` / ``<name>.down_proj.*`` for an MLP, and ``<name>`` for a plain
tensor stored as it is (a norm gain); the metadata holds ``format`` and one JSON entry per name.
"""

from __future__ import annotations

import json
from typing import Any, Mapping

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from .mlp import QuantMLP
from .quant import QuantLinear

FORMAT = "d3w8a8-v1"
GATE_UP_LAYOUT = "interleaved-32"  # kernels.interleave_gate_up


def _linear_tensors(prefix: str, lin: QuantLinear, out: dict) -> None:
    out[f"{prefix}.weight"] = lin.weight_rows().detach().contiguous().cpu()  # [out, in], row-major
    out[f"{prefix}.weight_scale"] = lin.weight_scale.detach().contiguous().cpu()


def save_quantized(path: str, modules: Mapping[str, nn.Module | torch.Tensor]) -> None:
    """Write the quantized buffers of ``modules`` (name -> QuantLinear, QuantMLP, or a plain tensor
    such as a norm gain) to ``path``."""
    tensors: dict[str, torch.Tensor] = {}
    meta = {"format": FORMAT}
    for name, m in modules.items():
        if "." in name or name == "format":
            raise ValueError(f"module name {name!r} may not contain '.' or be 'format'")
        if isinstance(m, QuantLinear):
            _linear_tensors(name, m, tensors)
            meta[name] = json.dumps({"kind": "linear", "mode": m.mode, "in": m.in_features, "out": m.out_features})
        elif isinstance(m, QuantMLP):
            _linear_tensors(f"{name}.gate_up_proj", m.gate_up_proj, tensors)
            _linear_tensors(f"{name}.down_proj", m.down_proj, tensors)
            meta[name] = json.dumps({"kind": "mlp", "mode": m.mode, "hidden": m.hidden_size,
                                     "intermediate": m.intermediate_size, "gate_up_layout": GATE_UP_LAYOUT})
        elif isinstance(m, torch.Tensor):
            tensors[name] = m.detach().contiguous().cpu()
            meta[name] = json.dumps({"kind": "tensor"})
        else:
            raise ValueError(f"{name!r}: only QuantLinear, QuantMLP and tensors are stored, got {type(m).__name__}")
    save_file(tensors, path, metadata=meta)


def _fill(lin: QuantLinear, handle: Any, prefix: str) -> None:
    w = handle.get_tensor(f"{prefix}.weight")
    s = handle.get_tensor(f"{prefix}.weight_scale")
    if w.dtype != lin.weight.dtype or tuple(w.shape) != (lin.out_features, lin.in_features):
        raise ValueError(f"{prefix}.weight: file has {w.dtype} {tuple(w.shape)}, module wants "
                         f"{lin.weight.dtype} {(lin.out_features, lin.in_features)}")
    if s.dtype != torch.float32 or tuple(s.shape) != tuple(lin.weight_scale.shape):
        raise ValueError(f"{prefix}.weight_scale: file has {s.dtype} {tuple(s.shape)}")
    with torch.no_grad():
        lin.set_weight_rows(w)
        lin.weight_scale.copy_(s)


def load_quantized(path: str, *, dtype: torch.dtype = torch.bfloat16,
                   device: Any = "cuda") -> dict[str, nn.Module | torch.Tensor]:
    """Modules stored by :func:`save_quantized`, built with output ``dtype`` on ``device`` (plain
    tensors come back as stored, on ``device``)."""
    out: dict[str, nn.Module | torch.Tensor] = {}
    with safe_open(path, framework="pt") as handle:
        meta = handle.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (format {meta.get('format')!r})")
        for name, text in meta.items():
            if name == "format":
                continue
            info = json.loads(text)
            if info["kind"] == "linear":
                m = QuantLinear(info["in"], info["out"], mode=info["mode"], dtype=dtype, device=device)
                _fill(m, handle, name)
            elif info["kind"] == "mlp":
                if info.get("gate_up_layout") != GATE_UP_LAYOUT:
                    raise ValueError(f"{name}: unknown gate_up layout {info.get('gate_up_layout')!r}")
                m = QuantMLP(info["hidden"], info["intermediate"], mode=info["mode"], dtype=dtype, device=device)
                _fill(m.gate_up_proj, handle, f"{name}.gate_up_proj")
                _fill(m.down_proj, handle, f"{name}.down_proj")
            elif info["kind"] == "tensor":
                m = handle.get_tensor(name).to(device)
            else:
                raise ValueError(f"{name}: unknown module kind {info['kind']!r}")
            out[name] = m
    return out
