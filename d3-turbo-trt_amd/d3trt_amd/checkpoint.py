"""Per-layer streaming of a bf16 safetensors checkpoint into the W8A8 projection stack.

The reference keeps a name -> shard map of the checkpoint and reads only the tensors of the layer it
is building (d3trt/model/weights.py:17-78), then quantizes each projection at load time through
QuantLinear.load_full, with gate_proj and up_proj concatenated into one gate_up weight
(d3trt/model/trtllm_stack.py:346-392, 366-368). Here the same per-layer walk fills a
:class:`~d3trt_amd.stack.LinearStack`: one layer's bf16 tensors are in host memory at a time, each
projection is quantized on the GPU by the per-row quantize kernel (``QuantLinear.load_full``), and the
gate_up rows are put in the interleaved order the fused SwiGLU epilogue reads
(``QuantMLP.load_full``). q_proj, k_proj and v_proj are concatenated into the stack's fused QKV
projection (a concatenation of weight rows: every output column is the same dot product).

:func:`convert_checkpoint` runs the same walk and writes each quantized layer to its own
pre-quantized file (:mod:`d3trt_amd.weights`), with an index; :func:`load_converted_stack` builds the
stack back from those files without re-quantizing.
"""

from __future__ import annotations

import json
import os
import time
from pathlib import Path
from typing import Any, Iterable, Mapping

import torch
from safetensors import safe_open

from .stack import LinearStack, StackLayer
from .weights import load_quantized, save_quantized

INDEX_NAME = "model.safetensors.index.json"
CONVERTED_INDEX = "d3w8a8_stack.json"
CONVERTED_FORMAT = "d3w8a8-stack-v1"


class ShardedCheckpoint:
    """Name -> shard map of a safetensors checkpoint directory (d3trt/model/weights.py:17-78).

    The map comes from ``model.safetensors.index.json`` when present, else from the keys of every
    ``*.safetensors`` file (``readout.safetensors`` excluded, as the reference does). Tensors are read
    only when asked for, shard by shard.
    """

    def __init__(self, root: str | os.PathLike):
        self.root = Path(root).expanduser().resolve()
        self.weight_map: dict[str, str] = {}
        self._total: int | None = None
        index = self.root / INDEX_NAME
        if index.exists():
            data = json.loads(index.read_text(encoding="utf-8"))
            self.weight_map = dict(data.get("weight_map") or {})
            total = (data.get("metadata") or {}).get("total_size")
            self._total = int(total) if total else None
        else:
            for shard in sorted(self.root.glob("*.safetensors")):
                if shard.name == "readout.safetensors":
                    continue
                with safe_open(str(shard), framework="pt") as handle:
                    for key in handle.keys():
                        self.weight_map[key] = shard.name
        if not self.weight_map:
            raise FileNotFoundError(f"no safetensors weights under {self.root}")
        self.shards = sorted(set(self.weight_map.values()))

    def keys(self) -> Iterable[str]:
        return self.weight_map.keys()

    def has(self, name: str) -> bool:
        return name in self.weight_map

    def total_bytes(self) -> int:
        """Checkpoint size: the index's metadata when present, else the shard files on disk."""
        if self._total is None:
            self._total = sum((self.root / s).stat().st_size for s in self.shards)
        return self._total

    def get(self, name: str, *, device: Any = "cpu") -> torch.Tensor:
        return self.get_many([name], device=device)[name]

    def get_many(self, names: Iterable[str], *, device: Any = "cpu") -> dict[str, torch.Tensor]:
        """The named tensors, each shard opened once; KeyError for a name the checkpoint lacks."""
        by_shard: dict[str, list[str]] = {}
        for name in names:
            shard = self.weight_map.get(name)
            if shard is None:
                raise KeyError(f"weight {name!r} is not in the checkpoint")
            by_shard.setdefault(shard, []).append(name)
        out: dict[str, torch.Tensor] = {}
        for shard, keys in by_shard.items():
            with safe_open(str(self.root / shard), framework="pt") as handle:
                for key in keys:
                    t = handle.get_tensor(key)
                    out[key] = t if str(device) == "cpu" else t.to(device)
        return out


def layer_names(index: int, prefix: str = "language_model") -> dict[str, str]:
    """Checkpoint names of one layer's linear-path tensors, by role (trtllm_stack.py:394-402 for the
    norms and the MLP; the attention projections of a full-attention layer)."""
    base = f"{prefix}.layers.{index}"
    return {
        "input_layernorm": f"{base}.input_layernorm.weight",
        "post_attention_layernorm": f"{base}.post_attention_layernorm.weight",
        "q_proj": f"{base}.self_attn.q_proj.weight",
        "k_proj": f"{base}.self_attn.k_proj.weight",
        "v_proj": f"{base}.self_attn.v_proj.weight",
        "o_proj": f"{base}.self_attn.o_proj.weight",
        "gate_proj": f"{base}.mlp.gate_proj.weight",
        "up_proj": f"{base}.mlp.up_proj.weight",
        "down_proj": f"{base}.mlp.down_proj.weight",
    }


def _copy_norm(param: torch.Tensor, full: torch.Tensor) -> None:
    if tuple(param.shape) != tuple(full.shape):
        raise ValueError(f"norm weight shape mismatch: module {tuple(param.shape)} vs checkpoint "
                         f"{tuple(full.shape)}")
    param.copy_(full.to(device=param.device, dtype=param.dtype))


@torch.no_grad()
def load_layer(layer: StackLayer, tensors: Mapping[str, torch.Tensor], names: Mapping[str, str]) -> None:
    """Quantize one layer's bf16 tensors (host or device) into ``layer`` on its GPU."""
    dev = layer.qkv_proj.weight.device
    _copy_norm(layer.input_layernorm, tensors[names["input_layernorm"]])
    _copy_norm(layer.post_attention_layernorm, tensors[names["post_attention_layernorm"]])
    qkv = torch.cat([tensors[names[k]].to(dev) for k in ("q_proj", "k_proj", "v_proj")], dim=0)
    layer.qkv_proj.load_full(qkv)
    del qkv
    layer.o_proj.load_full(tensors[names["o_proj"]].to(dev))
    gate_up = torch.cat([tensors[names["gate_proj"]].to(dev), tensors[names["up_proj"]].to(dev)], dim=0)
    layer.mlp.load_full(gate_up, tensors[names["down_proj"]].to(dev))  # trtllm_stack.py:366-368


@torch.no_grad()
def stream_into_stack(stack: LinearStack, checkpoint: ShardedCheckpoint | str | os.PathLike, *,
                      prefix: str = "language_model", first_layer: int = 0) -> dict:
    """Fill every layer of ``stack`` from checkpoint layers first_layer, first_layer + 1, ...

    One layer's tensors are read from their shards into host memory, quantized on the GPU, and
    released before the next layer is read (trtllm_stack.py:354-357). Returns load statistics.
    """
    ckpt = checkpoint if isinstance(checkpoint, ShardedCheckpoint) else ShardedCheckpoint(checkpoint)
    t0 = time.perf_counter()
    read = 0
    for i, layer in enumerate(stack.layers):
        names = layer_names(first_layer + i, prefix)
        tensors = ckpt.get_many(names.values(), device="cpu")
        read += sum(t.numel() * t.element_size() for t in tensors.values())
        load_layer(layer, tensors, names)
        del tensors
    torch.cuda.synchronize(next(stack.buffers()).device)
    return {"layers": len(stack.layers), "bytes_read": read, "seconds": round(time.perf_counter() - t0, 3)}


def _stack_geometry(ckpt: ShardedCheckpoint, prefix: str, index: int) -> tuple[int, int, int]:
    """(hidden, fused qkv width, intermediate) read from one layer's tensor shapes."""
    names = layer_names(index, prefix)
    shapes = {}
    for role in ("q_proj", "k_proj", "v_proj", "gate_proj"):
        shard = ckpt.weight_map.get(names[role])
        if shard is None:
            raise KeyError(f"weight {names[role]!r} is not in the checkpoint")
        with safe_open(str(ckpt.root / shard), framework="pt") as handle:
            shapes[role] = tuple(handle.get_slice(names[role]).get_shape())
    hidden = shapes["q_proj"][1]
    return hidden, sum(shapes[r][0] for r in ("q_proj", "k_proj", "v_proj")), shapes["gate_proj"][0]


@torch.no_grad()
def convert_checkpoint(checkpoint: ShardedCheckpoint | str | os.PathLike, out_dir: str | os.PathLike, *,
                       layers: int, mode: str, prefix: str = "language_model",
                       dtype: torch.dtype = torch.bfloat16, device: Any = "cuda") -> str:
    """Stream ``layers`` layers of a bf16 checkpoint through the GPU quantizer and write each quantized
    layer to ``out_dir/layer_XXXX.safetensors`` (one layer on the GPU at a time), plus an index.
    Returns the index path."""
    ckpt = checkpoint if isinstance(checkpoint, ShardedCheckpoint) else ShardedCheckpoint(checkpoint)
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    hidden, qkv_out, inter = _stack_geometry(ckpt, prefix, 0)
    files = []
    for i in range(layers):
        layer = StackLayer(hidden, qkv_out, inter, mode=mode, dtype=dtype, device=device)
        names = layer_names(i, prefix)
        tensors = ckpt.get_many(names.values(), device="cpu")
        load_layer(layer, tensors, names)
        del tensors
        name = f"layer_{i:04d}.safetensors"
        save_quantized(str(out / name), {"qkv_proj": layer.qkv_proj, "o_proj": layer.o_proj, "mlp": layer.mlp,
                                         "input_layernorm": layer.input_layernorm,
                                         "post_attention_layernorm": layer.post_attention_layernorm})
        files.append(name)
        del layer
    index = {"format": CONVERTED_FORMAT, "mode": mode, "layers": layers, "hidden": hidden, "qkv_out": qkv_out,
             "intermediate": inter, "files": files}
    path = out / CONVERTED_INDEX
    path.write_text(json.dumps(index, indent=1), encoding="utf-8")
    return str(path)


@torch.no_grad()
def load_converted_stack(out_dir: str | os.PathLike, *, dtype: torch.dtype = torch.bfloat16,
                         device: Any = "cuda") -> LinearStack:
    """The :class:`LinearStack` written by :func:`convert_checkpoint` (no re-quantization)."""
    out = Path(out_dir)
    index = json.loads((out / CONVERTED_INDEX).read_text(encoding="utf-8"))
    if index.get("format") != CONVERTED_FORMAT:
        raise ValueError(f"{out}: not a {CONVERTED_FORMAT} directory (format {index.get('format')!r})")
    stack = LinearStack(index["layers"], index["hidden"], index["qkv_out"], index["intermediate"],
                        mode=index["mode"], dtype=dtype, device=device)
    for layer, name in zip(stack.layers, index["files"]):
        mods = load_quantized(str(out / name), dtype=dtype, device=device)
        for attr in ("qkv_proj", "o_proj"):
            dst = getattr(layer, attr)
            dst.weight.copy_(mods[attr].weight)
            dst.weight_scale.copy_(mods[attr].weight_scale)
        for attr in ("gate_up_proj", "down_proj"):
            dst, src = getattr(layer.mlp, attr), getattr(mods["mlp"], attr)
            dst.weight.copy_(src.weight)
            dst.weight_scale.copy_(src.weight_scale)
        _copy_norm(layer.input_layernorm, mods["input_layernorm"])
        _copy_norm(layer.post_attention_layernorm, mods["post_attention_layernorm"])
    return stack
