"""Pre-quantized weight files: a save / load round trip keeps every buffer bit for bit (CPU)."""

from __future__ import annotations

import json

import pytest
import torch
from safetensors import safe_open

from oracle import quant_ref as R
from tests._util import gen
from d3trt_amd import QuantLinear, QuantMLP, load_quantized, save_quantized
from d3trt_amd import kernels as K


def _linear(mode, n, k, seed):
    lin = QuantLinear(k, n, mode=mode, dtype=torch.bfloat16, device="cpu")
    q, s = R.quantize_weight(R.gaussian_weight(gen(seed), n, k), mode)
    with torch.no_grad():
        lin.set_weight_rows(q)
        lin.weight_scale.copy_(s)
    return lin


def _mlp(mode, h, i, seed):
    mlp = QuantMLP(h, i, mode=mode, dtype=torch.bfloat16, device="cpu")
    g = gen(seed)
    gu_q, gu_s = R.quantize_weight(torch.cat([R.gaussian_weight(g, i, h), R.gaussian_weight(g, i, h)]), mode)
    d_q, d_s = R.quantize_weight(R.gaussian_weight(g, h, i), mode)
    with torch.no_grad():
        mlp.gate_up_proj.set_weight_rows(K.interleave_gate_up(gu_q.view(torch.uint8)).view(gu_q.dtype))
        mlp.gate_up_proj.weight_scale.copy_(K.interleave_gate_up(gu_s))
        mlp.down_proj.set_weight_rows(d_q)
        mlp.down_proj.weight_scale.copy_(d_s)
    return mlp


def _same(a, b):
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8)) if a.dtype == torch.float8_e4m3fn else torch.equal(a, b)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_round_trip_keeps_buffers(tmp_path, mode):
    mods = {"q_proj": _linear(mode, 96, 128, 1), "o_proj": _linear(mode, 128, 64, 2), "mlp": _mlp(mode, 64, 96, 3)}
    path = str(tmp_path / "w.safetensors")
    save_quantized(path, mods)
    back = load_quantized(path, device="cpu")
    assert set(back) == set(mods)
    for name in ("q_proj", "o_proj"):
        assert isinstance(back[name], QuantLinear) and back[name].mode == mode
        assert _same(back[name].weight, mods[name].weight)
        assert torch.equal(back[name].weight_scale, mods[name].weight_scale)
    m, b = mods["mlp"], back["mlp"]
    assert isinstance(b, QuantMLP) and (b.hidden_size, b.intermediate_size) == (64, 96)
    for part in ("gate_up_proj", "down_proj"):
        assert _same(getattr(b, part).weight, getattr(m, part).weight)
        assert torch.equal(getattr(b, part).weight_scale, getattr(m, part).weight_scale)
    with safe_open(path, framework="pt") as h:
        meta = h.metadata()
        assert meta["format"] == "d3w8a8-v1"
        assert json.loads(meta["mlp"])["gate_up_layout"] == "interleaved-32"
        assert h.get_tensor("q_proj.weight").dtype == (torch.int8 if mode == "int8" else torch.float8_e4m3fn)


def test_load_rejects_foreign_and_mismatched_files(tmp_path):
    from safetensors.torch import save_file

    path = str(tmp_path / "x.safetensors")
    save_file({"a": torch.zeros(2)}, path, metadata={"format": "other"})
    with pytest.raises(ValueError, match="not a d3w8a8-v1"):
        load_quantized(path, device="cpu")
    lin = _linear("int8", 32, 64, 4)
    save_file({"p.weight": lin.weight.float(), "p.weight_scale": lin.weight_scale}, path,
              metadata={"format": "d3w8a8-v1", "p": json.dumps({"kind": "linear", "mode": "int8", "in": 64, "out": 32})})
    with pytest.raises(ValueError, match="p.weight"):
        load_quantized(path, device="cpu")
    with pytest.raises(ValueError):
        save_quantized(path, {"bad.name": lin})
    with pytest.raises(ValueError):
        save_quantized(path, {"x": torch.nn.Linear(4, 4)})
