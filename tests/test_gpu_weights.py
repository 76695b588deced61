"""Pre-quantized weight files on the GPU: modules loaded from a file compute exactly what the modules
that quantized the bf16 weights at load time compute."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import gen
from d3trt_amd import QuantLinear, QuantMLP, load_quantized, save_quantized

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_loaded_modules_match_load_full(dev, tmp_path, mode):
    g = gen(41)
    lin = QuantLinear(512, 384, mode=mode, dtype=torch.bfloat16, device=dev)
    lin.load_full(R.gaussian_weight(g, 384, 512).to(dev))
    mlp = QuantMLP(512, 256, mode=mode, dtype=torch.bfloat16, device=dev)
    mlp.load_full(torch.cat([R.gaussian_weight(g, 256, 512), R.gaussian_weight(g, 256, 512)]).to(dev),
                  R.gaussian_weight(g, 512, 256).to(dev))
    path = str(tmp_path / "w.safetensors")
    save_quantized(path, {"o_proj": lin, "mlp": mlp})
    back = load_quantized(path, device=dev)
    x = R.outlier_activations(g, 64, 512).to(dev)
    assert torch.equal(back["o_proj"](x), lin(x))
    nw = (0.1 * torch.randn(512, generator=g)).to(torch.bfloat16).to(dev)
    assert torch.equal(back["mlp"].block(x, nw, 1e-6), mlp.block(x, nw, 1e-6))
