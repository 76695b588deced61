"""GPU: the reference's tests/test_quant.py cases, re-expressed against the HIP module."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import rel_err
from d3trt_amd import quant

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode,limit", [("fp8", 0.06), ("int8", 0.02)])
def test_quant_linear_matches_dense(dev, mode, limit):
    # tests/test_quant.py:15-26
    torch.manual_seed(0)
    weight = torch.randn(96, 256) * 0.02
    x = torch.randn(3, 5, 256, dtype=torch.bfloat16)
    layer = quant.QuantLinear(256, 96, mode=mode, dtype=torch.bfloat16, device=dev)
    layer.load_full(weight.to(torch.bfloat16).to(dev))
    out = layer(x.to(dev))
    assert out.shape == (3, 5, 96)
    assert out.dtype == torch.bfloat16
    assert layer.kernel == ("hip-f8" if mode == "fp8" else "hip-i8")
    assert rel_err(out.cpu(), x.float() @ weight.t()) < limit
    # and identical to the oracle's restatement of the reference path
    wq, ws = R.quantize_weight(weight.to(torch.bfloat16), mode)
    ref = R.linear_forward(x, wq, ws, mode, torch.bfloat16)
    if mode == "int8":
        assert torch.equal(out.cpu(), ref)
    else:
        assert rel_err(out.cpu(), ref) < 1e-2


def test_per_token_scale_handles_outlier_rows_and_zero_rows(dev):
    # tests/test_quant.py:29-40
    torch.manual_seed(0)
    weight = torch.randn(32, 64)
    x = torch.randn(4, 64)
    x[1] *= 1000.0
    x[3] = 0.0
    layer = quant.QuantLinear(64, 32, mode="int8", dtype=torch.float32, device=dev)
    layer.load_full(weight.to(dev))
    out = layer(x.to(dev)).cpu()
    ref = x @ weight.t()
    assert rel_err(out[0], ref[0]) < 0.02
    assert torch.all(out[3] == 0)
    wq, ws = R.quantize_weight(weight, "int8")
    assert torch.equal(out, R.linear_forward(x, wq, ws, "int8", torch.float32))


def test_weight_quantization_is_per_channel(dev):
    # tests/test_quant.py:43-50
    weight = torch.ones(16, 32)
    weight[0] *= 100.0
    q, scale = quant.quantize_weight(weight.to(dev), "int8")
    assert q.dtype == torch.int8 and scale.shape == (16,)
    assert torch.all(q == 127)
    assert float(scale[0]) == pytest.approx(100.0 / 127)
    assert float(scale[1]) == pytest.approx(1.0 / 127)


def test_quantize_rows_api(dev):
    x = torch.randn(6, 48, dtype=torch.bfloat16)
    for mode in ("int8", "fp8"):
        q, s = quant.quantize_rows(x.to(dev), mode)
        q_ref, s_ref = R.quantize_rows(x, mode)
        assert s.shape == (6, 1)
        assert torch.equal(s.cpu(), s_ref)
        assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_fp8_supported_and_resolve_mode_on_gfx950(dev):
    assert quant.fp8_supported(dev)
    assert quant.resolve_mode("fp8", dev) == "fp8"
    assert quant.resolve_mode("auto", dev, weight_bytes=1 << 60) == "fp8"
    assert quant.resolve_mode("auto", dev, weight_bytes=1 << 20) == "none"


def test_make_linear_and_summarize(dev):
    lin = quant.make_linear(256, 96, quant="int8", dtype=torch.bfloat16, mapping=None,
                            tensor_parallel_mode=None, device=dev)
    assert isinstance(lin, quant.QuantLinear)
    lin.load_full(torch.randn(96, 256, device=dev, dtype=torch.bfloat16))
    lin(torch.randn(4, 256, device=dev, dtype=torch.bfloat16))
    dense = quant.make_linear(256, 40, quant="int8", dtype=torch.bfloat16, mapping=None,
                              tensor_parallel_mode=None, device=dev)
    assert not isinstance(dense, quant.QuantLinear)
    report = quant.summarize([lin, dense])
    assert report["kernels"] == {"hip-i8": 1}


def test_bad_shapes_raise_value_error(dev):
    from d3trt_amd import kernels as K
    a = torch.zeros(4, 24, dtype=torch.int8, device=dev)   # K % 16 != 0
    w = torch.zeros(8, 24, dtype=torch.int8, device=dev)
    with pytest.raises(ValueError):
        K.gemm("int8", a, None, w, None, epilogue=1)
    with pytest.raises(ValueError):
        K.gemm("int8", torch.zeros(4, 32, dtype=torch.int8, device=dev), None,
               torch.zeros(8, 48, dtype=torch.int8, device=dev), None, epilogue=1)
