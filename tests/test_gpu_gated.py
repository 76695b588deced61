"""GPU parity of the gated o_proj input: quantize_rows(out * sigmoid(gate)) fused (core.py:297).

The product y follows the oracle's ``out * torch.sigmoid(gate)``; the device expf and the host's
may differ in the last fp32 bit, which moves a bf16 rounding of the sigmoid on a tiny fraction of
elements, so y is held to 1 bf16 ulp on < 1e-3 of elements. Quantization of the kernel's own y is
bit-exact (int8 and fp8 codes, and scales) against the oracle's quantize_rows, and the gate read in
place from the q_proj layout equals the gate passed as its own tensor bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen
from d3trt_amd import QuantLinear
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu


def _case(seed, M, K, dtype=torch.bfloat16):
    g = gen(seed)
    out = R.outlier_activations(g, M, K).to(dtype)
    gate = (torch.randn(M, K, generator=g) * 3).to(dtype)
    return out, gate


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,Kd", [(1, 128), (37, 1000), (130, 4096), (64, 12288)])
def test_gate_quantize_matches_oracle(dev, mode, M, Kd):
    out, gate = _case(M * 7 + Kd, M, Kd)
    q, s, y = K.gate_quantize(out.to(dev), gate.to(dev), mode, want_y=True)
    y = y.cpu()
    y_ref = R.gated_input(out, gate)
    d = bf16_ulp_diff(y, y_ref)
    print(f"1-ulp fraction {float((d > 0).float().mean()):.2e}")
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    q_ref, s_ref = R.quantize_rows(y, mode)  # the kernel's own product, quantized by the oracle
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_gate_quantize_fp16(dev):
    out, gate = _case(3, 40, 512, torch.float16)
    q, s, y = K.gate_quantize(out.to(dev), gate.to(dev), "int8", want_y=True)
    y_ref = R.gated_input(out, gate)
    assert float((y.cpu().float() - y_ref.float()).abs().max()) <= float(y_ref.float().abs().max()) * 2.0 ** -10
    q_ref, s_ref = R.quantize_rows(y.cpu(), "int8")
    assert torch.equal(q.cpu(), q_ref) and torch.equal(s.cpu(), s_ref)


def test_gate_known_values(dev):
    """sigmoid(0) = 1/2 exactly and saturation at +-30 pass through the kernel unchanged."""
    out, _ = _case(4, 16, 1024)
    for gv in (0.0, 30.0, -30.0):
        gate = torch.full_like(out, gv)
        _, _, y = K.gate_quantize(out.to(dev), gate.to(dev), "int8", want_y=True)
        assert torch.equal(y.cpu(), R.gated_input(out, gate))


@pytest.mark.parametrize("head_dim,Kd", [(64, 2048), (128, 2048), (256, 2048), (96, 1920), (200, 4000),
                                         (192, 12288), (8, 16384)])
@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_gate_in_place_from_q_proj_layout(dev, head_dim, Kd, mode):
    """Heads that do not divide 512 (96, 200, 192) and the longest rows check the kernel's
    multiply-high column mapping against the gate passed as its own tensor."""
    M = 50
    g = gen(head_dim)
    q_proj_out = (torch.randn(M, 2 * Kd, generator=g) * 3).to(torch.bfloat16)
    out = R.outlier_activations(g, M, Kd)
    _, gate = R.split_query_gate(q_proj_out, head_dim)
    qa, sa, ya = K.gate_quantize(out.to(dev), gate.contiguous().to(dev), mode, want_y=True)
    qb, sb, yb = K.gate_quantize(out.to(dev), q_proj_out.to(dev), mode, gate_head_dim=head_dim, want_y=True)
    assert torch.equal(ya, yb) and torch.equal(sa, sb)
    assert torch.equal(qa.view(torch.uint8), qb.view(torch.uint8))


def test_forward_gated_equals_forward_of_the_product(dev):
    M, Kd, N = 96, 1024, 768
    out, gate = _case(9, M, Kd)
    w = R.gaussian_weight(gen(10), N, Kd)
    lin = QuantLinear(Kd, N, mode="int8", dtype=torch.bfloat16, device=dev)
    lin.load_full(w.to(dev))
    got = lin.forward_gated(out.to(dev).view(2, M // 2, Kd), gate.to(dev).view(2, M // 2, Kd))
    _, _, y = K.gate_quantize(out.to(dev), gate.to(dev), "int8", want_y=True)
    assert got.shape == (2, M // 2, N)
    assert torch.equal(got.reshape(M, N), lin(y))
    assert lin.kernel == "hip-i8"


def test_gate_quantize_rejects_bad_arguments(dev):
    out, gate = _case(11, 8, 256)
    with pytest.raises(ValueError):
        K.gate_quantize(out.float().to(dev), gate.float().to(dev), "int8")  # fp32: not a 16-bit input
    with pytest.raises(ValueError):
        K.gate_quantize(out.to(dev), torch.cat([gate, gate], 1).to(dev), "int8", gate_head_dim=12)  # 12 % 8
    with pytest.raises(ValueError):
        K.gate_quantize(out.to(dev), gate.to(dev), "int8", gate_head_dim=64)  # q_proj layout needs [M, 2K]
