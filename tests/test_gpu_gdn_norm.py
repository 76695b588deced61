"""GPU parity of the GDN output projection's input: Qwen3_5RMSNormGated over heads, fused with the
per-token quantize (core.py:390-391).

The per-head sum of squares is reduced in a different order than torch's CPU mean, and the device
expf may differ from the host's in the last fp32 bit, so the normed, gated y is held to 1 bf16 ulp
on a small fraction of elements against the oracle. Quantization of the kernel's own y is bit-exact
(codes and scales) against the oracle's quantize_rows.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen
from d3trt_amd import QuantLinear
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu


def _case(seed, M, heads, hd, wdtype=torch.bfloat16, dtype=torch.bfloat16):
    g = gen(seed)
    x = R.outlier_activations(g, M, heads * hd).to(dtype)
    z = (torch.randn(M, heads * hd, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(hd, generator=g)).to(wdtype)
    return x, z, w


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,heads,hd", [(1, 1, 128), (37, 32, 128), (130, 8, 64), (64, 16, 256), (9, 24, 512),
                                        (20, 5, 128), (6, 256, 64), (5, 40, 64)])
def test_gdn_norm_quantize_matches_oracle(dev, mode, M, heads, hd):
    x, z, w = _case(M * 3 + heads + hd, M, heads, hd)
    q, s, y = K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, hd, mode, want_y=True)
    y = y.cpu()
    y_ref = R.gated_rmsnorm(x, z, w, 1e-6, hd)
    d = bf16_ulp_diff(y, y_ref)
    print(f"1-ulp fraction {float((d > 0).float().mean()):.2e}")
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 2e-3
    q_ref, s_ref = R.quantize_rows(y, mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_gdn_norm_fp32_weight_and_fp16(dev):
    x, z, w = _case(5, 24, 8, 128, wdtype=torch.float32)
    _, _, y = K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, 128, "int8", want_y=True)
    d = bf16_ulp_diff(y.cpu(), R.gated_rmsnorm(x, z, w, 1e-6, 128))
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 2e-3
    x, z, w = _case(6, 24, 8, 128, wdtype=torch.float16, dtype=torch.float16)
    q, s, y = K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, 128, "int8", want_y=True)
    y_ref = R.gated_rmsnorm(x, z, w, 1e-6, 128)
    assert float((y.cpu().float() - y_ref.float()).abs().max()) <= float(y_ref.float().abs().max()) * 2.0 ** -9
    q_ref, s_ref = R.quantize_rows(y.cpu(), "int8")
    assert torch.equal(q.cpu(), q_ref) and torch.equal(s.cpu(), s_ref)


def test_gdn_norm_zero_gate_and_head_independence(dev):
    """z = 0 gates every value to 0 (codes 0, scale 1e-12 / 127); scaling one head by 4 leaves the other
    heads' codes untouched."""
    x, z, w = _case(7, 16, 8, 128)
    q, s, y = K.gdn_norm_quantize(x.to(dev), torch.zeros_like(z).to(dev), w.to(dev), 1e-6, 128, "int8", want_y=True)
    assert int(y.abs().max()) == 0 and int(q.abs().max()) == 0
    _, _, ya = K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, 128, "int8", want_y=True)
    x2 = x.clone()
    x2[:, :128] *= 4
    _, _, yb = K.gdn_norm_quantize(x2.to(dev), z.to(dev), w.to(dev), 1e-6, 128, "int8", want_y=True)
    assert torch.equal(ya[:, 128:], yb[:, 128:])


def test_gdn_norm_rejects_bad_arguments(dev):
    x, z, w = _case(8, 4, 4, 128)
    with pytest.raises(ValueError):
        K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, 96, "int8")  # weight is 128 long
    with pytest.raises(ValueError):
        K.gdn_norm_quantize(x.to(dev), z.to(dev), torch.ones(96, dtype=torch.bfloat16, device=dev), 1e-6, 96, "int8")
    with pytest.raises(ValueError):
        K.gdn_norm_quantize(x.float().to(dev), z.float().to(dev), w.float().to(dev), 1e-6, 128, "int8")


def test_forward_gated_norm_equals_forward_of_the_normed_rows(dev):
    M, heads, hd, N = 48, 8, 128, 512
    x, z, w = _case(12, M, heads, hd)
    lin = QuantLinear(heads * hd, N, mode="fp8", dtype=torch.bfloat16, device=dev)
    lin.load_full(R.gaussian_weight(gen(13), N, heads * hd).to(dev))
    got = lin.forward_gated_norm(x.to(dev).view(3, M // 3, -1), z.to(dev).view(3, M // 3, -1), w.to(dev), 1e-6, hd)
    _, _, y = K.gdn_norm_quantize(x.to(dev), z.to(dev), w.to(dev), 1e-6, hd, "fp8", want_y=True)
    assert got.shape == (3, M // 3, N)
    assert torch.equal(got.reshape(M, N), lin(y))
