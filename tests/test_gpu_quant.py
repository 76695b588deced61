"""GPU parity: per-token quantization kernels vs the oracle (bit-exact)."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import gen
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 16), (3, 40), (7, 1000), (128, 1024), (33, 4096), (64, 12288), (5, 16384), (3, 20000), (257, 520),
]


def _edge_rows(x: torch.Tensor) -> torch.Tensor:
    x = x.clone()
    if x.shape[0] >= 4:
        x[0] = 0.0                    # zero row: q = 0, scale = 1e-12 / 127 (test_quant.py:34-40)
        x[1] *= 100.0                 # outlier token (stays finite in fp16)
        x[2] = 1.0                    # constant row: every q = 127
    return x


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,Kd", SHAPES)
def test_quantize_rows_bit_exact(dev, mode, dtype, M, Kd):
    g = gen(M * 7919 + Kd)
    x = _edge_rows(R.outlier_activations(g, M, Kd).to(dtype))
    q_ref, s_ref = R.quantize_rows(x, mode)
    q, s = K.quantize_rows(x.to(dev), mode)
    torch.cuda.synchronize()
    assert torch.equal(s.cpu(), s_ref), "per-token scales differ"
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8)), "quantized values differ"


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantize_rows_ties_round_half_even(dev, mode):
    # amax 127 -> scale exactly 1.0 (int8); x.5 values must round to even like torch.round
    row = torch.tensor([127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, 126.5, -126.5, -127.0, 0.0, 64.5, 65.5, -0.5,
                        100.5, 101.5], dtype=torch.float32)
    x = torch.stack([row, row * 448.0 / 127.0, row / 1024.0, -row]).to(torch.bfloat16)
    q_ref, s_ref = R.quantize_rows(x, mode)
    q, s = K.quantize_rows(x.to(dev), mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_quantize_rows_strided_input(dev):
    g = gen(5)
    big = R.outlier_activations(g, 64, 2048)
    x = big[:, 512:1536]  # row stride 2048, K = 1024
    q_ref, s_ref = R.quantize_rows(x, "int8")
    q, s = K.quantize_rows(big.to(dev)[:, 512:1536], "int8")
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu(), q_ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantize_weight_matches_oracle(dev, mode):
    from d3trt_amd import quant as Q
    g = gen(11)
    w = R.gaussian_weight(g, 96, 256)
    w[0] *= 100.0
    q_ref, s_ref = R.quantize_weight(w, mode)
    q, s = Q.quantize_weight(w.to(dev), mode)
    assert s.shape == (96,)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,Kd", [(4, 4096), (130, 12288), (1, 64)])
def test_quantize_rows_amax_bit_exact(dev, mode, M, Kd):
    g = gen(M + Kd)
    h = R.outlier_activations(g, M, Kd)
    amax = h.float().abs().amax(dim=1)
    q_ref, s_ref = R.quantize_rows(h, mode)
    q, s = K.quantize_rows_amax(h.to(dev), amax.to(dev), mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_quantize_rows_amax_external_amax_clamps(dev, mode):
    """An amax from outside that is not the row's own max: above it the codes shrink, below it the
    quotients pass the code range and clamp (the path the row's own amax never takes)."""
    g = gen(77)
    M, Kd = 12, 4096
    h = R.outlier_activations(g, M, Kd)
    own = h.float().abs().amax(dim=1)
    amax = own * torch.tensor([2.0, 0.5, 1.0, 0.25] * 3)
    q_ref, s_ref = R.quantize_rows_with_amax(h, amax, mode)
    q, s = K.quantize_rows_amax(h.to(dev), amax.to(dev), mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_fp8_int8_quotient_just_above_the_code_range(dev, mode):
    """Rows whose max element divided by the fp32 scale lands just above 127 / 448 in fp32 (the
    reference clamps it; the kernels, which skip the clamp for the row's own amax, must round it to
    127 / 448 as well)."""
    lim = 127.0 if mode == "int8" else 448.0
    cand = torch.linspace(0.5, 64.0, 200001, dtype=torch.float32)
    over = cand[(cand / (cand / lim)) > lim][:64]
    assert over.numel() == 64
    x = torch.randn(64, 1024, generator=gen(5)) * 0.1
    x[:, 17] = over
    x[:, 900] = -over
    q_ref, s_ref = R.quantize_rows(x, mode)
    q, s = K.quantize_rows(x.to(dev), mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("kblock", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_zero_codes_keep_the_sign(dev, dtype, kblock):
    """x / scale is a zero of x's sign for x = +-0, and e4m3fn keeps it: -0 -> 0x80, +0 -> 0x00
    (quant.py:98). The gated and GDN kernels quantize their own outputs the same way."""
    g = gen(77)
    M, Kd = 8, 4096
    x = R.outlier_activations(g, M, Kd).to(dtype)
    x[:, 0::3] = -0.0
    x[:, 1::7] = 0.0
    q_ref, s_ref = R.quantize_rows(x, "fp8")
    assert int((q_ref.view(torch.uint8) == 0x80).sum()) > M * Kd // 4
    q, s = K.quantize_rows(x.to(dev), "fp8", kblock=kblock)
    q = K.unblock(q) if kblock else q
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))
    if dtype != torch.float32:
        gate = torch.randn(M, Kd, generator=g).to(dtype)
        q, s, y = K.gate_quantize(x.to(dev), gate.to(dev), "fp8", want_y=True, kblock=kblock)
        q = K.unblock(q) if kblock else q
        q_ref, s_ref = R.quantize_rows(y.cpu(), "fp8")
        assert int((q_ref.view(torch.uint8) == 0x80).sum()) > M * Kd // 8
        assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s.cpu(), s_ref)
        w = (1 + 0.1 * torch.randn(128, generator=g)).to(dtype)
        q, s, y = K.gdn_norm_quantize(x.to(dev), gate.to(dev), w.to(dev), 1e-6, 128, "fp8", want_y=True,
                                      kblock=kblock)
        q = K.unblock(q) if kblock else q
        q_ref, s_ref = R.quantize_rows(y.cpu(), "fp8")
        assert int((q_ref.view(torch.uint8) == 0x80).sum()) > M * Kd // 16
        assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s.cpu(), s_ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_non_finite_rows_keep_nan_scale(dev, mode):
    """A NaN in a row makes the reference's amax, scale and linear output NaN (x.abs().amax() and
    clamp_min keep NaN, quant.py:95-100); an inf gives an inf scale and zero codes for the finite
    elements (x / inf). Finite rows around them stay bit-exact."""
    g = gen(31)
    M, Kd, N = 8, 1024, 256
    x = R.outlier_activations(g, M, Kd).float()
    x[1, 5] = float("nan")
    x[3, 700] = float("inf")
    x[4, 2] = -float("inf")
    x[6, 1000] = float("nan")
    x[6, 3] = float("inf")
    bad = [1, 3, 4, 6]
    good = [r for r in range(M) if r not in bad]
    for dtype in (torch.float32, torch.bfloat16):
        xd = x.to(dtype)
        q_ref, s_ref = R.quantize_rows(xd, mode)
        q, s = K.quantize_rows(xd.to(dev), mode)
        torch.testing.assert_close(s.cpu(), s_ref, rtol=0, atol=0, equal_nan=True)
        assert torch.isnan(s.cpu()[[1, 6]]).all() and torch.isinf(s.cpu()[[3, 4]]).all()
        assert torch.equal(q.cpu()[good].view(torch.uint8), q_ref[good].view(torch.uint8))
        # finite elements of the inf rows: x / inf is a zero of x's sign
        fin = torch.isfinite(xd[[3, 4]])
        assert torch.all(q.cpu()[[3, 4]].float()[fin] == 0)
    # the whole linear: NaN rows come out NaN, finite rows bit-exact (int8) / within the fp8 bar
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), mode)
    xb = x.to(torch.bfloat16)
    ref = R.emulated_linear(xb, wq, ws, mode, torch.bfloat16)
    q, s = K.quantize_rows(xb.to(dev), mode)
    out = K.gemm(mode, q, s.view(-1), wq.to(dev), ws.to(dev)).cpu()
    assert torch.isnan(out[[1, 6]]).all() and torch.isnan(ref[[1, 6]]).all()
    assert not torch.isfinite(out[[3, 4]]).any()
    if mode == "int8":
        assert torch.equal(out[good], R.linear_forward(xb[good], wq, ws, "int8", torch.bfloat16))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("zero_centered", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,Kd", [(64, 4096), (33, 1024), (8, 12288)])
def test_rmsnorm_quantize(dev, mode, zero_centered, dtype, M, Kd):
    """Norm output vs the Qwen3_5RMSNorm formula: the fp32 sum of squares is reduced in a different
    order than torch's CPU mean, so a bf16 output may differ by one ulp; the quantization of the
    GPU's own normed rows is then bit-exact."""
    g = gen(M * 31 + Kd)
    x = R.outlier_activations(g, M, Kd).to(dtype)
    w = (0.1 * torch.randn(Kd, generator=g) + (0.0 if zero_centered else 1.0)).to(dtype)
    amax_buf = torch.full((M,), 7.0, device=dev)
    q, s, normed = K.rmsnorm_quantize(x.to(dev), w.to(dev), 1e-6, mode, zero_centered=zero_centered,
                                      want_normed=True, clear_amax=amax_buf)
    torch.cuda.synchronize()
    ref = R.rmsnorm(x, w, 1e-6, zero_centered)
    from tests._util import bf16_ulp_diff
    d = bf16_ulp_diff(normed.cpu(), ref)  # same ordinal arithmetic holds for fp16 bit patterns
    assert int(d.max()) <= 1, "normed output more than one bf16 ulp from the formula"
    assert float((d > 0).float().mean()) < 1e-3
    # staged exactness: quantizing the GPU's normed rows on the oracle gives the GPU's q / scale
    q_ref, s_ref = R.quantize_rows(normed.cpu(), mode)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))
    assert torch.all(amax_buf.cpu() == 0.0)
