"""GPU parity: W8A8 GEMM kernels vs the oracle.

INT8: int32 accumulators bit-exact against the exact integer product, and
dequantized outputs bit-exact against ``(float(acc) * s_tok) * s_ch``.
FP8: bf16 outputs within 1e-2 (norm-wise relative, the stated FP8 bar) of the
float64-accumulated reference. The FP8 MFMA sums the products of one
instruction with less than fp32 precision (measured: an error of 3.5 on a
16-term sum of magnitude 2e5), so accumulators are held to 2**-14 of the sum
of |products| and bf16 outputs agree to one ulp on >= 99% of elements.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rand_fp8, rand_i8, rel_err
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

TILES = list(_lib.TILES)


def _dma_needs_k64(tile, Kd, a, w) -> bool:
    """The pipelined (DMA) tiles take K % 64 == 0 (K % 128 for the 128-byte-step tile) only; other K must be
    refused, not computed."""
    mult = _lib.tile_k_multiple(tile)
    if tile in _lib.DMA_TILES and Kd % mult:
        mode = "int8" if a.dtype == torch.int8 else "fp8"
        with pytest.raises(ValueError, match=f"K % {mult}"):
            K.gemm(mode, a.to("cuda"), None, w.to("cuda"), None, epilogue=_lib.EPI_RAW, tile=tile)
        return True
    return False
SHAPES = [(1, 16, 16), (33, 80, 48), (128, 1024, 1024), (255, 192, 1040), (300, 520, 4096), (64, 4096, 272),
          (257, 300, 192), (513, 1000, 640)]


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_int8_raw_accumulators_exact(dev, tile, M, N, Kd):
    g = gen(M * 131 + N * 7 + Kd)
    a, w = rand_i8(g, M, Kd), rand_i8(g, N, Kd)
    if _dma_needs_k64(tile, Kd, a, w):
        return
    acc = K.gemm("int8", a.to(dev), None, w.to(dev), None, epilogue=_lib.EPI_RAW, tile=tile)
    ref = R.int_accumulate(a, w)
    assert torch.equal(acc.cpu().to(torch.int64), ref)


def test_int8_raw_matches_c_bruteforce(dev):
    g = gen(3)
    a, w = rand_i8(g, 70, 1040), rand_i8(g, 48, 1040)
    acc = K.gemm("int8", a.to(dev), None, w.to(dev), None, epilogue=_lib.EPI_RAW)
    assert torch.equal(acc.cpu().to(torch.int64), R.int_accumulate_bruteforce(a, w))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("tile", TILES)
def test_int8_dequant_bit_exact(dev, out_dtype, tile):
    g = gen(17)
    M, N, Kd = 200, 384, 1024
    x = R.outlier_activations(g, M, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    q, s = R.quantize_rows(x, "int8")
    out = K.gemm("int8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), out_dtype=out_dtype, tile=tile)
    ref = R.dequant(R.int_accumulate(q, wq), s, ws, out_dtype)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_fp8_raw_accumulators(dev, tile, M, N, Kd):
    g = gen(M * 13 + N + Kd)
    a, w = rand_fp8(g, M, Kd), rand_fp8(g, N, Kd)
    if _dma_needs_k64(tile, Kd, a, w):
        return
    acc = K.gemm("fp8", a.to(dev), None, w.to(dev), None, epilogue=_lib.EPI_RAW, tile=tile).cpu()
    ref = R.fp8_accumulate(a, w)
    # MFMA FP8 accumulation: held to 2**-14 of the sum of |products|, element-wise
    bound = (a.double().abs() @ w.double().abs().t()) * 2.0 ** -14 + 1e-30
    assert torch.all((acc.double() - ref.double()).abs() <= bound)
    assert rel_err(acc, ref) < 1e-3


@pytest.mark.parametrize("tile", TILES)
def test_fp8_dequant_within_tolerance(dev, tile):
    g = gen(23)
    M, N, Kd = 256, 512, 2048
    x = R.outlier_activations(g, M, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "fp8")
    q, s = R.quantize_rows(x, "fp8")
    out = K.gemm("fp8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), tile=tile).cpu()
    ref = R.dequant(R.fp8_accumulate(q, wq), s, ws, torch.bfloat16)
    assert rel_err(out, ref) < 1e-2                      # the stated FP8 bar
    d = bf16_ulp_diff(out, ref)
    assert float((d <= 1).float().mean()) > 0.99


# full-size state-pass shapes (M = 4096): every column of a sample of rows against the oracle
C2_SHAPES = [(4096, 6144, 4096), (4096, 4096, 4096), (4096, 24576, 4096), (4096, 4096, 12288)]


@pytest.mark.parametrize("tile", [_lib.TILE_AUTO, *_lib.DMA_TILES])
@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,N,Kd", C2_SHAPES)
def test_state_pass_shapes_sampled(dev, mode, M, N, Kd, tile):
    g = gen(N + Kd)
    x = R.outlier_activations(g, M, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), mode)
    q, s = K.quantize_rows(x.to(dev), mode)
    out = K.gemm(mode, q, s.reshape(-1), wq.to(dev), ws.to(dev), tile=tile)
    rows = torch.randperm(M, generator=g)[:48]
    rows = torch.cat([rows, torch.tensor([0, M - 1])])
    qs, ss = R.quantize_rows(x[rows], mode)
    assert torch.equal(q.cpu()[rows].view(torch.uint8), qs.view(torch.uint8))
    if mode == "int8":
        acc = R.int_accumulate(qs, wq)
        raw = K.gemm(mode, q, None, wq.to(dev), None, epilogue=_lib.EPI_RAW, tile=tile)
        assert torch.equal(raw.cpu()[rows].to(torch.int64), acc)
        assert torch.equal(out.cpu()[rows], R.dequant(acc, ss, ws, torch.bfloat16))
    else:
        ref = R.dequant(R.fp8_accumulate(qs, wq), ss, ws, torch.bfloat16)
        assert rel_err(out.cpu()[rows], ref) < 1e-2
        assert float((bf16_ulp_diff(out.cpu()[rows], ref) <= 1).float().mean()) > 0.99
