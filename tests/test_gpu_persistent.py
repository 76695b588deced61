"""GPU parity of GEMMs with more output tiles than compute units, in both launch forms.

One workgroup per tile (the default), and the persistent walk (D3W8A8_GEMM_PERSIST=1): one workgroup
per CU walks several tiles and issues the next tile's operand DMA inside the current tile's epilogue.
These shapes have more than 256 tiles and a partial last tile row (edge tiles inside the walk); INT8
results are held bit-exact against the exact integer product, FP8 to the 1e-2 relative bar.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rel_err
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

M = 2200  # 9 tile rows of 256, the last one partial


@pytest.fixture(params=["0", "1"], ids=["one_tile", "walk"], autouse=True)
def launch_form(request, monkeypatch):
    """The library reads D3W8A8_GEMM_PERSIST at every launch."""
    monkeypatch.setenv("D3W8A8_GEMM_PERSIST", request.param)
    return request.param
KD = 256


def _operands(g, N, mode):
    x = R.outlier_activations(g, M, KD)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, KD), mode)
    q, s = R.quantize_rows(x, mode)
    return q, s, wq, ws


@pytest.mark.parametrize("tile,N", [(_lib.TILE_AUTO, 7936), (_lib.TILE_DMA_256_W4, 7936),
                                    (_lib.TILE_DMA_256x192_W4, 6144), (_lib.TILE_DMA_256x128_W4, 4096)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_int8_dequant_many_tiles(dev, tile, N, out_dtype):
    q, s, wq, ws = _operands(gen(N + tile), N, "int8")
    out = K.gemm("int8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), out_dtype=out_dtype, tile=tile)
    ref = R.dequant(R.int_accumulate(q, wq), s, ws, out_dtype)
    assert torch.equal(out.cpu(), ref)


def test_int8_residual_many_tiles(dev):
    N = 7936
    g = gen(5)
    q, s, wq, ws = _operands(g, N, "int8")
    res = R.outlier_activations(g, M, N)
    out = K.gemm("int8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), epilogue=_lib.EPI_RESIDUAL,
                 residual=res.to(dev), tile=_lib.TILE_DMA_256_W4)
    ref = res + R.dequant(R.int_accumulate(q, wq), s, ws, torch.bfloat16)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_swiglu_many_tiles(dev, mode):
    I = 4096  # gate_up N = 8192: 32 x 9 tiles
    g = gen(6)
    x = R.outlier_activations(g, M, KD)
    gate_up = torch.cat([R.gaussian_weight(g, I, KD), R.gaussian_weight(g, I, KD)], dim=0)
    wq, ws = R.quantize_weight(gate_up, mode)
    q, s = R.quantize_rows(x, mode)
    wq_il = K.interleave_gate_up(wq.view(torch.uint8)).view(wq.dtype)
    ws_il = K.interleave_gate_up(ws)
    amax = torch.zeros(M, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    K.gemm(mode, q.to(dev), s.reshape(-1).to(dev), wq_il.to(dev), ws_il.to(dev), epilogue=_lib.EPI_SWIGLU,
           out=h, row_amax=amax, tile=_lib.TILE_DMA_256_W4)
    h = h.cpu()
    acc = R.int_accumulate(q, wq) if mode == "int8" else R.fp8_accumulate(q, wq)
    h_ref = R.swiglu(R.dequant(acc, s, ws, torch.bfloat16))
    if mode == "int8":
        d = bf16_ulp_diff(h, h_ref)
        assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    else:
        assert rel_err(h, h_ref) < 1e-2
    assert torch.equal(amax.cpu(), h.float().abs().amax(dim=1))


def test_fp8_dequant_many_tiles(dev):
    N = 7936
    q, s, wq, ws = _operands(gen(7), N, "fp8")
    out = K.gemm("fp8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), tile=_lib.TILE_DMA_256_W4)
    ref = R.dequant(R.fp8_accumulate(q, wq), s, ws, torch.bfloat16)
    assert rel_err(out.cpu(), ref) < 1e-2
    d = bf16_ulp_diff(out.cpu(), ref)
    assert float((d <= 1).float().mean()) >= 0.99


def test_repeat_calls_identical(dev):
    """The walk order and the prefetch leave no state behind: two calls give identical bits."""
    N = 7936
    q, s, wq, ws = _operands(gen(8), N, "fp8")
    args = (q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev))
    a = K.gemm("fp8", *args, tile=_lib.TILE_DMA_256_W4)
    b = K.gemm("fp8", *args, tile=_lib.TILE_DMA_256_W4)
    assert torch.equal(a, b)
