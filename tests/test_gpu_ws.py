"""GPU parity of the weight-streaming tile (skinny M, the question batches' GEMMs).

One wave streams the weight slab, one wave per 32 rows computes, and the K blocks are summed in K
order with the same MFMA operand assignment as the 128x128 tile with 128-byte K steps: every result
equals that tile's unsplit result bit for bit (INT8 and FP8, every epilogue), so FP8 rows come out
identical whatever M is (a row computed alone equals the same row inside a 128-row batch), which is
what lets a packed question batch equal its blocks run one by one.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rand_fp8, rand_i8, rel_err
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu
WS = _lib.TILE_WS


@pytest.mark.parametrize("M", [1, 5, 32, 33, 64, 96, 127, 128, 129, 300])
@pytest.mark.parametrize("N,Kd", [(16, 128), (48, 256), (100, 384), (1024, 640), (6144, 4096), (64, 12288)])
def test_ws_int8_raw_exact(dev, M, N, Kd):
    g = gen(M * 1009 + N * 31 + Kd)
    a, w = rand_i8(g, M, Kd), rand_i8(g, N, Kd)
    acc = K.gemm("int8", a.to(dev), None, w.to(dev), None, epilogue=_lib.EPI_RAW, tile=WS)
    assert torch.equal(acc.cpu().to(torch.int64), R.int_accumulate(a, w))


@pytest.mark.parametrize("M,N,Kd", [(128, 4096, 4096), (77, 1000, 1280), (3, 6144, 4096), (128, 4096, 12288)])
def test_ws_int8_dequant_and_residual_bit_exact(dev, M, N, Kd):
    g = gen(M + N + Kd)
    x = R.outlier_activations(g, M, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    q, s = R.quantize_rows(x, "int8")
    res = R.outlier_activations(g, M, N)
    out = K.gemm("int8", q.to(dev), s.view(-1).to(dev), wq.to(dev), ws.to(dev), tile=WS)
    ref = R.dequant(R.int_accumulate(q, wq), s, ws, torch.bfloat16)
    assert torch.equal(out.cpu(), ref)
    out = K.gemm("int8", q.to(dev), s.view(-1).to(dev), wq.to(dev), ws.to(dev), epilogue=_lib.EPI_RESIDUAL,
                 residual=res.to(dev), tile=WS)
    assert torch.equal(out.cpu(), res + ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M", [16, 100, 128])
def test_ws_swiglu(dev, mode, M):
    g = gen(M * 3 + (mode == "fp8"))
    H, I = 1024, 768
    x = R.outlier_activations(g, M, H)
    gate_up = torch.cat([R.gaussian_weight(g, I, H), R.gaussian_weight(g, I, H)])
    wq, ws = R.quantize_weight(gate_up, mode)
    q, s = R.quantize_rows(x, mode)
    wq_il = K.interleave_gate_up(wq.view(torch.uint8)).view(wq.dtype)
    amax = torch.zeros(M, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    K.gemm(mode, q.to(dev), s.view(-1).to(dev), wq_il.to(dev), K.interleave_gate_up(ws).to(dev),
           epilogue=_lib.EPI_SWIGLU, out=h, row_amax=amax, tile=WS)
    acc = R.int_accumulate(q, wq) if mode == "int8" else R.fp8_accumulate(q, wq)
    h_ref = R.swiglu(R.dequant(acc, s, ws, torch.bfloat16))
    if mode == "int8":
        d = bf16_ulp_diff(h.cpu(), h_ref)
        assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    else:
        assert rel_err(h.cpu(), h_ref) < 1e-2
    assert torch.equal(amax.cpu(), h.cpu().float().abs().amax(dim=1))


@pytest.mark.parametrize("N,Kd", [(4096, 4096), (512, 12288), (96, 640)])
def test_ws_fp8_rows_independent_of_m(dev, N, Kd):
    """FP8: a row's bits do not depend on how many rows share the launch, and the product is within the
    FP8 bars of the float64 reference."""
    g = gen(N + Kd)
    a, w = rand_fp8(g, 128, Kd), rand_fp8(g, N, Kd)
    ad, wd = a.to(dev), w.to(dev)
    full = K.gemm("fp8", ad, None, wd, None, epilogue=_lib.EPI_RAW, tile=WS)
    for lo, hi in ((0, 1), (5, 6), (0, 32), (31, 96), (100, 128)):
        part = K.gemm("fp8", ad[lo:hi], None, wd, None, epilogue=_lib.EPI_RAW, tile=WS)
        assert torch.equal(part.view(torch.int32), full[lo:hi].view(torch.int32)), f"rows {lo}:{hi}"
    ref = R.fp8_accumulate(a, w).double()
    bound = (a.double().abs() @ w.double().abs().t()) * 2.0 ** -14
    assert torch.all((full.cpu().double() - ref).abs() <= bound + 1e-6)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_ws_ragged_row_map(dev, mode):
    g = gen(17)
    lengths = [16, 3, 0, 9, 16, 1, 12, 16]
    Wd, Kd, N = 16, 1024, 640
    x = torch.zeros(len(lengths), Wd, Kd, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), mode)
    xd, wd, wsd = x.to(dev), wq.to(dev), ws.to(dev)
    out = torch.full((len(lengths) * Wd, N), 5.0, dtype=torch.bfloat16, device=dev)
    q, s, rmap = K.quantize_rows_ragged(xd, lengths, mode, out=out)
    K.gemm(mode, q, s.view(-1), wd, wsd, out=out, row_map=rmap, tile=WS)
    out = out.view(len(lengths), Wd, N).cpu()
    for b, n in enumerate(lengths):
        if n:
            qb, sb = K.quantize_rows(xd[b, :n], mode)
            assert torch.equal(out[b, :n], K.gemm(mode, qb, sb.view(-1), wd, wsd, tile=WS).cpu())
        assert torch.all(out[b, n:] == 0)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M", [1, 7, 32, 45, 96, 128, 160, 300])
@pytest.mark.parametrize("N,Kd", [(64, 128), (100, 384), (640, 1024), (6144, 4096), (96, 12288)])
def test_ws_equals_the_unsplit_128_tile(dev, mode, M, N, Kd):
    """Dequant and residual epilogues: bit-equal to tile 7 without split-K (edge rows and columns
    included, M over 128 as several row parts)."""
    g = gen(M * 7 + N + Kd + (mode == "fp8"))
    mk = rand_i8 if mode == "int8" else rand_fp8
    a, w = mk(g, M, Kd).to(dev), mk(g, N, Kd).to(dev)
    sa = torch.rand(M, generator=g).mul(1e-2).to(dev)
    sw = torch.rand(N, generator=g).mul(1e-2).to(dev)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    k7 = _lib.TILE_DMA_128_W4_K128
    for kw in (dict(), dict(epilogue=_lib.EPI_RESIDUAL, residual=res)):
        got = K.gemm(mode, a, sa, w, sw, tile=WS, **kw)
        want = K.gemm(mode, a, sa, w, sw, tile=k7, ksplit=1, **kw)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), kw.get("epilogue", "dequant")


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M", [16, 33, 128])
@pytest.mark.parametrize("H,I", [(2048, 1536), (512, 12288), (256, 8224)])
def test_ws_swiglu_equals_the_unsplit_128_tile(dev, mode, M, H, I):
    """Slabs of one gate/up pair (I = 1536) and of two pairs (I = 12288: 64-column slabs would not fit
    one round of CUs; I = 8224: 257 pairs, so the last two-pair slab holds a single pair)."""
    g = gen(M + 5 * (mode == "fp8") + I)
    mk = rand_i8 if mode == "int8" else rand_fp8
    a, w = mk(g, M, H).to(dev), mk(g, 2 * I, H).to(dev)
    sa = torch.rand(M, generator=g).mul(1e-2).to(dev)
    sw = torch.rand(2 * I, generator=g).mul(1e-2).to(dev)
    outs = []
    for tile, ks in ((WS, _lib.KSPLIT_AUTO), (_lib.TILE_DMA_128_W4_K128, 1)):
        amax = torch.zeros(M, device=dev)
        h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
        K.gemm(mode, a, sa, w, sw, epilogue=_lib.EPI_SWIGLU, out=h, row_amax=amax, tile=tile, ksplit=ks)
        outs.append((h, amax))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])


def test_ws_never_splits_k(dev):
    lib = _lib.load()
    for M, N, Kd in ((128, 4096, 4096), (16, 24576, 4096), (128, 4096, 12288)):
        assert lib.d3w8a8_gemm_workspace(M, N, Kd, Kd, Kd, WS, _lib.KSPLIT_AUTO, 64 << 20) == 0
    with pytest.raises(ValueError, match="split"):
        a = torch.zeros(64, 256, dtype=torch.int8, device=dev)
        K.gemm("int8", a, None, a, None, epilogue=_lib.EPI_RAW, tile=WS, ksplit=2)
