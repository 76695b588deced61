"""GPU parity: split-K GEMMs (d3w8a8_gemm_ws) for the skinny question-pass shapes.

Split-K hands each output tile's K range to several workgroups and adds their
partial accumulators in a fixed order. INT8 must equal the exact integer product
and the unsplit GEMM bit for bit, for every epilogue; FP8 must be reproducible
(same split, same bits) and within the FP8 accumulator bound of the oracle.
The partial sums live in a per-stream workspace between the two launches of a
call; back-to-back calls of different shapes and graph replays reuse it.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import gen, rand_fp8, rand_i8, rel_err
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

# (M, N, K): question-batch rows against projection widths, ragged edges, uneven K splits
SHAPES = [(128, 1024, 4096), (77, 200, 448), (16, 640, 2048), (130, 384, 1024), (1, 64, 64)]
SPLITS = [2, 3, 7, 16]


def _splits(Kd, tile=_lib.TILE_DMA_128_W4):
    return [s for s in SPLITS if s <= Kd // _lib.tile_k_multiple(tile)]


SPLIT_TILES = (_lib.TILE_DMA_128_W4, _lib.TILE_DMA_128_W4_K128)


def test_split_needs_a_128_tile(dev):
    a = torch.zeros(128, 1024, dtype=torch.int8, device=dev)
    for tile in set(_lib.TILES) - set(SPLIT_TILES):
        with pytest.raises(ValueError, match="128x128"):
            K.gemm("int8", a, None, a, None, epilogue=_lib.EPI_RAW, tile=tile, ksplit=2)


@pytest.mark.parametrize("tile", SPLIT_TILES)
@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_int8_split_accumulators_exact(dev, tile, M, N, Kd):
    if Kd % _lib.tile_k_multiple(tile):
        pytest.skip("K is not a multiple of this tile's step (refusal covered in test_gpu_gemm)")
    g = gen(M * 7 + N + Kd)
    a, w = rand_i8(g, M, Kd), rand_i8(g, N, Kd)
    ref = R.int_accumulate(a, w)
    ad, wd = a.to(dev), w.to(dev)
    for s in _splits(Kd, tile) + [_lib.KSPLIT_AUTO]:
        acc = K.gemm("int8", ad, None, wd, None, epilogue=_lib.EPI_RAW, tile=tile, ksplit=s)
        assert torch.equal(acc.cpu().to(torch.int64), ref), f"ksplit {s}"


@pytest.mark.parametrize("tile", SPLIT_TILES)
@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_fp8_split_reproducible_and_bounded(dev, tile, M, N, Kd):
    if Kd % _lib.tile_k_multiple(tile):
        pytest.skip("K is not a multiple of this tile's step")
    g = gen(M * 5 + N * 3 + Kd)
    a, w = rand_fp8(g, M, Kd), rand_fp8(g, N, Kd)
    ref = R.fp8_accumulate(a, w)
    bound = (a.double().abs() @ w.double().abs().t()) * 2.0 ** -14 + 1e-30
    ad, wd = a.to(dev), w.to(dev)
    for s in _splits(Kd, tile):
        acc = K.gemm("fp8", ad, None, wd, None, epilogue=_lib.EPI_RAW, tile=tile, ksplit=s)
        again = K.gemm("fp8", ad, None, wd, None, epilogue=_lib.EPI_RAW, tile=tile, ksplit=s)
        assert torch.equal(acc.view(torch.int32), again.view(torch.int32)), f"ksplit {s} not reproducible"
        acc = acc.cpu()
        assert torch.all((acc.double() - ref.double()).abs() <= bound), f"ksplit {s}"
        assert rel_err(acc, ref) < 1e-3


@pytest.mark.parametrize("epi", ["dequant", "swiglu", "residual"])
def test_int8_split_epilogues_equal_unsplit(dev, epi):
    """The epilogue runs once, on the summed accumulators: every output bit equals the unsplit GEMM's."""
    g = gen(41)
    M, N, Kd = 96, 512, 2048
    x = R.outlier_activations(g, M, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    q, s = K.quantize_rows(x.to(dev), "int8")
    s = s.reshape(-1)
    wq, ws = wq.to(dev), ws.to(dev)
    code = {"dequant": _lib.EPI_DEQUANT, "swiglu": _lib.EPI_SWIGLU, "residual": _lib.EPI_RESIDUAL}[epi]
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev) if epi == "residual" else None
    outs, amaxes = [], []
    for ks in (1, 4, 9):
        amax = torch.zeros(M, dtype=torch.float32, device=dev) if epi == "swiglu" else None
        outs.append(K.gemm("int8", q, s, wq, ws, epilogue=code, residual=res, row_amax=amax,
                           tile=_lib.TILE_DMA_128_W4, ksplit=ks))
        amaxes.append(amax)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    if epi == "swiglu":
        for a in amaxes[1:]:
            assert torch.equal(a, amaxes[0])


def test_split_with_row_map_equals_unsplit(dev):
    """Ragged batches: packed rows scattered through row_map, with and without the split."""
    g = gen(43)
    lengths, W, Kd, N = [13, 0, 32, 7], 32, 1024, 256
    x = torch.zeros(len(lengths), W, Kd, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    wq, ws = wq.to(dev), ws.to(dev)
    outs = []
    for ks in (1, 5):
        out = torch.full((len(lengths) * W, N), 7.0, dtype=torch.bfloat16, device=dev)
        q, sc, rmap = K.quantize_rows_ragged(x.to(dev), lengths, "int8", out=out)
        K.gemm("int8", q, sc.reshape(-1), wq, ws, out=out, row_map=rmap, tile=_lib.TILE_DMA_128_W4, ksplit=ks)
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_back_to_back_calls_share_the_workspace(dev):
    """Calls of different shapes and splits share one workspace; each result is the exact product."""
    g = gen(47)
    cases = [(128, 1024, 2048, 8), (40, 256, 1024, 3), (128, 2048, 4096, 16), (40, 256, 1024, 16),
             (128, 1024, 2048, 2)]
    ops = []
    for M, N, Kd, s in cases:
        a, w = rand_i8(g, M, Kd), rand_i8(g, N, Kd)
        ops.append((a, w, s, R.int_accumulate(a, w)))
    outs = [K.gemm("int8", a.to(dev), None, w.to(dev), None, epilogue=_lib.EPI_RAW,
                   tile=_lib.TILE_DMA_128_W4, ksplit=s) for a, w, s, _ in ops]
    torch.cuda.synchronize()
    for out, (_, _, s, ref) in zip(outs, ops):
        assert torch.equal(out.cpu().to(torch.int64), ref), f"ksplit {s}"


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_split_gemm_graph_replays(dev, mode):
    """A captured split-K GEMM replays to the eager result, with eager work and syncs between replays."""
    g = gen(53)
    M, N, Kd = 64, 768, 2048
    mk = rand_i8 if mode == "int8" else rand_fp8
    a, w = mk(g, M, Kd).to(dev), mk(g, N, Kd).to(dev)
    sa = torch.rand(M, generator=g).mul(1e-2).to(dev)
    sw = torch.rand(N, generator=g).mul(1e-2).to(dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    t = _lib.TILE_DMA_128_W4_K128  # a splitting tile (the automatic one at this M streams without splits)
    with torch.cuda.stream(side):
        eager = K.gemm(mode, a, sa, w, sw, ksplit=8, tile=t).clone()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out = K.gemm(mode, a, sa, w, sw, ksplit=8, tile=t)
    for _ in range(3):
        K.gemm(mode, a, sa, w, sw, ksplit=4, tile=t)  # eager split-K work on another workspace between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_gemm_captured_on_torch_default_capture_stream(dev, mode):
    """The usual capture pattern: warm up on a side stream, then torch.cuda.graph(g) without a stream
    (torch captures on a stream of its own). Skinny GEMMs (no split) and split-K GEMMs both capture and
    every replay equals the eager result."""
    g = gen(59)
    M, N, Kd = 96, 1024, 2048
    mk = rand_i8 if mode == "int8" else rand_fp8
    a, w = mk(g, M, Kd).to(dev), mk(g, N, Kd).to(dev)
    sa = torch.rand(M, generator=g).mul(1e-2).to(dev)
    sw = torch.rand(N, generator=g).mul(1e-2).to(dev)
    calls = [dict(), dict(tile=_lib.TILE_DMA_128_W4_K128, ksplit=4)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = [K.gemm(mode, a, sa, w, sw, **c).clone() for c in calls]
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [K.gemm(mode, a, sa, w, sw, **c) for c in calls]
    for _ in range(3):
        K.gemm(mode, a, sa, w, sw)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16))
