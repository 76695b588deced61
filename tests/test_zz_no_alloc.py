"""d3w8a8_gemm_noalloc (split-K partial sums in the library's static scratch) against
d3w8a8_gemm_ws with a caller workspace, both called through the C ABI.

Two calls in a row on one GPU, the second on a smaller problem: the scratch keeps the first call's
partial sums, and the second must not see them. Both entry points get the same split plan (the
automatic split fits either buffer), so FP8 results are bit-identical too. The calls ask for the
128x128 tile with 128-byte K steps, the tile that splits K (the automatic tile of these skinny
shapes streams the weights without splitting).
"""

from __future__ import annotations

import pytest
import torch

from tests._util import gen, rand_fp8, rand_i8
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

WS_BYTES = 64 << 20
TILE = _lib.TILE_DMA_128_W4_K128


def _operands(mode, M, N, Kd, seed, dev):
    g = gen(seed)
    if mode == "int8":
        a, w = rand_i8(g, M, Kd), rand_i8(g, N, Kd)
    else:
        a, w = rand_fp8(g, M, Kd), rand_fp8(g, N, Kd)
    a_s = torch.rand(M, generator=g) * 1e-2 + 1e-3
    w_s = torch.rand(N, generator=g) * 1e-2 + 1e-3
    return a.to(dev), a_s.to(dev), w.to(dev), w_s.to(dev)


def _args(mode, a, a_s, w, w_s, out, epi, M, N, Kd):
    odt = _lib.BF16 if epi != _lib.EPI_RAW else 0
    return (K.mode_code(mode), a.data_ptr(), a.stride(0), a_s.data_ptr(), w.data_ptr(), w.stride(0), w_s.data_ptr(),
            M, N, Kd, epi, odt, out.data_ptr(), out.stride(0), None, 0, None, None, TILE, _lib.KSPLIT_AUTO)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_noalloc_equals_workspace_entry_point_two_calls(dev, mode):
    lib = _lib.load()
    ws = torch.empty(WS_BYTES, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    for (M, N, Kd), seed in (((128, 4096, 4096), 1), ((64, 2048, 2048), 2)):
        # the automatic plan splits K and fits the scratch: the scratch is what this call runs on
        need = lib.d3w8a8_gemm_workspace(M, N, Kd, Kd, Kd, TILE, _lib.KSPLIT_AUTO, _lib.NOALLOC_SCRATCH_BYTES)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        assert need == lib.d3w8a8_gemm_workspace(M, N, Kd, Kd, Kd, TILE, _lib.KSPLIT_AUTO, WS_BYTES)
        a, a_s, w, w_s = _operands(mode, M, N, Kd, seed, dev)
        for epi in (_lib.EPI_DEQUANT, _lib.EPI_RAW):
            odt = torch.bfloat16 if epi == _lib.EPI_DEQUANT else (torch.int32 if mode == "int8" else torch.float32)
            ref = torch.full((M, N), 3, dtype=odt, device=dev)
            got = torch.full((M, N), 5, dtype=odt, device=dev)
            args = _args(mode, a, a_s, w, w_s, ref, epi, M, N, Kd)
            _lib.check(lib.d3w8a8_gemm_ws(*args, ws.data_ptr(), WS_BYTES, st), "gemm_ws")
            args = _args(mode, a, a_s, w, w_s, got, epi, M, N, Kd)
            _lib.check(lib.d3w8a8_gemm_noalloc(*args, st), "gemm_noalloc")
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"{mode} {M}x{N}x{Kd} epilogue {epi}"


def test_noalloc_rejects_a_split_beyond_the_scratch(dev):
    lib = _lib.load()
    M, N, Kd = 128, 24576, 4096  # 192 tiles x 8 splits x 64 KiB = 96 MiB of partial sums
    a, a_s, w, w_s = _operands("int8", M, N, Kd, 3, dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    args = list(_args("int8", a, a_s, w, w_s, out, _lib.EPI_DEQUANT, M, N, Kd))
    args[-1] = 8  # ksplit
    rc = lib.d3w8a8_gemm_noalloc(*args, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.EINVAL
    assert "scratch" in lib.d3w8a8_last_error().decode()


def test_noalloc_through_the_torch_wrapper(dev):
    """kernels.gemm(noalloc=True) routes to the same entry point and matches the default path."""
    M, N, Kd = 100, 4096, 4096
    a, a_s, w, w_s = _operands("int8", M, N, Kd, 4, dev)
    ref = K.gemm("int8", a, a_s, w, w_s, tile=TILE)
    got = K.gemm("int8", a, a_s, w, w_s, tile=TILE, noalloc=True)
    assert torch.equal(got, ref)
