"""CPU: host-side API behaviour and the C-ABI library surface (no compute without a GPU)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from d3trt_amd import _lib, quant
from tests.conftest import ROOT


def test_shape_checks():
    # reference tests/test_quant.py:53-60
    assert quant.quantizable(5120, 17408)
    assert not quant.quantizable(5120, 40)
    with pytest.raises(ValueError):
        quant.QuantLinear(64, 40, mode="fp8", dtype=torch.bfloat16, device="cpu")
    layer = quant.QuantLinear(64, 32, mode="fp8", dtype=torch.bfloat16, device="cpu")
    with pytest.raises(ValueError):
        layer.load_full(torch.zeros(32, 48))


def test_resolve_mode_off_gpu():
    # reference tests/test_quant.py:63-68
    assert quant.resolve_mode("auto", "cpu") == "none"
    assert quant.resolve_mode("int8", "cpu") == "int8"
    assert quant.resolve_mode("fp8", "cpu") == "fp8"
    with pytest.raises(ValueError):
        quant.resolve_mode("nvfp4", "cpu")


def test_summarize_counts_quantized_bytes():
    # reference tests/test_quant.py:71-80
    layers = torch.nn.ModuleList(
        [
            quant.QuantLinear(64, 32, mode="int8", dtype=torch.float32, device="cpu"),
            torch.nn.Linear(64, 8, bias=False),
        ]
    )
    report = quant.summarize(layers.modules())
    assert report["kernels"] == {"unused": 1}
    assert report["quantized_gib"] == round(64 * 32 / 1024**3, 3)


def test_constructor_errors_and_buffers():
    with pytest.raises(ValueError):
        quant.QuantLinear(64, 32, mode="none", dtype=torch.bfloat16, device="cpu")
    layer = quant.QuantLinear(64, 32, mode="fp8", dtype=torch.bfloat16, device="cpu")
    assert layer.weight.dtype == torch.float8_e4m3fn and layer.weight_rows().shape == (32, 64)
    # stored K-blocked ([in / 64, out, 64]); the state dict carries the reference's [out, in]
    assert layer.weight.shape == (1, 32, 64) and layer.state_dict()["weight"].shape == (32, 64)
    assert layer.weight_scale.dtype == torch.float32 and torch.all(layer.weight_scale == 1)
    assert layer.tp_size == 1 and layer.kernel is None
    assert "weight" in dict(layer.named_buffers()) and "weight_scale" in dict(layer.named_buffers())
    assert repr(layer) == "QuantLinear(in=64, out=32, mode=fp8)"


def test_cpu_tensors_raise_instead_of_falling_back():
    layer = quant.QuantLinear(64, 32, mode="int8", dtype=torch.bfloat16, device="cpu")
    with pytest.raises(RuntimeError, match="HIP"):
        layer(torch.zeros(2, 64, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="HIP"):
        quant.quantize_rows(torch.zeros(2, 64), "int8")
    with pytest.raises(RuntimeError, match="HIP"):
        layer.load_full(torch.zeros(32, 64))


def test_make_linear_dense_branch_on_cpu():
    dense = quant.make_linear(64, 40, quant="int8", dtype=torch.float32, mapping=None,
                              tensor_parallel_mode=None, device="cpu")
    assert isinstance(dense, torch.nn.Linear) and dense.bias is None and dense.tp_size == 1
    q = quant.make_linear(64, 32, quant="fp8", dtype=torch.bfloat16, mapping=None,
                          tensor_parallel_mode=None, device="cpu")
    assert isinstance(q, quant.QuantLinear)


def _header_functions():
    text = open(os.path.join(ROOT, "include", "d3w8a8.h")).read()
    return re.findall(r"^\S.*?\b(d3w8a8_\w+)\s*\(", text, flags=re.M)


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert set(names) == set(_lib.SIGNATURES) | set(_lib.STRING_FUNCS) | set(_lib.INT64_FUNCS)
    for name in names:
        assert hasattr(lib, name), name
    assert "gfx950" in _lib.version()


def test_c_abi_rejects_bad_arguments_before_any_launch():
    lib = _lib.load()
    # unknown mode / dtype / epilogue and bad shapes return EINVAL on the host
    assert lib.d3w8a8_quantize_rows(7, 0, None, 16, 1, 16, None, 16, None, None) == _lib.EINVAL
    assert b"mode" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_quantize_rows(0, 9, None, 16, 1, 16, None, 16, None, None) == _lib.EINVAL
    assert lib.d3w8a8_gemm(0, None, 24, None, None, 24, None, 4, 8, 24, 1, 0, None, 8, None, 0, None, None,
                           -1, None) == _lib.EINVAL
    assert b"multiple of 16" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_gemm(0, None, 32, None, None, 32, None, 4, 8, 32, 9, 0, None, 8, None, 0, None, None,
                           -1, None) == _lib.EINVAL
    assert lib.d3w8a8_rmsnorm_quantize(0, 0, None, 20, 0, None, 4, 20, 1e-6, 1, None, 20, None, None, 0,
                                       None, None) == _lib.EINVAL
    # empty problems are a successful no-op
    assert lib.d3w8a8_quantize_rows(0, 0, None, 16, 0, 16, None, 16, None, None) == _lib.OK
    with pytest.raises(ValueError):
        _lib.check(_lib.EINVAL, "probe")


def test_gate_up_interleave_roundtrip():
    from d3trt_amd import kernels as K
    w = torch.arange(128 * 3).reshape(128, 3)
    il = K.interleave_gate_up(w)
    assert torch.equal(il[:32], w[:32]) and torch.equal(il[32:64], w[64:96])
    assert torch.equal(K.deinterleave_gate_up(il), w)
    with pytest.raises(ValueError):
        K.interleave_gate_up(torch.zeros(96, 2))


def test_ragged_lengths_are_checked_on_the_host():
    """Segment lengths travel by value; bad ones are refused before any launch."""
    import ctypes
    lib = _lib.load()
    dummy = 256  # never dereferenced: every call below fails in the host-side checks
    bad_len = (ctypes.c_int32 * 2)(3, 9)   # 9 > width 8
    assert lib.d3w8a8_quantize_rows_ragged(0, 0, dummy, 64, ctypes.addressof(bad_len), 2, 8, 64, dummy, 64, dummy,
                                           dummy, None, 0, 0, 0, None) == _lib.EINVAL
    assert b"length 9" in lib.d3w8a8_last_error()
    many = (ctypes.c_int32 * 300)(*([1] * 300))
    assert lib.d3w8a8_quantize_rows_ragged(0, 0, dummy, 64, ctypes.addressof(many), 300, 8, 64, dummy, 64, dummy,
                                           dummy, None, 0, 0, 0, None) == _lib.EINVAL
    header = open(os.path.join(ROOT, "include", "d3w8a8.h")).read()
    assert re.search(r"#define D3W8A8_MAX_SEGMENTS (\d+)", header).group(1) == str(_lib.MAX_SEGMENTS)


def test_split_k_plan_on_the_host():
    """Workspace sizing and split-K validation run on the host (no launch)."""
    lib = _lib.load()
    big = 64 << 20
    slot = 128 * 128 * 4
    k128 = _lib.TILE_DMA_128_W4_K128
    # the weight-streaming tile never splits K
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, _lib.TILE_WS, -1, big) == 0
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, _lib.TILE_WS, 2, big) == -1
    # the automatic tile at question-batch M (any M <= 128 alike): weight streaming where K <= 4096
    # and its slabs fit one round of CUs (o_proj, QKV), else the 128x128 tile with 128-byte steps,
    # split as below (down, K = 12288); 768 slabs of 32 columns exceed a round, and their 192 tiles
    # of 128x128 fill the GPU unsplit
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, -1, -1, big) == 0
    assert lib.d3w8a8_gemm_workspace(128, 6144, 4096, 4096, 4096, -1, -1, big) == 0
    assert lib.d3w8a8_gemm_workspace(128, 4096, 12288, 12288, 12288, -1, -1, big) == 32 * 8 * slot
    assert lib.d3w8a8_gemm_workspace(128, 24576, 4096, 4096, 4096, -1, -1, big) == 0
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, -1, -1, 0) == 0
    assert lib.d3w8a8_gemm_workspace(16, 4096, 12288, 12288, 12288, -1, -1, big) == 32 * 8 * slot
    # on the 128x128 tile, 128 rows x 4096 columns: 32 tiles leave the GPU idle -> 4 splits of 1 KiB of K
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, k128, -1, big) == 32 * 4 * slot
    # down projection (K = 12288): 8 splits make ~one workgroup per CU
    assert lib.d3w8a8_gemm_workspace(128, 4096, 12288, 12288, 12288, k128, -1, big) == 32 * 8 * slot
    # a smaller workspace lowers the automatic split; none at all means no split
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, k128, -1, 32 * 3 * slot) == 32 * 3 * slot
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, k128, -1, 0) == 0
    # state-pass shapes fill the GPU without splitting
    assert lib.d3w8a8_gemm_workspace(4096, 6144, 4096, 4096, 4096, -1, -1, big) == 0
    # explicit requests are checked, not adjusted
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, 5, 4, big) == \
        32 * 4 * slot
    assert lib.d3w8a8_gemm_workspace(128, 4096, 256, 256, 256, 5, 8, big) == -1   # 4 K steps < 8 splits
    assert b"ksplit" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, 5, 4, 1 << 20) == -1
    assert b"too small" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, 1, 2, big) == -1  # register-staged tile
    assert b"128x128" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, 4, 2, big) == -1  # 256x256 tile
    # the 192-column, 192-row and weight-streaming tiles are accepted (no split), the next tile code is not
    for t in (_lib.TILE_DMA_256x192_W4, _lib.TILE_WS, _lib.TILE_DMA_192x192_W4, _lib.TILE_DMA_192x128_W4):
        assert lib.d3w8a8_gemm_workspace(4096, 6144, 4096, 4096, 4096, t, -1, big) == 0, t
    for t in (_lib.TILE_DMA_256x192_W4, _lib.TILE_DMA_192x192_W4, _lib.TILE_DMA_192x128_W4):
        assert lib.d3w8a8_gemm_workspace(4096, 6144, 4096, 4096, 4096, t, 2, big) == -1, t
    assert lib.d3w8a8_gemm_workspace(4096, 6144, 4096, 4096, 4096, max(_lib.TILES) + 1, -1, big) == -1
    dummy = 256
    assert lib.d3w8a8_gemm_ws(0, dummy, 4096, dummy, dummy, 4096, dummy, 128, 4096, 4096, 0, 0, dummy, 4096,
                              None, 0, None, None, 5, 4, dummy, 1 << 20, None) == _lib.EINVAL
    header = open(os.path.join(ROOT, "include", "d3w8a8.h")).read()
    assert re.search(r"#define D3W8A8_KSPLIT_AUTO \((-?\d+)\)", header).group(1) == str(_lib.KSPLIT_AUTO)



def test_kblock_layout_checked_on_the_host():
    """The K-blocked activation layout (D3W8A8_KBLOCK in mode): its conditions are refused on the host."""
    import ctypes
    from d3trt_amd import kernels as K
    lib = _lib.load()
    header = open(os.path.join(ROOT, "include", "d3w8a8.h")).read()
    assert int(re.search(r"#define D3W8A8_KBLOCK (0x[0-9a-fA-F]+)", header).group(1), 16) == _lib.KBLOCK
    dummy = 256  # never dereferenced: every call below fails in the host-side checks
    f8k = _lib.FP8 | _lib.KBLOCK

    def gemm(mode, lda, M, K, tile):
        return lib.d3w8a8_gemm(mode, dummy, lda, dummy, dummy, K, dummy, M, 256, K, 0, 0, dummy, 256, None, 0,
                               None, None, tile, None)

    assert gemm(f8k, 512, 512, 4096, _lib.TILE_128) == _lib.EINVAL  # register-staged tiles: row-major only
    assert b"pipelined" in lib.d3w8a8_last_error()
    assert gemm(f8k, 512, 512, 4096 + 32, -1) == _lib.EINVAL  # K % 64 != 0
    assert gemm(f8k, 511, 512, 4096, -1) == _lib.EINVAL  # row capacity below M
    assert gemm(f8k, 1 << 25, 512, 4096, -1) == _lib.EINVAL  # beyond the 32-bit offsets
    assert b"K-blocked" in lib.d3w8a8_last_error()
    # row-major rules do not apply to a K-blocked a: lda (the row capacity) may be below K
    assert lib.d3w8a8_gemm_workspace(128, 4096, 4096, 4096, 4096, -1, -1, 64 << 20) == 0
    # quantize entry points: K % 64 and ldq >= rows
    assert lib.d3w8a8_quantize_rows(f8k, 0, dummy, 96, 4, 96, dummy, 4, dummy, None) == _lib.EINVAL
    assert b"K % 64" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_quantize_rows(f8k, 0, dummy, 128, 4, 128, dummy, 3, dummy, None) == _lib.EINVAL
    assert b"ldq" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_quantize_rows_amax(f8k, 0, dummy, 128, dummy, 8, 128, dummy, 7, dummy, None) == _lib.EINVAL
    lens = (ctypes.c_int32 * 2)(3, 5)
    assert lib.d3w8a8_quantize_rows_ragged(f8k, 0, dummy, 64, ctypes.addressof(lens), 2, 8, 64, dummy, 7, dummy,
                                           dummy, None, 0, 0, 0, None) == _lib.EINVAL  # 8 packed rows > ldq 7
    assert b"sum of the lengths" in lib.d3w8a8_last_error()
    # the weight flag belongs to the GEMMs only; an unknown flag is an unknown mode
    assert lib.d3w8a8_quantize_rows(_lib.FP8 | _lib.W_KBLOCK, 0, dummy, 128, 4, 128, dummy, 128, dummy,
                                    None) == _lib.EINVAL
    assert lib.d3w8a8_quantize_rows(_lib.FP8 | 0x400, 0, dummy, 128, 4, 128, dummy, 128, dummy, None) == _lib.EINVAL
    assert int(re.search(r"#define D3W8A8_W_KBLOCK (0x[0-9a-fA-F]+)", header).group(1), 16) == _lib.W_KBLOCK
    f8w = _lib.FP8 | _lib.W_KBLOCK
    assert lib.d3w8a8_gemm(f8w, dummy, 4096, dummy, dummy, 255, dummy, 512, 256, 4096, 0, 0, dummy, 256, None, 0,
                           None, None, -1, None) == _lib.EINVAL  # ldw (row capacity) below N
    assert b"K-blocked w" in lib.d3w8a8_last_error()
    assert lib.d3w8a8_gemm(f8w, dummy, 4096, dummy, dummy, 256, dummy, 512, 256, 4096, 0, 0, dummy, 256, None, 0,
                           None, None, _lib.TILE_256, None) == _lib.EINVAL  # register-staged tile
    # the layout itself: byte (m, k) at ((k // 64) * ld + m) * 64 + k % 64
    x = torch.arange(5 * 192, dtype=torch.int32).reshape(5, 192)
    blocked = x.reshape(5, 3, 64).permute(1, 0, 2).contiguous()
    flat = blocked.reshape(-1)
    for m, k in ((0, 0), (4, 191), (2, 64), (3, 127)):
        assert flat[((k // 64) * 5 + m) * 64 + k % 64] == x[m, k]
    assert torch.equal(K.unblock(blocked), x)


def test_weight_storage_and_state_dict_on_the_host():
    """QuantLinear stores its codes K-blocked where in % 64 == 0; weight_rows(), state_dict() and
    load_state_dict() exchange the reference's row-major [out, in] codes."""
    g = torch.Generator().manual_seed(3)
    lin = quant.QuantLinear(128, 48, mode="int8", dtype=torch.bfloat16, device="cpu")
    q = torch.randint(-127, 128, (48, 128), generator=g, dtype=torch.int16).to(torch.int8)
    lin.set_weight_rows(q)
    assert lin.weight.shape == (2, 48, 64) and torch.equal(lin.weight_rows(), q)
    assert torch.equal(lin.weight[1, 5], q[5, 64:])  # byte (n, k) at ((k // 64) * out + n) * 64 + k % 64
    sd = lin.state_dict()
    assert torch.equal(sd["weight"], q) and torch.equal(lin.weight_rows(), q)  # the buffer is untouched
    other = quant.QuantLinear(128, 48, mode="int8", dtype=torch.bfloat16, device="cpu")
    other.load_state_dict(sd)
    assert torch.equal(other.weight, lin.weight)
    with pytest.raises(ValueError):
        lin.set_weight_rows(q[:, :64])
    # K not a multiple of 64: row-major storage
    narrow = quant.QuantLinear(80, 16, mode="int8", dtype=torch.bfloat16, device="cpu")
    assert narrow.weight.shape == (16, 80) and narrow.state_dict()["weight"].shape == (16, 80)
