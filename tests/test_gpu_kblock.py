"""GPU parity of the K-blocked operand layout (D3W8A8_KBLOCK for activations, D3W8A8_W_KBLOCK for weights).

K-blocked quantized activations hold byte (m, k) at ((k // 64) * ld + m) * 64 + k % 64: a permutation
of the row-major bytes. Every quantize entry point must write, K-blocked, exactly the codes and scales
it writes row-major, and every pipelined GEMM tile must return, from a K-blocked A, exactly what it
returns from the row-major A (its MFMAs read the same operands in the same K order). The row-major
paths are pinned against the oracle by the other GPU tests; these chain onto them bit for bit, INT8 and
FP8 alike, with row capacities above M (ld > M) as well as equal to it. The same holds for K-blocked
weights, alone and together with K-blocked activations.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import gen, rand_fp8, rand_i8
from d3trt_amd import _lib
from d3trt_amd import kernels as K
from d3trt_amd.mlp import QuantMLP
from d3trt_amd.quant import QuantLinear
from d3trt_amd.stack import StackLayer

pytestmark = pytest.mark.gpu


def to_kblock(a: torch.Tensor, cap: int | None = None) -> torch.Tensor:
    """Row-major [M, K] codes -> K-blocked [K // 64, M, 64] with row capacity ``cap`` (>= M)."""
    M, Kd = a.shape
    cap = M if cap is None else cap
    buf = torch.full((Kd // 64, cap, 64), 0x7F, dtype=torch.uint8, device=a.device)  # junk past row M
    buf[:, :M] = a.contiguous().view(torch.uint8).reshape(M, Kd // 64, 64).permute(1, 0, 2)
    return buf.view(a.dtype)[:, :M]


def codes(mode, g, M, Kd):
    return rand_i8(g, M, Kd) if mode == "int8" else rand_fp8(g, M, Kd)


def same_bytes(x: torch.Tensor, y: torch.Tensor) -> bool:
    return x.shape == y.shape and torch.equal(x.contiguous().view(torch.uint8), y.contiguous().view(torch.uint8))


GEMM_SHAPES = [(1, 64, 256), (45, 320, 512), (128, 1024, 4096), (300, 576, 1024), (520, 768, 2048)]


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("tile", [_lib.TILE_AUTO, *_lib.DMA_TILES])
@pytest.mark.parametrize("M,N,Kd", GEMM_SHAPES)
def test_gemm_kblock_equals_row_major(dev, mode, tile, M, N, Kd):
    g = gen(M * 7 + N * 3 + Kd + (mode == "fp8"))
    a, w = codes(mode, g, M, Kd).to(dev), codes(mode, g, N, Kd).to(dev)
    s_a = (torch.rand(M, generator=g) * 1e-2 + 1e-4).to(dev)
    s_w = (torch.rand(N, generator=g) * 1e-2 + 1e-4).to(dev)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    a_kb = to_kblock(a, cap=M + 3 * (M % 2))
    w_kb = to_kblock(w, cap=N + 5 * (N % 3 == 0))
    # K-blocked a, K-blocked w, both
    variants = ((a_kb, w), (a, w_kb), (a_kb, w_kb))
    print(f"kblock gemm {mode} tile={tile} {M}x{N}x{Kd}", flush=True)
    for epi in (_lib.EPI_RAW, _lib.EPI_DEQUANT, _lib.EPI_RESIDUAL):
        kw = dict(epilogue=epi, tile=tile, residual=res if epi == _lib.EPI_RESIDUAL else None)
        sa, sw = (None, None) if epi == _lib.EPI_RAW else (s_a, s_w)
        ref = K.gemm(mode, a, sa, w, sw, **kw)
        for v, (av, wv) in enumerate(variants):
            assert torch.equal(K.gemm(mode, av, sa, wv, sw, **kw), ref), (epi, tile, v)
    if tile not in _lib.NO_SWIGLU_TILES:  # SwiGLU needs gate/up column pairs
        amax_r = torch.zeros(M, device=dev)
        h_r = K.gemm(mode, a, s_a, w, s_w, epilogue=_lib.EPI_SWIGLU, tile=tile, row_amax=amax_r)
        for v, (av, wv) in enumerate(variants):
            amax_k = torch.zeros(M, device=dev)
            h_k = K.gemm(mode, av, s_a, wv, s_w, epilogue=_lib.EPI_SWIGLU, tile=tile, row_amax=amax_k)
            assert torch.equal(h_k, h_r) and torch.equal(amax_k, amax_r), v


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("tile,ksplit", [(_lib.TILE_DMA_128_W4, 4), (_lib.TILE_DMA_128_W4_K128, 8),
                                         (_lib.TILE_DMA_128_W4_K128, _lib.KSPLIT_AUTO)])
def test_split_k_kblock_equals_row_major(dev, mode, tile, ksplit):
    g = gen(11 + tile + ksplit)
    M, N, Kd = 100, 1024, 4096
    a, w = codes(mode, g, M, Kd).to(dev), codes(mode, g, N, Kd).to(dev)
    s_a, s_w = torch.rand(M, generator=g).to(dev), torch.rand(N, generator=g).to(dev)
    a_kb, w_kb = to_kblock(a, cap=128), to_kblock(w)
    for noalloc in (False, True):
        ref = K.gemm(mode, a, s_a, w, s_w, tile=tile, ksplit=ksplit, noalloc=noalloc)
        for av, wv in ((a_kb, w), (a, w_kb), (a_kb, w_kb)):
            assert torch.equal(K.gemm(mode, av, s_a, wv, s_w, tile=tile, ksplit=ksplit, noalloc=noalloc), ref), noalloc


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("walk", ["0", "1"])
def test_many_tiles_kblock_equals_row_major(dev, mode, walk, monkeypatch):
    """More 256x256 tiles than CUs, one workgroup per tile and (D3W8A8_GEMM_PERSIST=1) the persistent walk,
    where each workgroup walks several tiles (their prologue DMAs issued inside the previous tile's
    epilogue)."""
    monkeypatch.setenv("D3W8A8_GEMM_PERSIST", walk)
    g = gen(5 + (mode == "fp8"))
    M, N, Kd = 2048 + 100, 8448, 256
    a, w = codes(mode, g, M, Kd).to(dev), codes(mode, g, N, Kd).to(dev)
    s_a, s_w = torch.rand(M, generator=g).to(dev), torch.rand(N, generator=g).to(dev)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    a_kb, w_kb = to_kblock(a), to_kblock(w)
    for tile in (_lib.TILE_AUTO, _lib.TILE_DMA_256_W4):
        ref = K.gemm(mode, a, s_a, w, s_w, tile=tile, epilogue=_lib.EPI_RESIDUAL, residual=res)
        for av, wv in ((a_kb, w), (a_kb, w_kb)):
            out = K.gemm(mode, av, s_a, wv, s_w, tile=tile, epilogue=_lib.EPI_RESIDUAL, residual=res)
            assert torch.equal(out, ref), tile


QUANT_SHAPES = [(1, 64), (37, 4096), (300, 1024), (129, 12288)]


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,Kd", QUANT_SHAPES)
def test_quantize_rows_kblock(dev, mode, dtype, M, Kd):
    x = R.outlier_activations(gen(M + Kd), M, Kd).to(dtype).to(dev)
    q, s = K.quantize_rows(x, mode)
    qk, sk = K.quantize_rows(x, mode, kblock=True)
    assert qk.shape == (Kd // 64, M, 64)
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s)
    # rows that are not 16-byte aligned take the generic two-pass kernel, which writes the same layout
    big = torch.zeros(M, Kd + 8, dtype=dtype, device=dev)
    big[:, 1:Kd + 1] = x
    q2, s2 = K.quantize_rows(big[:, 1:Kd + 1], mode, kblock=True)
    assert same_bytes(K.unblock(q2), q) and torch.equal(s2, s)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,Kd", [(1, 64), (200, 4096), (1500, 2048)])
def test_rmsnorm_quantize_kblock(dev, mode, M, Kd):
    """Both norm kernels: the block-per-row one (M <= 1024) and the row pipeline."""
    g = gen(M * 5 + Kd)
    x = R.outlier_activations(g, M, Kd).to(torch.bfloat16).to(dev)
    w = (0.1 * torch.randn(Kd, generator=g)).to(torch.bfloat16).to(dev)
    amax_r, amax_k = torch.ones(M, device=dev), torch.ones(M, device=dev)
    q, s, n = K.rmsnorm_quantize(x, w, 1e-6, mode, want_normed=True, clear_amax=amax_r)
    qk, sk, nk = K.rmsnorm_quantize(x, w, 1e-6, mode, want_normed=True, clear_amax=amax_k, kblock=True)
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s) and torch.equal(nk, n)
    assert torch.equal(amax_k, amax_r)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("M,Kd", [(3, 128), (300, 12288)])
def test_quantize_rows_amax_kblock(dev, mode, M, Kd):
    g = gen(M + 2 * Kd)
    h = R.outlier_activations(g, M, Kd).to(torch.bfloat16).to(dev)
    amax = h.float().abs().amax(dim=1).contiguous()
    q, s = K.quantize_rows_amax(h, amax, mode)
    qk, sk = K.quantize_rows_amax(h, amax, mode, kblock=True)
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("head_dim", [0, 256])
def test_gate_quantize_kblock(dev, mode, head_dim):
    g = gen(17 + head_dim)
    M, Kd = 77, 2048
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(M, 2 * Kd if head_dim else Kd, generator=g).to(torch.bfloat16).to(dev)
    q, s, y = K.gate_quantize(x, gate, mode, gate_head_dim=head_dim, want_y=True)
    qk, sk, yk = K.gate_quantize(x, gate, mode, gate_head_dim=head_dim, want_y=True, kblock=True)
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s) and torch.equal(yk, y)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_gdn_norm_quantize_kblock(dev, mode):
    g = gen(23)
    M, Kd, hd = 65, 4096, 128
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16).to(dev)
    z = torch.randn(M, Kd, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(hd, generator=g)).to(torch.bfloat16).to(dev)
    q, s, y = K.gdn_norm_quantize(x, z, w, 1e-6, hd, mode, want_y=True)
    qk, sk, yk = K.gdn_norm_quantize(x, z, w, 1e-6, hd, mode, want_y=True, kblock=True)
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s) and torch.equal(yk, y)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("lengths", [[16, 0, 9, 16], [0, 0], [5]])
def test_ragged_kblock(dev, mode, lengths):
    g = gen(sum(lengths) + len(lengths))
    B, W, H, N = len(lengths), 16, 1024, 576
    x = R.outlier_activations(g, B * W, H).to(torch.bfloat16).reshape(B, W, H).to(dev)
    wq = codes(mode, g, N, H).to(dev)
    w_s = torch.rand(N, generator=g).to(dev)
    outs = []
    for kb in (False, True):
        out = torch.full((B * W, N), 3.0, dtype=torch.bfloat16, device=dev)
        q, s, row_map = K.quantize_rows_ragged(x, lengths, mode, out=out, kblock=kb)
        if row_map.numel():
            K.gemm(mode, q, s.reshape(-1), wq, w_s, out=out, row_map=row_map)
        outs.append((q, s, row_map, out))
    (q, s, rm, o), (qk, sk, rmk, ok) = outs
    assert same_bytes(K.unblock(qk), q) and torch.equal(sk, s) and torch.equal(rmk, rm) and torch.equal(ok, o)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("lengths,W,H", [([0, 7, 1, 0, 13], 13, 4096), ([3] * 40, 5, 512),
                                         ([1, 119, 57], 119, 12288), ([2, 0], 4, 64)])
def test_ragged_kblock_pairs(dev, mode, dtype, lengths, W, H):
    """The ragged gather into a K-blocked q against the row-major one: empty segments first and in
    between, odd totals, every input dtype, short and long rows, with and without the zeroed output."""
    g = gen(len(lengths) * 131 + W + H)
    B, N = len(lengths), 64
    x = R.outlier_activations(g, B * W, H).to(dtype).reshape(B, W, H).to(dev)
    print(f"ragged pairs {mode} {dtype} lengths={lengths} W={W} H={H}", flush=True)
    for with_out in (False, True):
        res = []
        for kb in (False, True):
            out = torch.full((B * W, N), 3.0, dtype=torch.bfloat16, device=dev) if with_out else None
            q, s, rm = K.quantize_rows_ragged(x, lengths, mode, out=out, kblock=kb)
            res.append((K.unblock(q) if kb else q, s, rm, out))
        (q, s, rm, o), (qk, sk, rmk, ok) = res
        assert same_bytes(qk, q) and torch.equal(sk, s) and torch.equal(rmk, rm)
        if with_out:
            assert torch.equal(ok, o)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_modules_kblock_equal_row_major(dev, mode):
    """QuantLinear.forward / forward_ragged, the MLP block and a stack layer: the K-blocked hand-off between
    quantize and GEMM (the default where K % 64 == 0) returns what the row-major one does."""
    g = gen(31 + (mode == "fp8"))
    torch.manual_seed(0)
    H, Q, I, M = 512, 768, 1024, 300
    lin = QuantLinear(H, Q, mode=mode, dtype=torch.bfloat16, device=dev)
    lin.load_full(R.gaussian_weight(g, Q, H).to(dev))
    mlp = QuantMLP(H, I, mode=mode, dtype=torch.bfloat16, device=dev)
    mlp.load_full(R.gaussian_weight(g, 2 * I, H).to(dev), R.gaussian_weight(g, H, I).to(dev))
    layer = StackLayer(H, Q, I, mode=mode, dtype=torch.bfloat16, device=dev)
    for m in (layer.qkv_proj, layer.o_proj):
        m.load_full(R.gaussian_weight(g, m.out_features, m.in_features).to(dev))
    layer.mlp.load_full(R.gaussian_weight(g, 2 * I, H).to(dev), R.gaussian_weight(g, H, I).to(dev))
    x = R.outlier_activations(g, M, H).to(torch.bfloat16).to(dev)
    xr = x[:48].reshape(3, 16, H)
    nw = (0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    mods = [lin, mlp.gate_up_proj, mlp.down_proj, layer.qkv_proj, layer.o_proj, layer.mlp.gate_up_proj,
            layer.mlp.down_proj]
    assert all(m.kblock for m in mods)
    runs = []
    for kb in (True, False):
        for m in mods:
            m.kblock = kb
        runs.append([lin(x), lin.forward_ragged(xr, [16, 3, 11]), mlp(x), mlp.block(x, nw, 1e-6), layer(x)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
