"""GPU parity at the benchmark workloads' own sizes.

  C1  single INT8 linear, 128 x 1024 x 1024, seed 0, against the reference's CPU path
      (QuantLinear._emulated, d3trt/model/quant.py:158-162), bit for bit
  C3  ragged INT8 question batch: 16 blocks of 32-128 rows, K = 4096, N = 6144 / 4096 / 24576,
      packed == 16 separate GEMMs == the int64 oracle, on every tile the packed shape can take
  C4  INT8 MLP block at M = 4096, hidden 4096, intermediate 12288, stage by stage on sampled rows,
      with the agreement of the requantized codes against the pure CPU chain reported
  C5  one full-width FP8 layer of the projection stack at the 8192-token state pass (sampled rows
      against the oracle layer), and packed question passes over mixed-length blocks == per-block
      dense runs

The full-size CPU oracle work is done on sampled rows: every output row depends on its own input
row only (per-token scales, row-wise norm), so a row sample is checked exactly as a full run would.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rel_err
from d3trt_amd import LinearStack, QuantLinear, QuantMLP
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu


def _sample_rows(M: int, n: int, seed: int) -> torch.Tensor:
    """n distinct rows of [0, M): the first and last row plus a seeded draw."""
    g = gen(seed)
    rest = torch.randperm(M - 2, generator=g)[: n - 2] + 1
    return torch.cat([torch.tensor([0, M - 1]), rest]).sort().values


# ------------------------------------------------------------------------------------------- C1
def test_c1_single_int8_linear_seed0_equals_reference_cpu_path(dev):
    """BASELINE draw order at seed 0: x = randn(128, 1024) with round(0.01 K) = 10 outlier channels
    (randperm) scaled by 20, to bf16; then W = 0.02 randn(1024, 1024) to bf16. At K = 1024 every
    partial sum of the reference's fp32 accumulation is an integer below 2^24 (1024 * 127^2), so its
    emulated output is exact, and the HIP linear must equal it bit for bit."""
    g = torch.Generator().manual_seed(0)
    M, Kd, N = 128, 1024, 1024
    x = R.outlier_activations(g, M, Kd)
    w = R.gaussian_weight(g, N, Kd)
    wq_ref, ws_ref = R.quantize_weight(w, "int8")
    lin = QuantLinear(Kd, N, mode="int8", dtype=torch.bfloat16, device=dev)
    lin.load_full(w.to(dev))
    assert torch.equal(lin.weight_rows().cpu(), wq_ref) and torch.equal(lin.weight_scale.cpu(), ws_ref)
    out = lin(x.to(dev)).cpu()
    assert lin.kernel == "hip-i8"
    ref = R.emulated_linear(x, wq_ref, ws_ref, "int8", torch.bfloat16)
    assert torch.equal(out, ref)
    # and the int32 accumulators against the int64 brute force
    q, s = K.quantize_rows(x.to(dev), "int8")
    raw = K.gemm("int8", q, None, lin.weight, None, epilogue=_lib.EPI_RAW).cpu()
    assert torch.equal(raw.to(torch.int64), R.int_accumulate_bruteforce(q.cpu(), wq_ref))


# ------------------------------------------------------------------------------------------- C3
def _c3_batch():
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(32, 129, (16,), generator=g).tolist()
    W, Kd = max(lengths), 4096
    x = torch.zeros(16, W, Kd, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        x[b, :n] = R.outlier_activations(g, n, Kd)
    return g, lengths, x


@pytest.mark.parametrize("N", [6144, 4096, 24576])
def test_c3_ragged_int8_full_width(dev, N):
    g, lengths, x = _c3_batch()
    B, W, Kd = x.shape
    T = sum(lengths)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    wd, wsd = wq.to(dev), ws.to(dev)
    xd = x.to(dev)
    q, s, row_map = K.quantize_rows_ragged(xd, lengths, "int8")
    # the 16 blocks one by one (their own launches, their own tiles)
    sep_raw, sep_out = [], []
    for b, n in enumerate(lengths):
        qb, sb = K.quantize_rows(xd[b, :n], "int8")
        sep_raw.append(K.gemm("int8", qb, None, wd, None, epilogue=_lib.EPI_RAW))
        sep_out.append(K.gemm("int8", qb, sb.view(-1), wd, wsd))
    sep_raw = torch.cat(sep_raw)
    # packed, on the automatic tile and on every pipelined tile that takes a ragged batch of this size
    tiles = [_lib.TILE_AUTO, _lib.TILE_DMA_256_W4, _lib.TILE_DMA_256x192_W4, _lib.TILE_DMA_256x128_W4,
             _lib.TILE_DMA_128_W4, _lib.TILE_DMA_192x192_W4, _lib.TILE_DMA_192x128_W4]
    for tile in tiles:
        raw = K.gemm("int8", q, None, wd, None, epilogue=_lib.EPI_RAW, tile=tile)
        assert torch.equal(raw, sep_raw), f"tile {tile}: packed raw accumulators differ from separate GEMMs"
        out = torch.full((B * W, N), 7.0, dtype=torch.bfloat16, device=dev)
        K.quantize_rows_ragged(xd, lengths, "int8", out=out)  # zeroes the padded rows
        K.gemm("int8", q, s.view(-1), wd, wsd, out=out, row_map=row_map, tile=tile)
        out = out.view(B, W, N)
        for b, n in enumerate(lengths):
            assert torch.equal(out[b, :n], sep_out[b]), f"tile {tile}: block {b} differs"
            assert torch.all(out[b, n:] == 0)
    # int64 oracle on a row sample of the packed batch (every column)
    rows = _sample_rows(T, 48, N)
    x_packed = torch.cat([x[b, :n] for b, n in enumerate(lengths)])
    q_ref, _ = R.quantize_rows(x_packed[rows], "int8")
    assert torch.equal(q.cpu()[rows], q_ref)
    assert torch.equal(sep_raw.cpu()[rows].to(torch.int64), R.int_accumulate(q_ref, wq))


# ------------------------------------------------------------------------------------------- C4
def test_c4_mlp_block_int8_full_size(dev):
    """M = 4096, hidden 4096, intermediate 12288, INT8; norm weight N(1, 0.1) applied as (1 + w)."""
    g = torch.Generator().manual_seed(0)
    M, H, I = 4096, 4096, 12288
    x = R.outlier_activations(g, M, H)
    gate_up = torch.cat([R.gaussian_weight(g, I, H), R.gaussian_weight(g, I, H)])
    down = R.gaussian_weight(g, H, I)
    norm_w = (0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    mlp = QuantMLP(H, I, mode="int8", dtype=torch.bfloat16, device=dev)
    mlp.load_full(gate_up.to(dev), down.to(dev))
    xd = x.to(dev)
    out = mlp.block(xd, norm_w.to(dev), 1e-6)

    # the same launches, stage by stage
    amax = torch.empty(M, device=dev)
    q1, s1, normed = K.rmsnorm_quantize(xd, norm_w.to(dev), 1e-6, "int8", want_normed=True, clear_amax=amax)
    h, q2, s2 = mlp._swiglu_requant(q1, s1, amax)
    q2 = K.unblock(q2) if q2.dim() == 3 else q2  # the block hands q2 to down K-blocked
    d = mlp.down_proj
    out2 = K.gemm("int8", q2, s2.view(-1), d.weight, d.weight_scale, epilogue=_lib.EPI_RESIDUAL, residual=xd)
    assert torch.equal(out, out2)

    rows = _sample_rows(M, 40, 4)
    wq_gu, ws_gu = R.quantize_weight(gate_up, "int8")
    wq_d, ws_d = R.quantize_weight(down, "int8")
    xs = x[rows]
    n_gpu = normed.cpu()[rows]
    d_norm = bf16_ulp_diff(n_gpu, R.rmsnorm(xs, norm_w, 1e-6))
    assert int(d_norm.max()) <= 1 and float((d_norm > 0).float().mean()) < 1e-3
    q1_ref, s1_ref = R.quantize_rows(n_gpu, "int8")
    assert torch.equal(q1.cpu()[rows], q1_ref) and torch.equal(s1.cpu()[rows], s1_ref)
    h_ref = R.swiglu(R.dequant(R.int_accumulate(q1_ref, wq_gu), s1_ref, ws_gu, torch.bfloat16))
    h_gpu = h.cpu()[rows]
    d_h = bf16_ulp_diff(h_gpu, h_ref)
    assert int(d_h.max()) <= 1 and float((d_h > 0).float().mean()) < 1e-3
    assert torch.equal(amax.cpu()[rows], h_gpu.float().abs().amax(dim=1))
    q2_ref, s2_ref = R.quantize_rows(h_gpu, "int8")
    assert torch.equal(q2.cpu()[rows], q2_ref) and torch.equal(s2.cpu()[rows], s2_ref)
    out_ref = xs + R.dequant(R.int_accumulate(q2_ref, wq_d), s2_ref, ws_d, torch.bfloat16)
    assert torch.equal(out.cpu()[rows], out_ref)

    # against the pure CPU chain (its own norm, SwiGLU and requant): how many requantized codes agree
    full = R.mlp_block(xs, norm_w, 1e-6, wq_gu, ws_gu, wq_d, ws_d, "int8")
    agree = float((q2.cpu()[rows] == full["q2"]).float().mean())
    print(f"C4 requantized-code agreement with the pure CPU chain: {agree:.6f} over {len(rows)} rows x {I}")
    # a norm or silu result one bf16 ulp apart moves a code only next to a rounding boundary, or a
    # whole row when it is the row's max
    assert agree > 0.99
    assert rel_err(out.cpu()[rows] - xs, full["out"] - xs) < 2e-2


# ------------------------------------------------------------------------------------------- C5
def _oracle_layer_weights(layer):
    gu = layer.mlp.gate_up_proj
    return dict(w_in=layer.input_layernorm.cpu(), w_post=layer.post_attention_layernorm.cpu(),
                wqkv_q=layer.qkv_proj.weight_rows().cpu(), wqkv_s=layer.qkv_proj.weight_scale.cpu(),
                wo_q=layer.o_proj.weight_rows().cpu(), wo_s=layer.o_proj.weight_scale.cpu(),
                wgu_q=K.deinterleave_gate_up(gu.weight_rows().view(torch.uint8)).view(gu.weight.dtype).cpu(),
                wgu_s=K.deinterleave_gate_up(gu.weight_scale).cpu(),
                wd_q=layer.mlp.down_proj.weight_rows().cpu(), wd_s=layer.mlp.down_proj.weight_scale.cpu())


@pytest.fixture(scope="module")
def c5_stack(dev):
    st = LinearStack(1, 4096, 6144, 12288, mode="fp8", device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(0))
    return st


def test_c5_state_pass_layer_fp8_full_width(dev, c5_stack):
    M = 8192
    x = torch.randn(M, 4096, generator=gen(0)).to(torch.bfloat16)
    out = c5_stack(x.to(dev)).cpu()
    rows = _sample_rows(M, 32, 5)
    ref = R.stack_layer(x[rows], mode="fp8", **_oracle_layer_weights(c5_stack.layers[0]))
    xs = x[rows]
    # the whole layer (four chained FP8 GEMMs, their intermediate rows requantized to E4M3) against
    # the oracle's own chain
    assert rel_err(out[rows] - xs, ref["out"] - xs) < 2e-2
    # each GEMM on the GPU's own quantized inputs against the float64-accumulated product: the
    # north star's 1e-2 bar per projection
    layer = c5_stack.layers[0]
    w = _oracle_layer_weights(layer)
    xd = x.to(dev)
    q1, s1, _ = K.rmsnorm_quantize(xd, layer.input_layernorm, 1e-6, "fp8")
    qkv = K.gemm("fp8", q1, s1.view(-1), layer.qkv_proj.weight, layer.qkv_proj.weight_scale)
    q1r, s1r = q1.cpu()[rows], s1.cpu()[rows]
    assert rel_err(qkv.cpu()[rows], R.dequant(R.fp8_accumulate(q1r, w["wqkv_q"]), s1r, w["wqkv_s"],
                                              torch.bfloat16)) < 1e-2
    amax = torch.empty(M, device=dev)
    q3, s3, _ = K.rmsnorm_quantize(xd, layer.post_attention_layernorm, 1e-6, "fp8", clear_amax=amax)
    h, q4, s4 = layer.mlp._swiglu_requant(q3, s3, amax)
    q4 = K.unblock(q4) if q4.dim() == 3 else q4  # the block hands q4 to down K-blocked
    q3r, s3r = q3.cpu()[rows], s3.cpu()[rows]
    gu = R.dequant(R.fp8_accumulate(q3r, w["wgu_q"]), s3r, w["wgu_s"], torch.bfloat16)
    assert rel_err(h.cpu()[rows], R.swiglu(gu)) < 1e-2
    down = K.gemm("fp8", q4, s4.view(-1), layer.mlp.down_proj.weight, layer.mlp.down_proj.weight_scale)
    q4r, s4r = q4.cpu()[rows], s4.cpu()[rows]
    assert rel_err(down.cpu()[rows], R.dequant(R.fp8_accumulate(q4r, w["wd_q"]), s4r, w["wd_s"],
                                               torch.bfloat16)) < 1e-2


def test_c5_mixed_length_question_pass_equals_per_block(dev, c5_stack):
    """Question blocks of mixed lengths (0 and 1 included) through the packed pass, eager and graph
    replayed, == each block through the dense stack. One batch of at most 128 rows (the reference's
    default batch of 8 blocks x 16 tokens), so packed and per-block runs take the same tiles."""
    lengths = [16, 1, 0, 9, 16, 3, 12, 16]
    Wd = 16
    x = torch.zeros(len(lengths), Wd, 4096, dtype=torch.bfloat16)
    g = gen(12)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = torch.randn(n, 4096, generator=g).to(torch.bfloat16)
    xd = x.to(dev)
    eager = c5_stack.forward_ragged(xd, lengths)
    graphed = c5_stack.forward_ragged(xd, lengths, graph=True).clone()
    assert torch.equal(graphed, eager)
    eager = eager.cpu()
    for b, n in enumerate(lengths):
        if n:
            assert torch.equal(eager[b, :n], c5_stack(xd[b, :n]).cpu()), f"block {b} ({n} rows)"
        assert torch.all(eager[b, n:] == 0)


def test_c5_mixed_length_question_pass_int8_any_size(dev):
    """INT8 is exact in any tiling: a packed pass over 24 mixed-length blocks (216 rows, beyond one
    128-row tile) equals every block through the dense stack bit for bit."""
    st = LinearStack(1, 4096, 6144, 12288, mode="int8", device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(1))
    lengths = [16, 1, 0, 9, 16, 3, 12, 16] * 3
    lengths[5] = 0
    Wd = 16
    x = torch.zeros(len(lengths), Wd, 4096, dtype=torch.bfloat16)
    g = gen(13)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, 4096)
    xd = x.to(dev)
    out = st.forward_ragged(xd, lengths).cpu()
    for b, n in enumerate(lengths):
        if n:
            assert torch.equal(out[b, :n], st(xd[b, :n]).cpu()), f"block {b} ({n} rows)"
        assert torch.all(out[b, n:] == 0)
