"""GPU parity: SwiGLU / residual epilogues, the fused MLP block, and the ragged-M mode."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rel_err
from d3trt_amd import _lib
from d3trt_amd import kernels as K
from d3trt_amd.mlp import QuantMLP
from d3trt_amd.quant import QuantLinear

pytestmark = pytest.mark.gpu


def _swiglu_case(g, M, H, I, mode):
    x = R.outlier_activations(g, M, H)
    gate_up = torch.cat([R.gaussian_weight(g, I, H), R.gaussian_weight(g, I, H)], dim=0)
    wq, ws = R.quantize_weight(gate_up, mode)
    q, s = R.quantize_rows(x, mode)
    return x, wq, ws, q, s


@pytest.mark.parametrize("mode", ["int8", "fp8"])
@pytest.mark.parametrize("tile", list(_lib.TILES))
@pytest.mark.parametrize("M,H,I", [(96, 512, 256), (300, 1024, 1024)])
def test_swiglu_epilogue(dev, mode, tile, M, H, I):
    g = gen(M + H + I)
    x, wq, ws, q, s = _swiglu_case(g, M, H, I, mode)
    wq_il = K.interleave_gate_up(wq.view(torch.uint8)).view(wq.dtype)
    ws_il = K.interleave_gate_up(ws)
    assert torch.equal(K.deinterleave_gate_up(ws_il), ws)
    amax = torch.zeros(M, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    if tile in _lib.NO_SWIGLU_TILES:  # three 32-column blocks per wave: no gate/up pairs
        with pytest.raises(ValueError, match="SwiGLU"):
            K.gemm(mode, q.to(dev), s.reshape(-1).to(dev), wq_il.to(dev), ws_il.to(dev), epilogue=_lib.EPI_SWIGLU,
                   out=h, row_amax=amax, tile=tile)
        return
    K.gemm(mode, q.to(dev), s.reshape(-1).to(dev), wq_il.to(dev), ws_il.to(dev), epilogue=_lib.EPI_SWIGLU,
           out=h, row_amax=amax, tile=tile)
    h = h.cpu()
    acc = R.int_accumulate(q, wq) if mode == "int8" else R.fp8_accumulate(q, wq)
    h_ref = R.swiglu(R.dequant(acc, s, ws, torch.bfloat16))
    d = bf16_ulp_diff(h, h_ref)
    if mode == "int8":
        # same bf16 gate/up; only expf's last bit may differ between the GPU and CPU libm
        assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    else:
        assert rel_err(h, h_ref) < 1e-2
    assert torch.equal(amax.cpu(), h.float().abs().amax(dim=1))


@pytest.mark.parametrize("tile", list(_lib.TILES))
def test_residual_epilogue_int8_bit_exact(dev, tile):
    g = gen(99)
    M, N, Kd = 130, 640, 1536
    x = R.outlier_activations(g, M, Kd)
    res = R.outlier_activations(g, M, N)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    q, s = R.quantize_rows(x, "int8")
    out = K.gemm("int8", q.to(dev), s.reshape(-1).to(dev), wq.to(dev), ws.to(dev), epilogue=_lib.EPI_RESIDUAL,
                 residual=res.to(dev), tile=tile)
    ref = res + R.dequant(R.int_accumulate(q, wq), s, ws, torch.bfloat16)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_mlp_block_staged(dev, mode):
    """Fused MLP block (norm -> quant -> gate_up+SwiGLU -> requant -> down+residual), each stage
    checked on the GPU's own inputs to that stage; the end-to-end output against the pure oracle."""
    g = gen(4)
    M, H, I = 256, 1024, 2048
    x = R.outlier_activations(g, M, H)
    norm_w = (0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    gate_up = torch.cat([R.gaussian_weight(g, I, H), R.gaussian_weight(g, I, H)], dim=0)
    down = R.gaussian_weight(g, H, I)
    mlp = QuantMLP(H, I, mode=mode, dtype=torch.bfloat16, device=dev)
    mlp.load_full(gate_up.to(dev), down.to(dev))
    out = mlp.block(x.to(dev), norm_w.to(dev), 1e-6).cpu()
    assert mlp.gate_up_proj.kernel == ("hip-i8" if mode == "int8" else "hip-f8")

    # staged: run the same launches and check each against the oracle on its own inputs
    xd = x.to(dev)
    amax = torch.empty(M, device=dev)
    q1, s1, normed = K.rmsnorm_quantize(xd, norm_w.to(dev), 1e-6, mode, want_normed=True, clear_amax=amax)
    q1_ref, s1_ref = R.quantize_rows(normed.cpu(), mode)
    assert torch.equal(q1.cpu().view(torch.uint8), q1_ref.view(torch.uint8))
    h, q2, s2 = mlp._swiglu_requant(q1, s1, amax)
    q2 = K.unblock(q2) if q2.dim() == 3 else q2  # the block hands q2 to down K-blocked
    wq_gu, ws_gu = R.quantize_weight(gate_up, mode)
    acc1 = R.int_accumulate(q1_ref, wq_gu) if mode == "int8" else R.fp8_accumulate(q1_ref, wq_gu)
    h_ref = R.swiglu(R.dequant(acc1, s1_ref, ws_gu, torch.bfloat16))
    if mode == "int8":
        d = bf16_ulp_diff(h.cpu(), h_ref)
        assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3
    else:
        assert rel_err(h.cpu(), h_ref) < 1e-2
    q2_ref, s2_ref = R.quantize_rows(h.cpu(), mode)
    assert torch.equal(s2.cpu(), s2_ref)
    assert torch.equal(q2.cpu().view(torch.uint8), q2_ref.view(torch.uint8))
    wq_d, ws_d = R.quantize_weight(down, mode)
    acc2 = R.int_accumulate(q2_ref, wq_d) if mode == "int8" else R.fp8_accumulate(q2_ref, wq_d)
    out_staged = x + R.dequant(acc2, s2_ref, ws_d, torch.bfloat16)
    if mode == "int8":
        assert torch.equal(out, out_staged)
    else:
        assert float((bf16_ulp_diff(out, out_staged) <= 1).float().mean()) > 0.99
    # end to end against the pure oracle chain (its own norm / SwiGLU roundings)
    full = R.mlp_block(x, norm_w, 1e-6, wq_gu, ws_gu, wq_d, ws_d, mode)
    assert rel_err(out - x, full["out"] - x) < 2e-2


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_ragged_equals_separate_blocks(dev, mode):
    """16 question blocks with lengths in [32, 128] packed into one launch == 16 separate GEMMs."""
    g = gen(2024)
    lengths = torch.randint(32, 129, (16,), generator=g).tolist()
    W, Kd, N = max(lengths), 4096, 1024
    x = torch.zeros(16, W, Kd, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        x[b, :n] = R.outlier_activations(g, n, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), mode)
    lin = QuantLinear(Kd, N, mode=mode, dtype=torch.bfloat16, device=dev)
    lin.set_weight_rows(wq.to(dev))
    lin.weight_scale.copy_(ws.to(dev))
    xd = x.to(dev)
    out = lin.forward_ragged(xd, lengths).cpu()
    for b, n in enumerate(lengths):
        sep = lin(xd[b, :n]).cpu()
        assert torch.equal(out[b, :n], sep)
        assert torch.all(out[b, n:] == 0)
    if mode == "int8":
        q, s, row_map = K.quantize_rows_ragged(xd, lengths, mode)
        raw = K.gemm(mode, q, None, lin.weight, None, epilogue=_lib.EPI_RAW).cpu()
        start = 0
        for b, n in enumerate(lengths):
            qb, _ = K.quantize_rows(xd[b, :n], mode)
            sep_raw = K.gemm(mode, qb, None, lin.weight, None, epilogue=_lib.EPI_RAW).cpu()
            assert torch.equal(raw[start:start + n], sep_raw)
            assert torch.equal(row_map[start:start + n].cpu(), torch.arange(b * W, b * W + n, dtype=torch.int32))
            start += n
        qr, _ = R.quantize_rows(torch.cat([x[b, :n] for b, n in enumerate(lengths)]), mode)
        assert torch.equal(raw.to(torch.int64), R.int_accumulate(qr, wq))


def test_ragged_with_empty_blocks(dev):
    g = gen(7)
    lengths = [0, 5, 0, 17, 1]
    W, Kd, N = 20, 256, 128
    x = torch.zeros(len(lengths), W, Kd, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, Kd)
    wq, ws = R.quantize_weight(R.gaussian_weight(g, N, Kd), "int8")
    lin = QuantLinear(Kd, N, mode="int8", dtype=torch.bfloat16, device=dev)
    lin.set_weight_rows(wq.to(dev))
    lin.weight_scale.copy_(ws.to(dev))
    out = lin.forward_ragged(x.to(dev), lengths).cpu()
    for b, n in enumerate(lengths):
        if n:
            ref = R.linear_forward(x[b, :n], wq, ws, "int8", torch.bfloat16)
            assert torch.equal(out[b, :n], ref)
        assert torch.all(out[b, n:] == 0)
    zero = lin.forward_ragged(x.to(dev), [0] * len(lengths)).cpu()
    assert torch.all(zero == 0)
