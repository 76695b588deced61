"""GPU parity: the backbone projection stack (identity mixer) and its ragged question pass."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import bf16_ulp_diff, gen, rel_err
from d3trt_amd import LinearStack
from d3trt_amd import _lib
from d3trt_amd import kernels as K

pytestmark = pytest.mark.gpu

H, QKV, I = 512, 768, 1024


def _stack(dev, layers, mode, seed):
    st = LinearStack(layers, H, QKV, I, mode=mode, device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(seed))
    return st


def _oracle_weights(layer, mode):
    """Quantized weights of one layer in the oracle's layout (gate_up back in [gate; up] order)."""
    gu = layer.mlp.gate_up_proj
    wgu_q = K.deinterleave_gate_up(gu.weight_rows().view(torch.uint8)).view(gu.weight.dtype).cpu()
    wgu_s = K.deinterleave_gate_up(gu.weight_scale).cpu()
    return dict(w_in=layer.input_layernorm.cpu(), w_post=layer.post_attention_layernorm.cpu(),
                wqkv_q=layer.qkv_proj.weight_rows().cpu(), wqkv_s=layer.qkv_proj.weight_scale.cpu(),
                wo_q=layer.o_proj.weight_rows().cpu(), wo_s=layer.o_proj.weight_scale.cpu(),
                wgu_q=wgu_q, wgu_s=wgu_s, wd_q=layer.mlp.down_proj.weight_rows().cpu(),
                wd_s=layer.mlp.down_proj.weight_scale.cpu())


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_stack_layer_matches_oracle(dev, mode):
    st = _stack(dev, 1, mode, 1)
    x = R.outlier_activations(gen(5), 200, H)
    out = st(x.to(dev)).cpu()
    ref = R.stack_layer(x, mode=mode, **_oracle_weights(st.layers[0], mode))
    # norm reductions run in a different order than torch's CPU mean (one bf16 ulp, rarely), which can
    # move a per-token scale: the block output is held to the FP8 bar in both modes, the INT8 stages
    # below bit-exactly on the GPU's own inputs
    assert rel_err(out - x, ref["out"] - x) < 2e-2
    if mode == "int8":
        layer = st.layers[0]
        xd = x.to(dev)
        q1, s1, normed = K.rmsnorm_quantize(xd, layer.input_layernorm, 1e-6, mode, want_normed=True)
        w = _oracle_weights(layer, mode)
        qkv_ref = R.int8_linear(normed.cpu(), w["wqkv_q"], w["wqkv_s"], torch.bfloat16)[0]
        qkv = K.gemm(mode, q1, s1.view(-1), layer.qkv_proj.weight, layer.qkv_proj.weight_scale)
        assert torch.equal(qkv.cpu(), qkv_ref)
        o_ref = R.int8_linear(qkv_ref[:, :H], w["wo_q"], w["wo_s"], torch.bfloat16)[0]
        q2, s2 = K.quantize_rows(qkv[:, :H], mode)
        h = K.gemm(mode, q2, s2.view(-1), layer.o_proj.weight, layer.o_proj.weight_scale, epilogue=_lib.EPI_RESIDUAL,
                   residual=xd)
        assert torch.equal(h.cpu(), x + o_ref)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_stack_ragged_equals_per_block(dev, mode):
    """Packed question pass == each block through the dense stack, bit for bit; padded rows zero."""
    st = _stack(dev, 2, mode, 2)
    g = gen(9)
    lengths = [5, 16, 0, 11, 16, 1]
    W = 16
    x = torch.zeros(len(lengths), W, H, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, H)
    xd = x.to(dev)
    out = st.forward_ragged(xd, lengths).cpu()
    for b, n in enumerate(lengths):
        if n:
            assert torch.equal(out[b, :n], st(xd[b, :n]).cpu())
        assert torch.all(out[b, n:] == 0)


def test_stack_two_layers_fp8_against_oracle(dev):
    st = _stack(dev, 2, "fp8", 3)
    x = R.outlier_activations(gen(6), 64, H)
    out = st(x.to(dev)).cpu()
    ref = x
    for layer in st.layers:
        ref = R.stack_layer(ref, mode="fp8", **_oracle_weights(layer, "fp8"))["out"]
    assert rel_err(out - x, ref - x) < 3e-2
    assert float((bf16_ulp_diff(out, ref) <= 2).float().mean()) > 0.9


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_graph_replays_match_eager(dev, mode):
    """Each replay of the captured stack equals the eager pass on the same input, with eager work and
    synchronizations between the replays."""
    st = _stack(dev, 2, mode, 4)
    g = gen(10)
    xs = [R.outlier_activations(g, 48, H).to(dev) for _ in range(3)]
    graphed = st.graphed(48)
    for x in xs:
        eager = st(x).clone()
        st(xs[0])  # unrelated eager work between replays
        torch.cuda.synchronize()
        out = graphed(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_fp16_stack_graph_replays_match_eager(dev, mode):
    """An fp16 stack: the captured pass takes fp16 rows (its norm weights' dtype), dense and ragged."""
    st = LinearStack(2, H, QKV, I, mode=mode, dtype=torch.float16, device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(21))
    g = gen(22)
    x = R.outlier_activations(g, 32, H).to(torch.float16).to(dev)
    eager = st(x).clone()
    assert eager.dtype == torch.float16
    graphed = st.graphed(32)
    for _ in range(3):
        st(x)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(graphed(x).clone(), eager)
    lengths = [16, 5, 0, 11]
    xr = torch.zeros(len(lengths), 16, H, dtype=torch.float16)
    for b_, n in enumerate(lengths):
        if n:
            xr[b_, :n] = R.outlier_activations(g, n, H).to(torch.float16)
    xr = xr.to(dev)
    ragged = st.forward_ragged(xr, lengths).clone()
    assert torch.equal(st.forward_ragged(xr, lengths, graph=True), ragged)
    for b_, n in enumerate(lengths):
        if n:
            assert torch.equal(ragged[b_, :n], st(xr[b_, :n]))


def test_graphed_ragged_pass_equals_eager(dev):
    st = _stack(dev, 2, "int8", 5)
    g = gen(11)
    lengths = [16, 3, 16, 0, 9]
    x = torch.zeros(len(lengths), 16, H, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        if n:
            x[b, :n] = R.outlier_activations(g, n, H)
    xd = x.to(dev)
    eager = st.forward_ragged(xd, lengths).clone()
    for _ in range(3):
        assert torch.equal(st.forward_ragged(xd, lengths, graph=True), eager)
