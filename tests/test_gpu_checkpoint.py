"""GPU: per-layer streaming of a bf16 checkpoint into the stack, its pre-quantized conversion, and
packed question passes over variable-length blocks."""

from __future__ import annotations

import pytest
import torch

from oracle import quant_ref as R
from tests._util import gen
from tests.test_checkpoint import write_checkpoint
from d3trt_amd import LinearStack, QuestionScheduler, ShardedCheckpoint, convert_checkpoint, \
    load_converted_stack, stream_into_stack
from d3trt_amd import kernels as K
from d3trt_amd.checkpoint import layer_names

pytestmark = pytest.mark.gpu

H, Q, KV, I = 256, 256, 128, 256


def _same(a, b):
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_streamed_weights_equal_oracle_quantization(dev, tmp_path, mode):
    """Every streamed projection's codes and scales equal the oracle's quantize_weight of the same bf16
    tensors (q|k|v concatenated; [gate; up] concatenated, then put in the interleaved SwiGLU order)."""
    tensors = write_checkpoint(tmp_path, layers=2, hidden=H, q=Q, kv=KV, inter=I)
    st = LinearStack(2, H, Q + 2 * KV, I, mode=mode, device=dev)
    info = stream_into_stack(st, ShardedCheckpoint(tmp_path))
    assert info["layers"] == 2 and info["bytes_read"] > 0
    for i, layer in enumerate(st.layers):
        n = layer_names(i)
        wq, ws = R.quantize_weight(torch.cat([tensors[n["q_proj"]], tensors[n["k_proj"]], tensors[n["v_proj"]]]), mode)
        assert _same(layer.qkv_proj.weight_rows().cpu(), wq) and torch.equal(layer.qkv_proj.weight_scale.cpu(), ws)
        wq, ws = R.quantize_weight(tensors[n["o_proj"]], mode)
        assert _same(layer.o_proj.weight_rows().cpu(), wq) and torch.equal(layer.o_proj.weight_scale.cpu(), ws)
        wq, ws = R.quantize_weight(torch.cat([tensors[n["gate_proj"]], tensors[n["up_proj"]]]), mode)
        gu = layer.mlp.gate_up_proj
        assert _same(K.deinterleave_gate_up(gu.weight_rows().view(torch.uint8)).cpu(), wq)
        assert torch.equal(K.deinterleave_gate_up(gu.weight_scale).cpu(), ws)
        wq, ws = R.quantize_weight(tensors[n["down_proj"]], mode)
        assert _same(layer.mlp.down_proj.weight_rows().cpu(), wq)
        assert torch.equal(layer.mlp.down_proj.weight_scale.cpu(), ws)
        assert torch.equal(layer.input_layernorm.cpu(), tensors[n["input_layernorm"]])
        assert torch.equal(layer.post_attention_layernorm.cpu(), tensors[n["post_attention_layernorm"]])


def test_shape_mismatch_raises(dev, tmp_path):
    write_checkpoint(tmp_path, layers=1, hidden=H, q=Q, kv=KV, inter=I)
    st = LinearStack(1, H, Q + 2 * KV, 2 * I, mode="int8", device=dev)  # intermediate too wide
    with pytest.raises(ValueError, match="shape mismatch"):
        stream_into_stack(st, tmp_path)


@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_converted_stack_computes_what_the_streamed_stack_computes(dev, tmp_path, mode):
    src = tmp_path / "bf16"
    src.mkdir()
    write_checkpoint(src, layers=2, hidden=H, q=Q, kv=KV, inter=I)
    idx = convert_checkpoint(src, tmp_path / "w8a8", layers=2, mode=mode, device=dev)
    assert idx.endswith(".json")
    back = load_converted_stack(tmp_path / "w8a8", device=dev)
    st = LinearStack(2, H, Q + 2 * KV, I, mode=mode, device=dev)
    stream_into_stack(st, src)
    x = R.outlier_activations(gen(3), 40, H).to(dev)
    assert torch.equal(back(x), st(x))


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("batch_size", [1, 3, 8, None])
def test_scheduler_equals_per_block_dense_runs(dev, graph, batch_size):
    """INT8 (exact in any tiling): variable-length blocks, 0 and 1 included, scheduled in packed batches,
    come back in input order equal to each block run through the dense stack on its own."""
    st = LinearStack(2, 512, 768, 1024, mode="int8", device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(7))
    g = gen(8)
    lengths = [5, 0, 16, 1, 33, 3, 9, 0, 12, 1, 7, 20]
    pieces = [R.outlier_activations(g, n, 512).to(dev) if n else torch.empty(0, 512, dtype=torch.bfloat16,
                                                                               device=dev) for n in lengths]
    res = QuestionScheduler(st, batch_size=batch_size, graph=graph).run(pieces)
    for i, n in enumerate(lengths):
        assert res.rows[i].shape == (n, 512)
        if n:
            dense = st(pieces[i])
            assert torch.equal(res.rows[i], dense), f"block {i} ({n} rows)"
            assert torch.equal(res.last[i], dense[-1])
        else:
            assert torch.all(res.last[i] == 0)
    assert sorted(i for b in res.batches for i in b.blocks) == list(range(len(lengths)))


def test_scheduler_fp8_batch_of_eight_equals_per_block(dev):
    """FP8 with the reference's default batch (8 blocks of <= 16 tokens: <= 128 packed rows, the tile
    per-block runs take as well): bit-equal to per-block dense runs."""
    st = LinearStack(1, 512, 768, 1024, mode="fp8", device=dev)
    st.init_random(torch.Generator(device=dev).manual_seed(9))
    g = gen(10)
    lengths = [16, 3, 1, 16, 8, 0, 11, 16, 5, 2]
    pieces = [torch.randn(n, 512, generator=g).to(torch.bfloat16).to(dev) for n in lengths]
    res = QuestionScheduler(st, batch_size=8, graph=True).run(pieces)
    for i, n in enumerate(lengths):
        if n:
            assert torch.equal(res.rows[i], st(pieces[i])), f"block {i}"
