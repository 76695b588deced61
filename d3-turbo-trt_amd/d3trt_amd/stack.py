"""The W8A8 projection stack of d3's backbone, with the token mixer replaced by identity.

Per layer this is D3Core._layer (d3trt/model/core.py:184-225) with every
projection quantized (d3trt/model/quant.py) and the attention/GDN mixer left
out, so that only the linear path runs:

    h   = x + o_proj(mix(qkv_proj(input_norm(x))))       core.py:207-214
    out = h + down(silu(gate) * up),  gate, up = gate_up(post_norm(h)).chunk(2)
                                                          core.py:215, trtllm_stack.py:131-134

``mix`` is the identity on the query block: the first ``hidden`` columns of
the fused [q | k | v] projection are the o_proj input (q_proj's output width
equals o_proj's input width). The reference runs q/k/v as three projections
(trtllm_stack.py:79-93); fusing them is a concatenation of weight rows, so
each output column is the same dot product.

Every layer is eight launches of libd3w8a8 kernels, each one HBM pass:
norm+quant, QKV GEMM, quant of the q block, o_proj GEMM with the residual
add, norm+quant, gate_up GEMM with SwiGLU and the row amax, requant, down
GEMM with the residual add. Question batches (core.py:158-181 runs them
right-padded) are packed to their valid rows once, run through all layers at
M = sum(lengths), and scattered back: rows are independent through every
step, so packing changes no result and computes no padded row.
"""

from __future__ import annotations

from typing import Any, Sequence

import torch
import torch.nn as nn

from . import _lib
from . import kernels as K
from .mlp import QuantMLP
from .quant import QuantLinear


class StackLayer(nn.Module):
    """One layer's norms and quantized projections."""

    def __init__(self, hidden: int, qkv_out: int, intermediate: int, *, mode: str, dtype: torch.dtype,
                 device: Any, eps: float = 1e-6):
        super().__init__()
        if qkv_out < hidden:
            raise ValueError("the fused qkv projection must be at least as wide as the hidden size")
        self.hidden = hidden
        self.eps = eps
        self.input_layernorm = nn.Parameter(torch.zeros(hidden, dtype=dtype, device=device), requires_grad=False)
        self.post_attention_layernorm = nn.Parameter(torch.zeros(hidden, dtype=dtype, device=device),
                                                     requires_grad=False)
        self.qkv_proj = QuantLinear(hidden, qkv_out, mode=mode, dtype=dtype, device=device)
        self.o_proj = QuantLinear(hidden, hidden, mode=mode, dtype=dtype, device=device)
        self.mlp = QuantMLP(hidden, intermediate, mode=mode, dtype=dtype, device=device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[M, hidden] bf16 (rows contiguous) -> [M, hidden]."""
        mode = self.qkv_proj.mode
        q1, s1, _ = K.rmsnorm_quantize(x, self.input_layernorm, self.eps, mode, kblock=self.qkv_proj.kblock)
        qkv = K.gemm(mode, q1, s1.reshape(-1), self.qkv_proj.weight, self.qkv_proj.weight_scale,
                     epilogue=_lib.EPI_DEQUANT, out_dtype=x.dtype)
        q2, s2 = K.quantize_rows(qkv[:, : self.hidden], mode, kblock=self.o_proj.kblock)
        h = K.gemm(mode, q2, s2.reshape(-1), self.o_proj.weight, self.o_proj.weight_scale,
                   epilogue=_lib.EPI_RESIDUAL, out_dtype=x.dtype, residual=x)
        return self.mlp.block(h, self.post_attention_layernorm, self.eps)


class LinearStack(nn.Module):
    """``layers`` x (fused QKV, o_proj, gate_up + SwiGLU, down) with zero-centred RMSNorms."""

    def __init__(self, layers: int, hidden: int, qkv_out: int, intermediate: int, *, mode: str,
                 dtype: torch.dtype = torch.bfloat16, device: Any = "cuda", eps: float = 1e-6):
        super().__init__()
        self.layers = nn.ModuleList(
            StackLayer(hidden, qkv_out, intermediate, mode=mode, dtype=dtype, device=device, eps=eps)
            for _ in range(layers)
        )
        self.hidden = hidden

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """State pass: [..., hidden] -> [..., hidden] through every layer (M = all rows)."""
        shape = x.shape
        h = x.reshape(-1, self.hidden).contiguous()
        for layer in self.layers:
            h = layer(h)
        return h.reshape(shape)

    def forward_ragged(self, x: torch.Tensor, lengths: Sequence[int], *, graph: bool = False) -> torch.Tensor:
        """Question pass over a right-padded batch [B, W, hidden] with ``lengths[b]`` valid rows.

        The valid rows are packed, run at M = sum(lengths), and scattered back;
        padded rows of the result are zero (core.py:167-171 zeroes padded
        inputs; the reference then computes them anyway). With ``graph=True``
        the packed pass replays a HIP graph captured once per row count
        (:class:`GraphedStack`), so the ~8 launches per layer cost one launch.
        """
        B, W, H = x.shape
        lengths = [int(n) for n in lengths]
        if len(lengths) != B or any(n < 0 or n > W for n in lengths):
            raise ValueError(f"lengths {lengths} do not fit a [{B}, {W}] batch")
        rows, pad = self._packed_rows(tuple(lengths), W, x.device)
        flat = x.reshape(B * W, H)
        out = torch.empty_like(flat, memory_format=torch.contiguous_format)
        if rows.numel():
            packed = flat.index_select(0, rows)
            res = self.graphed(rows.numel())(packed) if graph else self.forward(packed)
            out.index_copy_(0, rows, res)
        if pad.numel():
            out.index_fill_(0, pad, 0)  # only the padded rows: no pass over the whole batch
        return out.reshape(B, W, H)

    def _packed_rows(self, lengths: tuple, width: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        """Device indices of the valid rows and of the padded rows of a [B, width] batch (cached per
        shape)."""
        cache = self.__dict__.setdefault("_rows_cache", {})
        key = (lengths, width, str(device))
        if key not in cache:
            idx = [b * width + t for b, n in enumerate(lengths) for t in range(n)]
            pad = [b * width + t for b, n in enumerate(lengths) for t in range(n, width)]
            cache[key] = (torch.tensor(idx, dtype=torch.long).to(device), torch.tensor(pad, dtype=torch.long).to(device))
        return cache[key]

    def graphed(self, rows: int) -> "GraphedStack":
        """The HIP-graph replay of :meth:`forward` for ``rows`` packed rows (captured on first use)."""
        graphs = self.__dict__.setdefault("_graphs", {})
        if rows not in graphs:
            graphs[rows] = GraphedStack(self, rows)
        return graphs[rows]

    @torch.no_grad()
    def init_random(self, generator: torch.Generator, *, weight_std: float = 0.02, norm_std: float = 0.1) -> None:
        """Random-init every layer: N(0, weight_std) projections (quantized on the GPU), N(0, norm_std)
        zero-centred norm weights (gain 1 + w)."""
        for layer in self.layers:
            dev = layer.qkv_proj.weight.device
            for lin in (layer.qkv_proj, layer.o_proj):
                w = torch.randn(lin.out_features, lin.in_features, generator=generator, device=dev,
                                dtype=torch.float32).mul_(weight_std).to(torch.bfloat16)
                lin.load_full(w)
                del w
            gu, dn = layer.mlp.gate_up_proj, layer.mlp.down_proj
            w = torch.randn(gu.out_features, gu.in_features, generator=generator, device=dev,
                            dtype=torch.float32).mul_(weight_std).to(torch.bfloat16)
            w2 = torch.randn(dn.out_features, dn.in_features, generator=generator, device=dev,
                             dtype=torch.float32).mul_(weight_std).to(torch.bfloat16)
            layer.mlp.load_full(w, w2)
            del w, w2
            for norm in (layer.input_layernorm, layer.post_attention_layernorm):
                norm.copy_(torch.randn(norm.shape[0], generator=generator, device=dev,
                                       dtype=torch.float32).mul_(norm_std))


class GraphedStack:
    """:meth:`LinearStack.forward` on a fixed number of rows, captured as one HIP graph.

    A question batch runs every layer at a small M (e.g. 8 blocks x 16 tokens),
    where each of the ~8 launches per layer is cheaper on the GPU than on the
    host. The capture records the same kernels the eager pass launches (no
    memset or host copy happens inside it); a call copies the input into the
    static buffer, replays, and returns the static output, which the next call
    overwrites.
    """

    def __init__(self, stack: LinearStack, rows: int):
        dev = next(stack.buffers()).device
        dtype = stack.layers[0].input_layernorm.dtype  # the stack's activation dtype (its norm weights')
        self.static_in = torch.zeros(rows, stack.hidden, dtype=dtype, device=dev)
        # one capture stream per stack: its graphs share that stream's split-K workspace (replays run in
        # order on the caller's stream) instead of each capture bringing its own
        side = stack.__dict__.setdefault("_capture_stream", torch.cuda.Stream(device=dev))
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):  # warm the allocator (and the stream's split-K workspace) outside the capture
                stack.forward(self.static_in)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            self.static_out = stack.forward(self.static_in)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        self.static_in.copy_(x)
        self.graph.replay()
        return self.static_out
