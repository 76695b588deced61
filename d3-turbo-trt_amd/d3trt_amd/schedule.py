"""Question passes over variable-length blocks, packed row-wise through the projection stack.

The reference's question loop (d3trt/backends/trtllm.py:149-179) sorts the question pieces by
length, takes them ``batch_size`` at a time, right-pads each batch to ``[B, W]`` and runs the
stack's question pass on it (``D3Core.questions``, d3trt/model/core.py:158-181, masks the padded
rows and then computes them anyway); results go back to their pieces by index, so the output order
is the input order.

Here a batch is formed the same way (stable sort by length, ``batch_size`` blocks per batch, or all
blocks in one batch), but its rows are packed: the blocks' rows are concatenated into one
``[T, hidden]`` matrix, T = the sum of the batch's lengths, and the stack runs at M = T. Every
projection, norm and quantization is row-wise, so packing changes no result and no padded row is
computed. Packed row counts are rounded up to a multiple of ``bucket`` rows (zero rows, whose results
are dropped) so that a serving loop replays a bounded set of captured HIP graphs, one per bucket.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from .stack import LinearStack


@dataclass
class Batch:
    """One packed batch: ``blocks`` (indices into the input), their packed row offsets, and the row
    count the stack runs at (the rows rounded up to the bucket)."""
    blocks: list[int]
    offsets: list[int]  # len(blocks) + 1 entries; block blocks[k] owns packed rows [offsets[k], offsets[k+1])
    rows: int           # packed rows with data (offsets[-1])
    run_rows: int       # rows the stack runs at (>= rows)


def plan_batches(lengths: Sequence[int], batch_size: Optional[int], bucket: int = 1) -> list[Batch]:
    """Batches of a question pass (backends/trtllm.py:149-155): blocks sorted by length (stable),
    ``batch_size`` per batch (None: one batch of every block); each batch's rows packed in that order.
    Blocks of length 0 take part in a batch and own no rows."""
    lengths = [int(n) for n in lengths]
    if any(n < 0 for n in lengths):
        raise ValueError(f"block lengths must be >= 0, got {lengths}")
    if batch_size is not None and batch_size < 1:
        raise ValueError(f"batch_size must be >= 1 or None, got {batch_size}")
    if bucket < 1:
        raise ValueError(f"bucket must be >= 1, got {bucket}")
    order = sorted(range(len(lengths)), key=lambda i: lengths[i])
    step = len(order) if batch_size is None else batch_size
    batches = []
    for start in range(0, len(order), max(step, 1)):
        blocks = order[start:start + step]
        offs = [0]
        for i in blocks:
            offs.append(offs[-1] + lengths[i])
        rows = offs[-1]
        batches.append(Batch(blocks, offs, rows, -(-rows // bucket) * bucket))
    return batches


@dataclass
class QuestionResult:
    """Per-block results in input order: every row of each block, and each block's last row (the
    hidden state the reference reads out per question, core.py:178-180; a zero row for an empty
    block)."""
    rows: list[torch.Tensor]
    last: torch.Tensor
    batches: list[Batch] = field(default_factory=list)


class QuestionScheduler:
    """Runs variable-length question blocks through a :class:`LinearStack` in packed batches.

    ``batch_size`` is the reference's ``d3.batch_size`` (blocks per batch; None for one batch of all
    blocks). With ``graph=True`` each packed row count (rounded up to ``bucket``) replays a HIP graph
    of the whole stack captured on first use (:meth:`LinearStack.graphed`).
    """

    def __init__(self, stack: LinearStack, *, batch_size: Optional[int] = 8, graph: bool = True, bucket: int = 16):
        self.stack = stack
        self.batch_size = batch_size
        self.graph = graph
        self.bucket = bucket if graph else 1

    @torch.no_grad()
    def run(self, pieces: Sequence[torch.Tensor]) -> QuestionResult:
        """``pieces[i]`` is block i's hidden states, [n_i, hidden] on the stack's GPU."""
        H = self.stack.hidden
        if not pieces:
            raise ValueError("no question blocks")
        dev, dtype = pieces[0].device, pieces[0].dtype
        for p in pieces:
            if p.dim() != 2 or p.shape[1] != H or p.device != dev or p.dtype != dtype:
                raise ValueError(f"every block must be [n, {H}] {dtype} on {dev}; got {tuple(p.shape)} "
                                 f"{p.dtype} on {p.device}")
        batches = plan_batches([p.shape[0] for p in pieces], self.batch_size, self.bucket)
        rows: list[Optional[torch.Tensor]] = [None] * len(pieces)
        last = torch.zeros(len(pieces), H, dtype=dtype, device=dev)
        for b in batches:
            if b.rows == 0:
                for i in b.blocks:
                    rows[i] = pieces[i][:0]
                continue
            parts = [pieces[i] for i in b.blocks if pieces[i].shape[0]]
            if b.run_rows > b.rows:
                parts.append(torch.zeros(b.run_rows - b.rows, H, dtype=dtype, device=dev))
            packed = torch.cat(parts) if len(parts) > 1 else parts[0].contiguous()
            if self.graph:
                out = self.stack.graphed(b.run_rows)(packed).clone()  # the graph's output is reused
            else:
                out = self.stack.forward(packed)
            for k, i in enumerate(b.blocks):
                r0, r1 = b.offsets[k], b.offsets[k + 1]
                rows[i] = out[r0:r1]
            ends = [(i, b.offsets[k + 1] - 1) for k, i in enumerate(b.blocks) if b.offsets[k + 1] > b.offsets[k]]
            if ends:
                dst = torch.tensor([i for i, _ in ends], device=dev)
                src = torch.tensor([r for _, r in ends], device=dev)
                last.index_copy_(0, dst, out.index_select(0, src))
        return QuestionResult(rows=rows, last=last, batches=batches)  # type: ignore[arg-type]
