"""Thin torch wrappers over the C ABI: allocate outputs, pass pointers, raise on errors.

Every function requires CUDA (ROCm) tensors and enqueues on the current
stream. There is no CPU implementation behind any of them.
"""

from __future__ import annotations

import ctypes
import threading
from typing import Optional, Sequence

import torch

from . import _lib

FP8 = torch.float8_e4m3fn
_DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}
_MODE = {"int8": _lib.INT8, "fp8": _lib.FP8}


def qdtype(mode: str) -> torch.dtype:
    return torch.int8 if mode == "int8" else FP8


def mode_code(mode: str) -> int:
    try:
        return _MODE[mode]
    except KeyError:
        raise ValueError(f"quant mode must be 'int8' or 'fp8', got {mode!r}") from None


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32") from None


def _gpu(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} is on {t.device}; the d3trt_amd W8A8 path runs only as HIP kernels on the GPU"
        )
    return t


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """2-D view with unit column stride (copying only if the layout needs it)."""
    _gpu(t, name)
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _qbuf(M: int, K: int, mode: str, device, kblock: bool) -> tuple[torch.Tensor, int, int]:
    """Output of a quantize call: (q, its ld, the mode code with the layout flag).

    Row-major q is [M, K] (ld K). A K-blocked q (``kblock=True``) is [K // 64, M, 64]: slice b holds
    bytes 64 b .. 64 b + 63 of every row, rows back to back (ld M, the row capacity). The pipelined
    GEMM tiles read it as whole 128-byte lines; :func:`gemm` takes either form.
    """
    if kblock:
        if K % 64:
            raise ValueError(f"a K-blocked q needs K % 64 == 0, got K={K}")
        return (torch.empty(K // 64, M, 64, dtype=qdtype(mode), device=device), M,
                mode_code(mode) | _lib.KBLOCK)
    return torch.empty(M, K, dtype=qdtype(mode), device=device), K, mode_code(mode)


def _kblocked(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(rows, K, row capacity) of a K-blocked operand [K // 64, rows, 64]."""
    _gpu(t, name)
    if t.shape[2] != 64 or t.stride(2) != 1 or t.stride(1) != 64 or t.stride(0) < 64 * t.shape[1] \
            or t.stride(0) % 64:
        raise ValueError(f"a K-blocked {name} is a [K // 64, rows, 64] tensor with rows of 64 contiguous bytes, "
                         f"got shape {tuple(t.shape)} stride {tuple(t.stride())}")
    return t.shape[1], 64 * t.shape[0], t.stride(0) // 64


def to_kblock(t: torch.Tensor) -> torch.Tensor:
    """Row-major [rows, K] (K % 64 == 0) -> K-blocked [K // 64, rows, 64] (a copy)."""
    rows, K = t.shape
    if K % 64:
        raise ValueError(f"K-blocking needs K % 64 == 0, got K={K}")
    u = t.view(torch.uint8) if t.element_size() == 1 else t  # byte copies for the float8 codes
    return u.reshape(rows, K // 64, 64).permute(1, 0, 2).contiguous().view(t.dtype)


def unblock(q: torch.Tensor) -> torch.Tensor:
    """A K-blocked q [K // 64, M, 64] as the row-major [M, K] it holds (a copy)."""
    if q.dim() != 3 or q.shape[2] != 64:
        raise ValueError(f"a K-blocked q is [K // 64, M, 64], got {tuple(q.shape)}")
    u = q.view(torch.uint8) if q.element_size() == 1 else q
    return u.permute(1, 0, 2).reshape(q.shape[1], q.shape[0] * 64).view(q.dtype)


def quantize_rows(x: torch.Tensor, mode: str, *, kblock: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """[M, K] float -> (q [M, K] int8/e4m3fn, scale [M, 1] fp32); q K-blocked with ``kblock``."""
    x = _rows(x, "x")
    M, K = x.shape
    q, ldq, mc = _qbuf(M, K, mode, x.device, kblock)
    s = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rc = lib.d3w8a8_quantize_rows(mc, dtype_code(x.dtype), x.data_ptr(), x.stride(0), M, K,
                                  q.data_ptr(), ldq, s.data_ptr(), _stream(x))
    _lib.check(rc, "quantize_rows")
    return q, s


def rmsnorm_quantize(x: torch.Tensor, weight: torch.Tensor, eps: float, mode: str, *,
                     zero_centered: bool = True, want_normed: bool = False,
                     clear_amax: Optional[torch.Tensor] = None, kblock: bool = False):
    """Fused RMSNorm + per-token quant. Returns (q, scale [M,1], normed or None); q K-blocked with
    ``kblock``."""
    x = _rows(x, "x")
    M, K = x.shape
    w = _gpu(weight, "weight").contiguous()
    if w.shape != (K,):
        raise ValueError(f"norm weight shape {tuple(w.shape)} does not match hidden size {K}")
    q, ldq, mc = _qbuf(M, K, mode, x.device, kblock)
    s = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    normed = torch.empty_like(x, memory_format=torch.contiguous_format) if want_normed else None
    if clear_amax is not None and (clear_amax.numel() < M or clear_amax.dtype != torch.float32):
        raise ValueError("clear_amax must be a float32 buffer of at least M entries")
    lib = _lib.load()
    rc = lib.d3w8a8_rmsnorm_quantize(
        mc, dtype_code(x.dtype), x.data_ptr(), x.stride(0), dtype_code(w.dtype), w.data_ptr(),
        M, K, float(eps), 1 if zero_centered else 0, q.data_ptr(), ldq, s.data_ptr(), _ptr(normed),
        K if normed is not None else 0, _ptr(clear_amax), _stream(x))
    _lib.check(rc, "rmsnorm_quantize")
    return q, s, normed


def quantize_rows_amax(h: torch.Tensor, amax: torch.Tensor, mode: str, *, kblock: bool = False):
    """Quantize rows whose amax is already known (SwiGLU output); q K-blocked with ``kblock``."""
    h = _rows(h, "h")
    M, K = h.shape
    if amax.dtype != torch.float32 or amax.numel() < M:
        raise ValueError("amax must be float32 with one entry per row")
    q, ldq, mc = _qbuf(M, K, mode, h.device, kblock)
    s = torch.empty(M, 1, dtype=torch.float32, device=h.device)
    lib = _lib.load()
    rc = lib.d3w8a8_quantize_rows_amax(mc, dtype_code(h.dtype), h.data_ptr(), h.stride(0),
                                       amax.data_ptr(), M, K, q.data_ptr(), ldq, s.data_ptr(), _stream(h))
    _lib.check(rc, "quantize_rows_amax")
    return q, s


def gate_quantize(x: torch.Tensor, gate: torch.Tensor, mode: str, *, gate_head_dim: int = 0,
                  want_y: bool = False, kblock: bool = False):
    """quantize_rows(x * sigmoid(gate)) fused: the o_proj input of a gated attention layer (core.py:297).

    ``gate`` is [M, K] (``gate_head_dim=0``), or the q_proj output [M, 2K] whose rows hold per head
    [query (head_dim) | gate (head_dim)] (core.py:231), read in place with ``gate_head_dim=head_dim``.
    Returns (q [M, K], scale [M, 1], y or None), y = the product in x's dtype; q K-blocked with ``kblock``.
    """
    x = _rows(x, "x")
    gate = _rows(gate, "gate")
    M, K = x.shape
    want_cols = 2 * K if gate_head_dim else K
    if gate.shape != (M, want_cols):
        raise ValueError(f"gate shape {tuple(gate.shape)} does not match x {tuple(x.shape)} "
                         f"(expected [{M}, {want_cols}])")
    if gate.dtype != x.dtype:
        raise ValueError("gate and x must share a dtype")
    q, ldq, mc = _qbuf(M, K, mode, x.device, kblock)
    s = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    y = torch.empty(M, K, dtype=x.dtype, device=x.device) if want_y else None
    lib = _lib.load()
    rc = lib.d3w8a8_gate_quantize(mc, dtype_code(x.dtype), x.data_ptr(), x.stride(0), gate.data_ptr(),
                                  gate.stride(0), int(gate_head_dim), M, K, q.data_ptr(), ldq, s.data_ptr(), _ptr(y),
                                  K if y is not None else 0, _stream(x))
    _lib.check(rc, "gate_quantize")
    return q, s, y


def gdn_norm_quantize(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float, head_dim: int,
                      mode: str, *, want_y: bool = False, kblock: bool = False):
    """Qwen3_5RMSNormGated over heads of ``head_dim`` (``delta.norm(core, z)``, core.py:390) fused with the
    per-token quantize of out_proj's input. x, z [M, heads * head_dim]; weight [head_dim].
    Returns (q [M, K], scale [M, 1], y or None), y = the normed, gated rows in x's dtype; q K-blocked with
    ``kblock``."""
    x = _rows(x, "x")
    z = _rows(z, "z")
    M, K = x.shape
    if z.shape != x.shape or z.dtype != x.dtype:
        raise ValueError(f"z {tuple(z.shape)} {z.dtype} must match x {tuple(x.shape)} {x.dtype}")
    w = _gpu(weight, "weight").contiguous()
    if w.shape != (head_dim,):
        raise ValueError(f"norm weight shape {tuple(w.shape)} does not match head_dim {head_dim}")
    q, ldq, mc = _qbuf(M, K, mode, x.device, kblock)
    s = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    y = torch.empty(M, K, dtype=x.dtype, device=x.device) if want_y else None
    lib = _lib.load()
    rc = lib.d3w8a8_gdn_norm_quantize(mc, dtype_code(x.dtype), x.data_ptr(), x.stride(0),
                                      z.data_ptr(), z.stride(0), dtype_code(w.dtype), w.data_ptr(), int(head_dim),
                                      float(eps), M, K, q.data_ptr(), ldq, s.data_ptr(), _ptr(y),
                                      K if y is not None else 0, _stream(x))
    _lib.check(rc, "gdn_norm_quantize")
    return q, s, y


def quantize_rows_ragged(x: torch.Tensor, lengths: Sequence[int], mode: str, *,
                         out: Optional[torch.Tensor] = None, kblock: bool = False):
    """Right-padded [B, W, K] -> packed (q [T, K], scale [T, 1], row_map [T] int32), T = sum(lengths).

    The lengths stay on the host: the library folds them into packed-row
    offsets passed to the kernel by value (no host-to-device copy, so the call
    can be captured in a graph). When ``out`` ([B*W, N] view of the final
    output) is given, its padded rows are zeroed. With ``kblock`` q is K-blocked, [K // 64, T, 64].
    """
    _gpu(x, "x")
    if x.dim() != 3:
        raise ValueError(f"ragged input must be [blocks, width, K], got {tuple(x.shape)}")
    B, W, K = x.shape
    lengths = [int(n) for n in lengths]
    if len(lengths) != B or any(n < 0 or n > W for n in lengths):
        raise ValueError(f"lengths {lengths} do not fit a [{B}, {W}] batch")
    if B > _lib.MAX_SEGMENTS:
        raise ValueError(f"at most {_lib.MAX_SEGMENTS} blocks per ragged batch, got {B}")
    x2 = x.reshape(B * W, K)
    x2 = _rows(x2, "x")
    if out is not None:
        # the kernel zeroes every padded row b * W + t of `out` (t >= lengths[b]) through its row pitch
        _gpu(out, "out")
        if out.dim() != 2 or out.stride(1) != 1 or out.shape[0] < B * W or out.stride(0) < out.shape[1]:
            raise ValueError(f"out must be a row-major [>= {B * W}, N] tensor, got shape {tuple(out.shape)} "
                             f"stride {tuple(out.stride())}")
        if out.dtype not in _DT:
            raise ValueError(f"unsupported out dtype {out.dtype}")
    T = sum(lengths)
    dev = x.device
    host_lengths = (ctypes.c_int32 * max(B, 1))(*lengths)
    # at least one row so the pointers are valid when every block is empty (the kernel
    # still runs to zero the padded output rows)
    q, ldq, mc = _qbuf(max(T, 1), K, mode, dev, kblock)
    s = torch.empty(max(T, 1), 1, dtype=torch.float32, device=dev)
    row_map = torch.empty(max(T, 1), dtype=torch.int32, device=dev)
    N = out.shape[1] if out is not None else 0
    lib = _lib.load()
    rc = lib.d3w8a8_quantize_rows_ragged(
        mc, dtype_code(x2.dtype), x2.data_ptr(), x2.stride(0), ctypes.addressof(host_lengths), B, W,
        K, q.data_ptr(), ldq, s.data_ptr(), row_map.data_ptr(), _ptr(out),
        dtype_code(out.dtype) if out is not None else 0, out.stride(0) if out is not None else 0, N,
        _stream(x2))
    _lib.check(rc, "quantize_rows_ragged")
    row_map = row_map[:T]
    row_map.d3_rows = B * W  # output rows the map addresses; gemm() checks its `out` against it
    return (q[:, :T] if kblock else q[:T]), s[:T], row_map


def gemm(mode: str, a: torch.Tensor, a_scale: Optional[torch.Tensor], w: torch.Tensor,
         w_scale: Optional[torch.Tensor], *, epilogue: int = _lib.EPI_DEQUANT,
         out_dtype: torch.dtype = torch.bfloat16, out: Optional[torch.Tensor] = None,
         residual: Optional[torch.Tensor] = None, row_amax: Optional[torch.Tensor] = None,
         row_map: Optional[torch.Tensor] = None, tile: int = _lib.TILE_AUTO,
         ksplit: int = _lib.KSPLIT_AUTO, noalloc: bool = False) -> torch.Tensor:
    """W8A8 GEMM ``a @ w.T`` with a fused epilogue (see include/d3w8a8.h).

    ``a`` is row-major [M, K] or K-blocked [K // 64, M, 64] (from a quantize call with ``kblock``), and
    ``w`` row-major [N, K] or K-blocked [K // 64, N, 64]; the results are the same.

    Skinny problems may split K over several workgroups per output tile
    (``ksplit``, automatic by default); the split-K workspace is this module's
    per-(device, stream) buffer from :func:`workspace`. With ``noalloc=True``
    the partial sums go to the library's static per-GPU scratch instead
    (``d3w8a8_gemm_noalloc``: nothing is allocated for them; such calls on one
    GPU must run in order).
    """
    a_kblk, w_kblk = a.dim() == 3, w.dim() == 3
    if a_kblk:
        M, K, lda = _kblocked(a, "a")
    else:
        a = _rows(a, "a")
        (M, K), lda = a.shape, a.stride(0)
    if w_kblk:
        N, Kw, ldw = _kblocked(w, "w")
    else:
        w = _rows(w, "w")
        (N, Kw), ldw = w.shape, w.stride(0)
    mc = mode_code(mode) | (_lib.KBLOCK if a_kblk else 0) | (_lib.W_KBLOCK if w_kblk else 0)
    if Kw != K:
        raise ValueError(f"inner dimensions differ: a {tuple(a.shape)} vs w {tuple(w.shape)}")
    if a.dtype != qdtype(mode) or w.dtype != qdtype(mode):
        raise ValueError(f"{mode} GEMM wants {qdtype(mode)} operands, got {a.dtype} and {w.dtype}")
    if epilogue == _lib.EPI_RAW:
        odt = torch.int32 if mode == "int8" else torch.float32
        ncols = N
    else:
        odt = out_dtype
        ncols = N // 2 if epilogue == _lib.EPI_SWIGLU else N
    if out is None:
        rows = M
        if row_map is not None:
            raise ValueError("a row_map GEMM needs an explicit output tensor")
        out = torch.empty(rows, ncols, dtype=odt, device=a.device)
    else:
        _gpu(out, "out")
        if out.dtype != odt or out.dim() != 2 or out.stride(1) != 1 or out.shape[1] < ncols:
            raise ValueError("output tensor has the wrong dtype or layout")
        if row_map is None and out.shape[0] < M:
            raise ValueError("output tensor has too few rows")
    if residual is not None:
        _gpu(residual, "residual")
        if residual.dtype != odt or residual.dim() != 2 or residual.stride(1) != 1:
            raise ValueError("residual must be a row-major tensor of the output dtype")
        if residual.shape[0] < out.shape[0] or residual.shape[1] < N:
            raise ValueError("residual is smaller than the output")
    if row_amax is not None and (row_amax.dtype != torch.float32 or row_amax.numel() < M
                                 or not row_amax.is_contiguous()):
        raise ValueError("row_amax must be a contiguous float32 buffer with one entry per GEMM row")
    if row_map is not None:
        if row_map.dtype != torch.int32 or row_map.numel() != M or not row_map.is_contiguous():
            raise ValueError("row_map must be contiguous int32 with one entry per GEMM row")
        # rows a map from quantize_rows_ragged can address (its batch's B * W); a map built elsewhere
        # must hold indices below out.shape[0] (checking its values here would synchronize the device)
        need = getattr(row_map, "d3_rows", M)
        if out.shape[0] < need:
            raise ValueError(f"output tensor has {out.shape[0]} rows; the row_map addresses {need}")
    for t, name in ((a_scale, "a_scale"), (w_scale, "w_scale")):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous float32")
    if epilogue != _lib.EPI_RAW:
        if a_scale is None or w_scale is None or a_scale.numel() != M or w_scale.numel() != N:
            raise ValueError("dequantizing epilogues need a_scale [M] and w_scale [N]")
    lib = _lib.load()
    st = _stream(a)
    if noalloc:
        rc = lib.d3w8a8_gemm_noalloc(
            mc, a.data_ptr(), lda, _ptr(a_scale), w.data_ptr(), ldw, _ptr(w_scale),
            M, N, K, epilogue, dtype_code(odt) if epilogue != _lib.EPI_RAW else 0, out.data_ptr(), out.stride(0),
            _ptr(residual), residual.stride(0) if residual is not None else 0, _ptr(row_amax), _ptr(row_map),
            tile, ksplit, st)
        _lib.check(rc, "gemm_noalloc")
        return out
    ws = None
    if ksplit != 1:
        # only a plan that splits K touches the workspace (the state-pass shapes never do)
        need = lib.d3w8a8_gemm_workspace(M, N, K, K if a_kblk else lda, K if w_kblk else ldw, tile, ksplit,
                                         WORKSPACE_BYTES)
        if need < 0:
            _lib.check(_lib.EINVAL, "gemm")
        if need > 0:
            ws = workspace(a.device, st)
    rc = lib.d3w8a8_gemm_ws(
        mc, a.data_ptr(), lda, _ptr(a_scale), w.data_ptr(), ldw, _ptr(w_scale),
        M, N, K, epilogue, dtype_code(odt) if epilogue != _lib.EPI_RAW else 0, out.data_ptr(), out.stride(0),
        _ptr(residual), residual.stride(0) if residual is not None else 0, _ptr(row_amax), _ptr(row_map),
        tile, ksplit, _ptr(ws), ws.numel() if ws is not None else 0, st)
    _lib.check(rc, "gemm")
    return out


WORKSPACE_BYTES = 64 << 20
_workspaces: dict = {}
_workspaces_lock = threading.Lock()


def workspace(device: torch.device, stream: int) -> torch.Tensor:
    """The split-K workspace of one (device, stream): WORKSPACE_BYTES of device memory.

    GEMMs on one stream run in order, so they can share it; streams never
    share one. The first split-K GEMM on a stream allocates it through torch's
    caching allocator. Inside a graph capture (torch.cuda.graph captures on a
    stream of its own) that allocation comes from the graph's private memory
    pool, which torch allows; the buffer stays cached for the capture stream,
    so later captures on it reuse the same memory. Graphs captured on one
    stream therefore share a workspace: replay them in order (one stream).
    """
    device = torch.device(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None:
        with _workspaces_lock:
            ws = _workspaces.get(key)
            if ws is None:
                ws = torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device=device)
                _workspaces[key] = ws
    return ws


def interleave_gate_up(full: torch.Tensor) -> torch.Tensor:
    """Row permutation [gate; up] (the reference's cat layout, trtllm_stack.py:366-368)
    -> blocks of 32: [g0..g31, u0..u31, g32..g63, u32..u63, ...].

    Works on any tensor whose first dimension is 2*I with I % 32 == 0 (weights [2I, K]
    or per-channel scales [2I]).
    """
    two_i = full.shape[0]
    if two_i % 64:
        raise ValueError(f"gate_up rows {two_i} must be a multiple of 64 for the SwiGLU layout")
    i = two_i // 2
    rest = full.shape[1:]
    gate = full[:i].reshape(i // 32, 32, *rest)
    up = full[i:].reshape(i // 32, 32, *rest)
    return torch.stack([gate, up], dim=1).reshape(two_i, *rest).contiguous()


def deinterleave_gate_up(inter: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`interleave_gate_up`."""
    two_i = inter.shape[0]
    i = two_i // 2
    rest = inter.shape[1:]
    blocks = inter.reshape(i // 32, 2, 32, *rest)
    return torch.cat([blocks[:, 0].reshape(i, *rest), blocks[:, 1].reshape(i, *rest)], dim=0).contiguous()
