"""ctypes binding of libd3w8a8.so (the C ABI declared in include/d3w8a8.h).

The library is loaded from this package directory; there is no fallback. If
it is missing or fails to load, every entry point raises, so a GPU run can
never silently take another path.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libd3w8a8.so")

OK, EINVAL, EHIP = 0, 1, 2
INT8, FP8 = 0, 1
# D3W8A8_KBLOCK, OR-ed into a mode: K-blocked quantized activations (q of the quantize calls, a of
# the GEMMs): byte (m, k) at ((k // 64) * ld + m) * 64 + k % 64, ld the row capacity
KBLOCK = 0x100
W_KBLOCK = 0x200  # D3W8A8_W_KBLOCK: the same layout for the weights of a GEMM
BF16, F16, F32 = 0, 1, 2
EPI_DEQUANT, EPI_RAW, EPI_SWIGLU, EPI_RESIDUAL = 0, 1, 2, 3
TILE_AUTO, TILE_256, TILE_128, TILE_64x128 = -1, 0, 1, 2
MAX_SEGMENTS = 256  # D3W8A8_MAX_SEGMENTS: blocks of one ragged batch
KSPLIT_AUTO = -1  # D3W8A8_KSPLIT_AUTO
NOALLOC_SCRATCH_BYTES = 16 << 20  # D3W8A8_NOALLOC_SCRATCH_BYTES: split-K scratch of d3w8a8_gemm_noalloc
TILE_DMA_256_W8, TILE_DMA_256_W4, TILE_DMA_128_W4, TILE_DMA_256x128_W4 = 3, 4, 5, 6
TILE_DMA_128_W4_K128 = 7  # 128-byte K steps: K % 128 == 0
TILE_DMA_256x192_W4 = 8  # 3 column blocks per wave: not for the SwiGLU epilogue
TILE_WS = 9  # weight streaming for skinny M: K % 128 == 0, never splits K
TILE_DMA_192x192_W4 = 10  # 3 column blocks per wave: not for the SwiGLU epilogue
TILE_DMA_192x128_W4 = 11
TILES = (TILE_256, TILE_128, TILE_64x128, TILE_DMA_256_W8, TILE_DMA_256_W4, TILE_DMA_128_W4, TILE_DMA_256x128_W4,
         TILE_DMA_128_W4_K128, TILE_DMA_256x192_W4, TILE_WS, TILE_DMA_192x192_W4, TILE_DMA_192x128_W4)
DMA_TILES = (TILE_DMA_256_W8, TILE_DMA_256_W4, TILE_DMA_128_W4, TILE_DMA_256x128_W4, TILE_DMA_128_W4_K128,
             TILE_DMA_256x192_W4, TILE_WS, TILE_DMA_192x192_W4, TILE_DMA_192x128_W4)
NO_SWIGLU_TILES = (TILE_DMA_256x192_W4, TILE_DMA_192x192_W4)  # three 32-column blocks per wave


def tile_k_multiple(tile: int) -> int:
    """K must be a multiple of this for `tile` (16 for the register-staged tiles)."""
    return 128 if tile in (TILE_DMA_128_W4_K128, TILE_WS) else 64 if tile in DMA_TILES else 16

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (every entry point returns int status)
SIGNATURES = {
    "d3w8a8_quantize_rows": [_i32, _i32, _p, _i64, _i64, _i64, _p, _i64, _p, _p],
    "d3w8a8_rmsnorm_quantize": [_i32, _i32, _p, _i64, _i32, _p, _i64, _i64, _f32, _i32, _p, _i64, _p, _p,
                                _i64, _p, _p],
    "d3w8a8_quantize_rows_amax": [_i32, _i32, _p, _i64, _p, _i64, _i64, _p, _i64, _p, _p],
    "d3w8a8_gdn_norm_quantize": [_i32, _i32, _p, _i64, _p, _i64, _i32, _p, _i64, _f32, _i64, _i64, _p, _i64, _p,
                                 _p, _i64, _p],
    "d3w8a8_gate_quantize": [_i32, _i32, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _p],
    "d3w8a8_quantize_rows_ragged": [_i32, _i32, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i32,
                                    _i64, _i64, _p],
    "d3w8a8_gemm": [_i32, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p, _i64, _p,
                    _p, _i32, _p],
    "d3w8a8_gemm_ws": [_i32, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p, _i64, _p,
                       _p, _i32, _i32, _p, _i64, _p],
    "d3w8a8_gemm_noalloc": [_i32, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p, _i64,
                            _p, _p, _i32, _i32, _p],
}
# name -> argtypes of the entry points that return int64
INT64_FUNCS = {
    "d3w8a8_gemm_workspace": [_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64],
}
STRING_FUNCS = ("d3w8a8_version", "d3w8a8_last_error")

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class LibraryMissing(RuntimeError):
    """The HIP library is not built or cannot be loaded."""


def load() -> ctypes.CDLL:
    """Load and type the library once; raise LibraryMissing if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run `python d3-turbo-trt_amd/build.py` "
                    "(the W8A8 path has no non-HIP implementation)"
                )
            try:
                lib = ctypes.CDLL(LIB_PATH)
            except OSError as exc:  # pragma: no cover - depends on the ROCm install
                raise LibraryMissing(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            for name, argtypes in INT64_FUNCS.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int64
            for name in STRING_FUNCS:
                fn = getattr(lib, name)
                fn.argtypes = []
                fn.restype = ctypes.c_char_p
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception types (ValueError / RuntimeError)."""
    if rc == OK:
        return
    msg = load().d3w8a8_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def version() -> str:
    return load().d3w8a8_version().decode()
