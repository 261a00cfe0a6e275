"""zstd frames through the system libzstd (ctypes), for the .tsk container.

The reference container (container.py:46) uses the `zstandard` Python
package, which this image does not ship; the frame format is zstd's own, so a
frame written here decompresses with `zstandard` and vice versa. Frames carry
their content size (as `zstandard.ZstdCompressor().compress` writes them),
which decompression reads to size its output.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import os
from typing import Optional

_lib: Optional[ctypes.CDLL] = None
ZSTD_c_compressionLevel = 100  # zstd.h: ZSTD_cParameter values
ZSTD_c_nbWorkers = 400
ZSTD_e_end = 2
_CONTENTSIZE_ERROR = (1 << 64) - 2
_CONTENTSIZE_UNKNOWN = (1 << 64) - 1


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = ctypes.util.find_library("zstd") or "libzstd.so.1"
        try:
            z = ctypes.CDLL(path)
        except OSError as e:  # pragma: no cover - the image ships libzstd.so.1
            raise RuntimeError("the .tsk container needs libzstd (libzstd.so.1)") from e
        sz, vp, cvp = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
        z.ZSTD_compressBound.restype, z.ZSTD_compressBound.argtypes = sz, [sz]
        z.ZSTD_isError.restype, z.ZSTD_isError.argtypes = ctypes.c_uint, [sz]
        z.ZSTD_getErrorName.restype, z.ZSTD_getErrorName.argtypes = cvp, [sz]
        z.ZSTD_createCCtx.restype, z.ZSTD_createCCtx.argtypes = vp, []
        z.ZSTD_freeCCtx.restype, z.ZSTD_freeCCtx.argtypes = sz, [vp]
        z.ZSTD_CCtx_setParameter.restype, z.ZSTD_CCtx_setParameter.argtypes = sz, [vp, ctypes.c_int, ctypes.c_int]
        z.ZSTD_compress2.restype, z.ZSTD_compress2.argtypes = sz, [vp, vp, sz, vp, sz]
        z.ZSTD_decompress.restype, z.ZSTD_decompress.argtypes = sz, [vp, sz, vp, sz]
        z.ZSTD_getFrameContentSize.restype, z.ZSTD_getFrameContentSize.argtypes = ctypes.c_ulonglong, [vp, sz]
        _lib = z
    return _lib


def _check(rc: int, what: str) -> int:
    z = lib()
    if z.ZSTD_isError(rc):
        raise RuntimeError(f"zstd {what}: {z.ZSTD_getErrorName(rc).decode()}")
    return rc


def compress(data: bytes, level: int = 12, threads: Optional[int] = None) -> bytes:
    """One zstd frame (content size in the header) at `level`, on `threads`
    worker threads where libzstd was built with them."""
    z = lib()
    src = bytes(data)
    cap = z.ZSTD_compressBound(len(src))
    dst = ctypes.create_string_buffer(max(1, cap))
    cctx = z.ZSTD_createCCtx()
    if not cctx:
        raise MemoryError("ZSTD_createCCtx")
    try:
        _check(z.ZSTD_CCtx_setParameter(cctx, ZSTD_c_compressionLevel, int(level)), "level")
        n_threads = threads if threads is not None else min(8, os.cpu_count() or 1)
        if n_threads > 1 and len(src) > (1 << 20):
            z.ZSTD_CCtx_setParameter(cctx, ZSTD_c_nbWorkers, int(n_threads))  # an error = built without threads
        n = _check(z.ZSTD_compress2(cctx, dst, cap, src, len(src)), "compress")
    finally:
        z.ZSTD_freeCCtx(cctx)
    return dst.raw[:n]


def decompress(frame: bytes) -> bytes:
    """Inverse of compress(): one frame with its content size recorded."""
    z = lib()
    src = bytes(frame)
    size = z.ZSTD_getFrameContentSize(src, len(src))
    if size in (_CONTENTSIZE_ERROR, _CONTENTSIZE_UNKNOWN):
        raise RuntimeError("zstd frame without a content size")
    dst = ctypes.create_string_buffer(max(1, size))
    n = _check(z.ZSTD_decompress(dst, size, src, len(src)), "decompress")
    if n != size:
        raise RuntimeError(f"zstd frame decompressed to {n} bytes, header says {size}")
    return dst.raw[:n]
