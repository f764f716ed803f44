"""Host zstd through the system libzstd (ctypes), for the optional hi-plane
compression of spilled pages.

The reference compresses spilled KV with zstd level 1 (runtime/kv_paged.py:
79-91, compression.zstd) and vpack compresses the hi byte plane the same way
(formats/packed.py:49, 277-282).  Only the stable public API is bound:
ZSTD_compress, ZSTD_decompress, ZSTD_compressBound, ZSTD_isError,
ZSTD_getErrorName.  Compressed bytes depend on the libzstd version; the round
trip is what is guaranteed (and tested).
"""

from __future__ import annotations

import ctypes
import ctypes.util
import threading

import numpy as np

_lock = threading.Lock()
_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            name = ctypes.util.find_library("zstd") or "libzstd.so.1"
            lib = ctypes.CDLL(name)
            lib.ZSTD_compressBound.restype = ctypes.c_size_t
            lib.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
            lib.ZSTD_compress.restype = ctypes.c_size_t
            lib.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_int]
            lib.ZSTD_decompress.restype = ctypes.c_size_t
            lib.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                            ctypes.c_size_t]
            lib.ZSTD_isError.restype = ctypes.c_uint
            lib.ZSTD_isError.argtypes = [ctypes.c_size_t]
            lib.ZSTD_getErrorName.restype = ctypes.c_char_p
            lib.ZSTD_getErrorName.argtypes = [ctypes.c_size_t]
            _lib = lib
    return _lib


def available() -> bool:
    try:
        _load()
        return True
    except OSError:
        return False


def _check(rc: int, what: str) -> int:
    lib = _load()
    if lib.ZSTD_isError(rc):
        raise RuntimeError(f"zstd {what}: {lib.ZSTD_getErrorName(rc).decode()}")
    return rc


def compress(src: np.ndarray, level: int = 1) -> np.ndarray:
    """Compress a contiguous uint8 array; returns a new uint8 array (one frame)."""
    lib = _load()
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty(lib.ZSTD_compressBound(src.nbytes), dtype=np.uint8)
    n = _check(lib.ZSTD_compress(dst.ctypes.data, dst.nbytes, src.ctypes.data, src.nbytes, level),
               "compress")
    return dst[:n].copy()


def decompress_into(src: np.ndarray, dst: np.ndarray) -> int:
    """Decompress one frame into the preallocated uint8 array ``dst``; returns bytes written."""
    lib = _load()
    src = np.ascontiguousarray(src, dtype=np.uint8)
    n = _check(lib.ZSTD_decompress(dst.ctypes.data, dst.nbytes, src.ctypes.data, src.nbytes),
               "decompress")
    if n != dst.nbytes:
        raise RuntimeError(f"zstd decompress: frame holds {n} bytes, expected {dst.nbytes}")
    return n


def compress_into(src: np.ndarray, dst: np.ndarray, level: int = 1) -> int:
    """Compress the contiguous uint8 array ``src`` into the preallocated
    ``dst`` (at least compress_bound(src.nbytes) bytes); returns the frame
    length.  No Python-side copies, so worker threads spend their time inside
    libzstd, with the GIL released."""
    lib = _load()
    return _check(lib.ZSTD_compress(dst.__array_interface__["data"][0], dst.nbytes,
                                    src.__array_interface__["data"][0], src.nbytes, level),
                  "compress")


def compress_bound(nbytes: int) -> int:
    return int(_load().ZSTD_compressBound(nbytes))
