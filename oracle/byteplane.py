"""Byte-plane codec, restated on the CPU (test infrastructure only).

vpack splits a little-endian 16-bit tensor into its low-byte plane (stored
raw) and its high-byte plane (zstd'd): lo = raw[0::2], hi = raw[1::2]
(formats/packed.py:49-50, 277-282), and merges them back with
raw[0::2] = lo; raw[1::2] = hi (formats/packed.py:376-378).  The same split is
applied here to spilled KV pages.  ``byteplane.c`` is an independent C
restatement; ``load_c()`` binds it when built.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

C_LIB = Path(__file__).resolve().parent / "liboracle_byteplane.so"


def split(raw_u16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    raw = np.ascontiguousarray(raw_u16, dtype=np.uint16).view(np.uint8)
    return raw[0::2].copy(), raw[1::2].copy()


def merge(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    raw = np.empty(len(hi) * 2, dtype=np.uint8)
    raw[0::2] = np.frombuffer(np.ascontiguousarray(lo, dtype=np.uint8), dtype=np.uint8)
    raw[1::2] = np.frombuffer(np.ascontiguousarray(hi, dtype=np.uint8), dtype=np.uint8)
    return raw.view(np.uint16)


def load_c():
    """ctypes handle of the C restatement, or None when it is not built."""
    if not C_LIB.exists():
        return None
    lib = ctypes.CDLL(str(C_LIB))
    lib.oracle_byteplane_split.restype = None
    lib.oracle_byteplane_split.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_size_t]
    lib.oracle_byteplane_merge.restype = None
    lib.oracle_byteplane_merge.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_size_t]
    return lib


def split_c(lib, raw_u16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    raw = np.ascontiguousarray(raw_u16, dtype=np.uint16)
    lo = np.empty(raw.size, dtype=np.uint8)
    hi = np.empty(raw.size, dtype=np.uint8)
    lib.oracle_byteplane_split(raw.ctypes.data, lo.ctypes.data, hi.ctypes.data, raw.size)
    return lo, hi


def merge_c(lib, lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    lo = np.ascontiguousarray(lo, dtype=np.uint8)
    hi = np.ascontiguousarray(hi, dtype=np.uint8)
    out = np.empty(lo.size, dtype=np.uint16)
    lib.oracle_byteplane_merge(lo.ctypes.data, hi.ctypes.data, out.ctypes.data, lo.size)
    return out
