"""bf16 <-> fp32 on uint16 words (test infrastructure only).

bf16 is the top half of an IEEE binary32.  fp32 -> bf16 rounds to nearest,
ties to even, the IEEE default; NaNs are kept quiet.  This is the conversion
the reference relies on whenever MLX casts to bfloat16 (e.g.
runtime/glm.py:159-161) and the storage view of runtime/kv_paged.py:56-61.
"""

from __future__ import annotations

import numpy as np


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 value after a round trip through bf16."""
    return bf16_to_f32(f32_to_bf16(x))
