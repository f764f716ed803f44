"""Spilled-page checksums restated on the CPU (test infrastructure only).

The reference keeps no checksum for spilled KV (runtime/kv_paged.py:77-113
writes and reads raw or zstd bytes); this build adds one, computed by the GPU
split kernel and re-checked by the merge (voom_amd/csrc/byteplane.hip).  The
definition, restated here with numpy: for one pool slot viewed as 32-bit
little-endian words w_0 .. w_{n-1},

    sum = SUM_j fmix32((w_j + j * 0x9E3779B9) mod 2^32)  mod 2^32

where fmix32 is the 32-bit finaliser of MurmurHash3 (Austin Appleby's public
domain hash): h ^= h >> 16; h *= 0x85EBCA6B; h ^= h >> 13; h *= 0xC2B2AE35;
h ^= h >> 16, all mod 2^32.
"""

from __future__ import annotations

import numpy as np

KEY = 0x9E3779B9


def fmix32(h: np.ndarray) -> np.ndarray:
    h = np.asarray(h, dtype=np.uint32).copy()
    h ^= h >> np.uint32(16)
    h *= np.uint32(0x85EBCA6B)
    h ^= h >> np.uint32(13)
    h *= np.uint32(0xC2B2AE35)
    h ^= h >> np.uint32(16)
    return h


def slot_sum(words: np.ndarray) -> int:
    """Checksum of one slot given as uint32 words (or any buffer, viewed as such)."""
    w = np.ascontiguousarray(words).view(np.uint32).reshape(-1)
    j = np.arange(w.size, dtype=np.uint64)
    keyed = ((w.astype(np.uint64) + j * KEY) & 0xFFFFFFFF).astype(np.uint32)
    return int(fmix32(keyed).astype(np.uint64).sum() & 0xFFFFFFFF)


def slot_sums(pool: np.ndarray, slots) -> np.ndarray:
    """int32 checksums of pool[slots[i]] (pool [num_slots, ...] of 16-bit words)."""
    out = [slot_sum(np.ascontiguousarray(pool[int(s)])) for s in slots]
    return np.asarray(out, dtype=np.uint32).view(np.int32)
