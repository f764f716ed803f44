"""Device page pool: per-layer slot storage plus a free list of slot ids.

A slot holds one page of one sequence for one layer, as one or more tensors
that share the slot index:
  KV pool      k [capacity, num_kv_heads, page_tokens, head_dim]   token-major
               v [capacity, num_kv_heads, page_tokens/VB, head_dim, VB]
                 V^T in blocks of VB = min(page_tokens, 32) tokens
  latent pool  lat [capacity, page_tokens, latent_dim]             token-major
Allocation, recycling and 25 % geometric growth follow the reference's
PositionFreePagePool (runtime/kv_cache.py:316-414), with page_tokens-wide slots
instead of one-token pages.  Growth reallocates and copies the pool, so slot
ids stay valid while tensor addresses change.
"""

from __future__ import annotations

import math

import torch


V_BLOCK = 32  # tokens per transposed V block inside a page


def v_slot_shape(num_kv_heads: int, head_dim: int, page_tokens: int) -> tuple[int, ...]:
    """Shape of one V slot: [NKV, page_tokens / VB, head_dim, VB], VB = min(PT, 32)."""
    vb = min(page_tokens, V_BLOCK)
    return (num_kv_heads, page_tokens // vb, head_dim, vb)


def v_pages_to_tokens(v: torch.Tensor) -> torch.Tensor:
    """Blocked V^T pages [n, NKV, PT/VB, D, VB] -> token-major view [n, NKV, PT, D]."""
    n, nkv, nb, d, vb = v.shape
    return v.permute(0, 1, 2, 4, 3).reshape(n, nkv, nb * vb, d)


def v_tokens_to_pages(v: torch.Tensor) -> torch.Tensor:
    """Token-major [n, NKV, PT, D] -> contiguous blocked V^T pages [n, NKV, PT/VB, D, VB]."""
    n, nkv, pt, d = v.shape
    vb = min(pt, V_BLOCK)
    return v.reshape(n, nkv, pt // vb, vb, d).transpose(3, 4).contiguous()


class DevicePagePool:
    def __init__(self, slot_shapes: list[tuple[int, ...]], *, capacity: int = 0,
                 dtype=torch.bfloat16, device=None, min_grow: int = 64):
        if not slot_shapes or any(d <= 0 for shp in slot_shapes for d in shp):
            raise ValueError("page pool geometry must be positive")
        self.slot_shapes = [tuple(int(d) for d in shp) for shp in slot_shapes]
        self.dtype = dtype
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.min_grow = int(min_grow)
        self.tensors = [self._empty(shp, 0) for shp in self.slot_shapes]
        self._free: list[int] = []
        self._live = 0
        if capacity:
            self.ensure_capacity(capacity)

    @classmethod
    def kv(cls, num_kv_heads: int, head_dim: int, page_tokens: int, **kw) -> "DevicePagePool":
        return cls([(num_kv_heads, page_tokens, head_dim),
                    v_slot_shape(num_kv_heads, head_dim, page_tokens)], **kw)

    @classmethod
    def rows(cls, page_tokens: int, row_elems: int, **kw) -> "DevicePagePool":
        return cls([(page_tokens, row_elems)], **kw)

    def _empty(self, shp, n):
        return torch.empty((n,) + shp, dtype=self.dtype, device=self.device)

    @property
    def k(self) -> torch.Tensor:
        return self.tensors[0]

    @property
    def v(self) -> torch.Tensor:
        return self.tensors[1]

    @property
    def lat(self) -> torch.Tensor:
        return self.tensors[0]

    @property
    def capacity(self) -> int:
        return self.tensors[0].shape[0]

    @property
    def live_slots(self) -> int:
        return self._live

    @property
    def free_slots(self) -> int:
        return len(self._free)

    def tensor_slot_bytes(self, i: int) -> int:
        """Bytes of one slot of tensor i."""
        return math.prod(self.slot_shapes[i]) * self.tensors[i].element_size()

    @property
    def slot_bytes(self) -> int:
        """Bytes of one slot across all tensors."""
        return sum(self.tensor_slot_bytes(i) for i in range(len(self.tensors)))

    def ensure_capacity(self, required: int) -> None:
        cap = self.capacity
        if required <= cap:
            return
        target = max(required, cap + max(self.min_grow, cap // 4))
        new = [self._empty(shp, target) for shp in self.slot_shapes]
        if cap:
            for dst, src in zip(new, self.tensors):
                dst[:cap].copy_(src)
        self.tensors = new
        # new ids are handed out lowest first
        self._free.extend(range(target - 1, cap - 1, -1))

    def allocate(self, count: int) -> list[int]:
        if count < 0:
            raise ValueError("allocation count must be non-negative")
        if count > len(self._free):
            self.ensure_capacity(self.capacity + count - len(self._free))
        ids = [self._free.pop() for _ in range(count)]
        self._live += count
        return ids

    def release(self, ids) -> None:
        ids = [int(i) for i in ids]
        if ids and not (0 <= min(ids) and max(ids) < self.capacity):
            raise RuntimeError(f"slot outside the pool (capacity {self.capacity})")
        self._free.extend(ids)
        self._live -= len(ids)
        if self._live < 0:
            raise RuntimeError("page pool released more slots than it allocated")
