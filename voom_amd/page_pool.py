"""Device page pool: per-layer K/V slot storage plus a free list of slot ids.

One slot holds one page of one sequence for one layer:
  k [capacity, num_kv_heads, page_tokens, head_dim]   token-major
  v [capacity, num_kv_heads, head_dim, page_tokens]   transposed page (V^T)
Allocation, recycling and 25 % geometric growth follow the reference's
PositionFreePagePool (runtime/kv_cache.py:316-414), with page_tokens-wide slots
instead of one-token pages.  Growth reallocates and copies the pool, so slot
ids stay valid while tensor addresses change.
"""

from __future__ import annotations

import torch


class DevicePagePool:
    def __init__(self, num_kv_heads: int, head_dim: int, page_tokens: int, *,
                 capacity: int = 0, dtype=torch.bfloat16, device=None, min_grow: int = 64):
        if num_kv_heads <= 0 or head_dim <= 0 or page_tokens <= 0:
            raise ValueError("page pool geometry must be positive")
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.page_tokens = int(page_tokens)
        self.dtype = dtype
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.min_grow = int(min_grow)
        self.k = self._empty_k(0)
        self.v = self._empty_v(0)
        self._free: list[int] = []
        self._live = 0
        if capacity:
            self.ensure_capacity(capacity)

    def _empty_k(self, n):
        return torch.empty((n, self.num_kv_heads, self.page_tokens, self.head_dim),
                           dtype=self.dtype, device=self.device)

    def _empty_v(self, n):
        return torch.empty((n, self.num_kv_heads, self.head_dim, self.page_tokens),
                           dtype=self.dtype, device=self.device)

    @property
    def capacity(self) -> int:
        return self.k.shape[0]

    @property
    def live_slots(self) -> int:
        return self._live

    @property
    def free_slots(self) -> int:
        return len(self._free)

    @property
    def slot_bytes(self) -> int:
        """Bytes of one K slot (the same for V)."""
        return self.num_kv_heads * self.page_tokens * self.head_dim * self.k.element_size()

    def ensure_capacity(self, required: int) -> None:
        cap = self.capacity
        if required <= cap:
            return
        target = max(required, cap + max(self.min_grow, cap // 4))
        k, v = self._empty_k(target), self._empty_v(target)
        if cap:
            k[:cap].copy_(self.k)
            v[:cap].copy_(self.v)
        self.k, self.v = k, v
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
        for i in ids:
            i = int(i)
            if not 0 <= i < self.capacity:
                raise RuntimeError(f"slot {i} outside the pool")
            self._free.append(i)
        self._live -= len(ids)
        if self._live < 0:
            raise RuntimeError("page pool released more slots than it allocated")
