"""Position-free page pool and cache: K stored before RoPE in shared,
refcounted, write-once one-token pages; attention rotates each key at its
logical position (voom_position_free_attention).

Restates PositionFreePagePool / PositionFreeKVCache (runtime/kv_cache.py:
255-701) with the same names, invariants and errors:
  * one physical page id names the same logical token in every layer; a page
    is written exactly once per layer, by its only owner (refcount 1);
  * a page may be retained (shared) only after every layer has been written;
  * release drops one reference per occurrence; dead pages are recycled;
  * storage grows by 25 % geometric steps, so ids stay valid across growth.
Pages live in device tensors [capacity, NKV, 1, D] per layer; the fp32 RoPE
tables are cached grow-only, as the reference does (kv_cache.py:504-526).
"""

from __future__ import annotations

import torch

from . import ops


class PositionFreePagePool:
    """Engine-wide immutable K/V pages for position-independent reuse."""

    block_size = 1

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, *,
                 min_capacity: int = 256, device=None, dtype=torch.bfloat16):
        if num_layers <= 0 or num_kv_heads <= 0 or head_dim <= 0:
            raise ValueError("position-free page geometry must be positive")
        if min_capacity <= 0:
            raise ValueError("position-free minimum capacity must be positive")
        self.num_layers = int(num_layers)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.min_capacity = int(min_capacity)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.dtype = dtype
        self.key_pages: list[torch.Tensor | None] = [None] * self.num_layers
        self.value_pages: list[torch.Tensor | None] = [None] * self.num_layers
        self._refs: list[int] = []
        self._written_masks: list[int] = []
        self._free: list[int] = []
        self._next_id = 0
        self._live_pages = 0
        self._capacity = 0
        self._rope_entries: dict = {}
        self._closed = False

    @property
    def capacity(self) -> int:
        return self._capacity

    @property
    def live_pages(self) -> int:
        return self._live_pages

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def reference_count(self, page_id: int) -> int:
        if not 0 <= page_id < self._next_id:
            raise IndexError(page_id)
        return self._refs[page_id]

    def _check_open(self):
        if self._closed:
            raise RuntimeError("position-free page pool is closed")

    def _ensure_capacity(self, required: int):
        if required <= self._capacity:
            return
        if self._capacity == 0:
            target = max(required, self.min_capacity)
        else:
            target = max(required, self._capacity + max(self.min_capacity, self._capacity // 4))
        shape = (target, self.num_kv_heads, 1, self.head_dim)
        for layer in range(self.num_layers):
            for pages in (self.key_pages, self.value_pages):
                old = pages[layer]
                if old is None:
                    continue
                new = torch.zeros(shape, dtype=old.dtype, device=self.device)
                new[:self._capacity].copy_(old)
                pages[layer] = new
        extra = target - self._capacity
        self._refs.extend([0] * extra)
        self._written_masks.extend([0] * extra)
        self._capacity = target

    def allocate(self, count: int) -> tuple[int, ...]:
        """Allocate ``count`` unique pages and transfer one reference to the caller."""
        self._check_open()
        if isinstance(count, bool) or not isinstance(count, int) or count < 0:
            raise ValueError("position-free allocation count must be non-negative")
        if count == 0:
            return ()
        recycled_count = min(count, len(self._free))
        new_count = count - recycled_count
        self._ensure_capacity(self._next_id + new_count)
        recycled = self._free[-recycled_count:] if recycled_count else []
        if recycled_count:
            del self._free[-recycled_count:]
        fresh = list(range(self._next_id, self._next_id + new_count))
        self._next_id += new_count
        page_ids = recycled + fresh
        for page_id in page_ids:
            if self._refs[page_id] != 0:
                raise RuntimeError("position-free allocator recycled a live page")
            self._refs[page_id] = 1
            self._live_pages += 1
            self._written_masks[page_id] = 0
        return tuple(page_ids)

    def reserve_additional(self, count: int) -> None:
        """Reserve enough physical ids for ``count`` further allocations."""
        self._check_open()
        if isinstance(count, bool) or not isinstance(count, int) or count < 0:
            raise ValueError("position-free reserve count must be non-negative")
        self._ensure_capacity(self._next_id + max(0, count - len(self._free)))

    def retain(self, page_ids) -> None:
        """Add one reference per logical occurrence in ``page_ids``."""
        self._check_open()
        full_mask = (1 << self.num_layers) - 1
        ids = tuple(int(value) for value in page_ids)
        for page_id in ids:
            if not 0 <= page_id < self._next_id or self._refs[page_id] <= 0:
                raise ValueError(f"cannot retain inactive page {page_id}")
            if self._written_masks[page_id] != full_mask:
                raise ValueError(f"cannot share incomplete page {page_id}")
        for page_id in ids:
            self._refs[page_id] += 1

    def release(self, page_ids) -> None:
        """Drop one reference per occurrence and return dead pages to the free list."""
        if self._closed:
            return
        for value in page_ids:
            page_id = int(value)
            if not 0 <= page_id < self._next_id or self._refs[page_id] <= 0:
                raise RuntimeError(f"position-free page {page_id} released twice")
            self._refs[page_id] -= 1
            if self._refs[page_id] == 0:
                self._live_pages -= 1
                self._written_masks[page_id] = 0
                self._free.append(page_id)

    def _ensure_layer(self, layer: int, dtype):
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        if dtype != self.dtype:
            raise ValueError(f"position-free pool dtype is {self.dtype}, got {dtype}")
        if self.key_pages[layer] is None:
            shape = (self._capacity, self.num_kv_heads, 1, self.head_dim)
            self.key_pages[layer] = torch.zeros(shape, dtype=dtype, device=self.device)
            self.value_pages[layer] = torch.zeros(shape, dtype=dtype, device=self.device)

    def write(self, layer: int, page_ids, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Write newly allocated pages of one layer exactly once.

        ``keys`` / ``values`` [1, NKV, L, D]: unrotated K and ordinary V.
        """
        self._check_open()
        ids = tuple(int(value) for value in page_ids)
        if (keys.dim() != 4 or values.shape != keys.shape or keys.shape[0] != 1
                or keys.shape[1] != self.num_kv_heads or keys.shape[2] != len(ids)
                or keys.shape[3] != self.head_dim):
            raise ValueError("position-free K/V write shape mismatch")
        self._ensure_layer(layer, keys.dtype)
        bit = 1 << layer
        for page_id in ids:
            if not 0 <= page_id < self._next_id or self._refs[page_id] != 1:
                raise ValueError(f"position-free page {page_id} is not exclusively writable")
            if self._written_masks[page_id] & bit:
                raise ValueError(f"position-free page {page_id} layer {layer} written twice")
        if ids:
            # [1, NKV, L, D] -> [L, NKV, 1, D], the physical page layout
            idx = torch.tensor(ids, dtype=torch.long, device=self.device)
            self.key_pages[layer].index_copy_(0, idx, keys.permute(2, 1, 0, 3).contiguous())
            self.value_pages[layer].index_copy_(0, idx, values.permute(2, 1, 0, 3).contiguous())
            for page_id in ids:
                self._written_masks[page_id] |= bit

    def _validate_read(self, layer: int, page_ids):
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        if self.key_pages[layer] is None:
            raise ValueError(f"position-free layer {layer} has no pages")
        bit = 1 << layer
        for page_id in page_ids:
            if (not 0 <= page_id < self._next_id or self._refs[page_id] <= 0
                    or not (self._written_masks[page_id] & bit)):
                raise ValueError(f"position-free layer {layer} page {page_id} is unreadable")

    def pages(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_open()
        if not 0 <= layer < self.num_layers or self.key_pages[layer] is None:
            raise ValueError(f"position-free layer {layer} has no materialized pages")
        return self.key_pages[layer], self.value_pages[layer]

    def gather(self, layer: int, page_ids) -> tuple[torch.Tensor, torch.Tensor]:
        """Logical order as ordinary [1, NKV, S, D] tensors (unrotated K)."""
        self._check_open()
        ids = tuple(int(value) for value in page_ids)
        self._validate_read(layer, ids)
        keys, values = self.pages(layer)
        idx = torch.tensor(ids, dtype=torch.long, device=self.device)
        return (keys.index_select(0, idx).permute(2, 1, 0, 3),
                values.index_select(0, idx).permute(2, 1, 0, 3))

    def rope(self, max_position: int, theta: float, denominators=None):
        """Grow-only fp32 cos/sin tables [n >= max_position, D/2] for the kernel."""
        self._check_open()
        if max_position <= 0:
            raise ValueError("position-free RoPE length must be positive")
        identity = (float(theta), id(denominators))
        existing = self._rope_entries.get(identity)
        if existing is not None and existing[0] >= max_position:
            return existing[1], existing[2]
        target = max_position if existing is None else max(
            max_position, existing[0] + max(256, existing[0] // 4))
        cos, sin = ops.rope_cache(target, self.head_dim, theta, denominators=denominators,
                                  device=self.device)
        self._rope_entries[identity] = (target, cos, sin)
        return cos, sin

    def bytes_per_page(self) -> int:
        itemsize = torch.empty((), dtype=self.dtype).element_size()
        return self.num_layers * 2 * self.num_kv_heads * self.head_dim * self.block_size * itemsize

    def live_nbytes(self) -> int:
        return self.live_pages * self.bytes_per_page()

    def close(self):
        self.key_pages = [None] * self.num_layers
        self.value_pages = [None] * self.num_layers
        self._rope_entries.clear()
        self._refs.clear()
        self._written_masks.clear()
        self._free.clear()
        self._next_id = 0
        self._live_pages = 0
        self._capacity = 0
        self._closed = True


class PositionFreeKVCache:
    """One request's logical block table over a shared PositionFreePagePool."""

    position_free = True
    custom_attention_query_limit = 4

    def __init__(self, pool: PositionFreePagePool):
        self.pool = pool
        self.num_layers = pool.num_layers
        self._page_ids: list[int] = []
        self._layer_lengths = [0] * pool.num_layers
        self._table_cache: torch.Tensor | None = None
        self._positions_cache: torch.Tensor | None = None
        self._released = False

    @property
    def page_ids(self) -> tuple[int, ...]:
        return tuple(self._page_ids)

    @property
    def offset(self) -> int:
        return len(self._page_ids)

    @property
    def is_complete(self) -> bool:
        return not self._released and all(n == self.offset for n in self._layer_lengths)

    def _check_owned(self):
        if self._released:
            raise RuntimeError("position-free cache has been released")

    def _invalidate(self):
        self._table_cache = None
        self._positions_cache = None

    def update_unrotated(self, layer: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append unrotated K and ordinary V [1, NKV, L, D] to a layer.  The first
        layer to reach a new span allocates its pages; every layer must append
        the same span."""
        self._check_owned()
        if not 0 <= layer < len(self._layer_lengths):
            raise IndexError(layer)
        width = int(keys.shape[2]) if keys.dim() == 4 else -1
        previous = self._layer_lengths[layer]
        if previous == self.offset:
            self._page_ids.extend(self.pool.allocate(width))
            self._invalidate()
        if width < 0 or previous + width != self.offset:
            raise ValueError("position-free layers must append the same complete token span")
        self.pool.write(layer, self._page_ids[previous:previous + width], keys, values)
        self._layer_lengths[layer] = previous + width

    def gather_unrotated(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_owned()
        if self._layer_lengths[layer] != self.offset:
            raise ValueError(f"position-free layer {layer} is incomplete")
        return self.pool.gather(layer, self._page_ids)

    def block_table(self) -> torch.Tensor:
        self._check_owned()
        if self._table_cache is None:
            self._table_cache = torch.tensor(self._page_ids, dtype=torch.int32,
                                             device=self.pool.device)
        return self._table_cache

    def key_positions(self) -> torch.Tensor:
        self._check_owned()
        if self._positions_cache is None:
            self._positions_cache = torch.arange(self.offset, dtype=torch.int32,
                                                 device=self.pool.device)
        return self._positions_cache

    def paged_attention(self, layer: int, queries: torch.Tensor, query_positions: torch.Tensor,
                        *, theta: float, denominators=None, scale: float) -> torch.Tensor:
        """Attention of rotated queries [B, NQ, TQ, D] over this request's pages
        (runtime/kv_cache.py:688-701)."""
        self._check_owned()
        if self._layer_lengths[layer] != self.offset:
            raise ValueError(f"position-free layer {layer} is incomplete")
        keys, values = self.pool.pages(layer)
        qpos = query_positions.to(device=self.pool.device, dtype=torch.int32).contiguous()
        n = max(self.offset, int(qpos.max()) + 1 if qpos.numel() else 1)
        cos, sin = self.pool.rope(n, theta, denominators)
        return ops.position_free_paged_attention(
            queries.contiguous(), keys, values, self.block_table(), self.key_positions(), qpos,
            cos, sin, scale=scale)

    @classmethod
    def share_prefix(cls, source: "PositionFreeKVCache", length: int) -> "PositionFreeKVCache":
        """A new cache whose first ``length`` tokens are the source's pages,
        shared by reference (the pages must be complete in every layer)."""
        source._check_owned()
        if not 0 <= length <= source.offset:
            raise ValueError("shared prefix longer than the source")
        ids = source._page_ids[:length]
        source.pool.retain(ids)
        dest = cls(source.pool)
        dest._page_ids = list(ids)
        dest._layer_lengths = [length] * source.num_layers
        return dest

    def release(self) -> None:
        if self._released:
            return
        self.pool.release(self._page_ids)
        self._page_ids = []
        self._layer_lengths = [0] * self.num_layers
        self._invalidate()
        self._released = True
