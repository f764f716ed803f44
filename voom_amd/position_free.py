"""Position-free page pool and per-request cache over it.

K is stored before RoPE in one-token pages shared by reference between
requests; attention rotates each key at its logical position inside the HIP
kernel (voom_position_free_attention).  The interface, invariants and error
texts are those of the reference's PositionFreePagePool / PositionFreeKVCache
(runtime/kv_cache.py:255-808):

  * one page id names the same logical token in every layer;
  * a page is written once per layer, and only while its one owner holds it;
  * a page may be shared (``retain``) only after every layer is written;
  * ``release`` drops one reference per occurrence; dead pages are recycled;
  * ids stay valid while storage grows (25 % geometric steps, as there).

The bookkeeping is this build's own: reference counts and per-layer written
flags are numpy arrays, so allocate / retain / release / write validate and
update whole id lists at once (and a failing call changes nothing); free ids
sit on a stack that hands the most recently freed pages out first; a
request's page ids live in a device int32 vector that grows geometrically, so
``block_table()`` is a view uploaded incrementally instead of a tensor rebuilt
from a Python list; key positions are one grow-only device ``arange`` shared by
every request of the pool; RoPE tables are keyed by the denominators' values.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import ops


# The plan types of the reference's PIC path (runtime/tool_capsules.py:39-60):
# same fields, so plans built for the reference drive from_pic_plan unchanged.
@dataclass(frozen=True)
class ReusedRange:
    start: int
    end: int
    source_start: int
    kind: str

    @property
    def length(self) -> int:
        return self.end - self.start


@dataclass(frozen=True)
class ToolPICPlan:
    reused: tuple
    selected_positions: tuple
    exact_prefix_tokens: int
    capsule_tokens_reused: int
    capsule_tokens_repaired: int

    @property
    def selected_tokens(self) -> int:
        return len(self.selected_positions)


def _count_arg(value, what: str) -> int:
    if isinstance(value, bool) or not isinstance(value, (int, np.integer)) or value < 0:
        raise ValueError(f"position-free {what} count must be non-negative")
    return int(value)


def _ids(page_ids) -> np.ndarray:
    return np.asarray([int(v) for v in page_ids], dtype=np.int64)


class PositionFreePagePool:
    """Engine-wide write-once K/V pages for position-independent reuse."""

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
        self._storage: list[tuple[torch.Tensor, torch.Tensor] | None] = [None] * self.num_layers
        self._refs = np.zeros(0, dtype=np.int64)
        self._written = np.zeros((self.num_layers, 0), dtype=bool)
        self._stack = np.zeros(0, dtype=np.int64)  # free ids; the top is handed out first
        self._nfree = 0
        self._high = 0  # ids below this have been handed out at least once
        self._live = 0
        self._tables: dict = {}
        self._positions: torch.Tensor | None = None
        self._closed = False

    # ---- counters ---------------------------------------------------------------

    @property
    def capacity(self) -> int:
        return int(self._refs.size)

    @property
    def live_pages(self) -> int:
        return self._live

    @property
    def free_pages(self) -> int:
        return self._nfree

    def reference_count(self, page_id: int) -> int:
        if not 0 <= page_id < self._high:
            raise IndexError(page_id)
        return int(self._refs[page_id])

    def _check_open(self):
        if self._closed:
            raise RuntimeError("position-free page pool is closed")

    # ---- storage ----------------------------------------------------------------

    def _grow(self, required: int) -> None:
        cap = self.capacity
        if required <= cap:
            return
        # first allocation: at least min_capacity; then 25 % steps (at least
        # min_capacity each), the reference's growth rule
        target = max(required, cap + max(self.min_capacity, cap // 4) if cap else
                     self.min_capacity)
        extra = target - cap
        self._refs = np.concatenate([self._refs, np.zeros(extra, dtype=np.int64)])
        self._written = np.concatenate(
            [self._written, np.zeros((self.num_layers, extra), dtype=bool)], axis=1)
        self._stack = np.concatenate([self._stack, np.zeros(extra, dtype=np.int64)])
        for layer, kv in enumerate(self._storage):
            if kv is not None:
                self._storage[layer] = tuple(self._widen(t, target) for t in kv)

    def _widen(self, t: torch.Tensor, rows: int) -> torch.Tensor:
        new = torch.zeros((rows,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
        new[:t.shape[0]].copy_(t)
        return new

    def _layer_storage(self, layer: int, dtype) -> tuple[torch.Tensor, torch.Tensor]:
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        if dtype != self.dtype:
            raise ValueError(f"position-free pool dtype changed: {self.dtype} -> {dtype}")
        if self._storage[layer] is None:
            shape = (self.capacity, self.num_kv_heads, 1, self.head_dim)
            self._storage[layer] = (torch.zeros(shape, dtype=dtype, device=self.device),
                                    torch.zeros(shape, dtype=dtype, device=self.device))
        return self._storage[layer]

    # ---- ownership --------------------------------------------------------------

    def allocate(self, count: int) -> tuple[int, ...]:
        """Allocate ``count`` unique pages and transfer one reference to the caller."""
        self._check_open()
        count = _count_arg(count, "allocation")
        if count == 0:
            return ()
        take = min(count, self._nfree)
        fresh = count - take
        self._grow(self._high + fresh)
        # the top `take` free ids in the order they were freed: the reference
        # hands out _free[-take:] as a list slice (runtime/kv_cache.py:367-371)
        recycled = self._stack[self._nfree - take:self._nfree]
        ids = np.concatenate([recycled, np.arange(self._high, self._high + fresh)])
        if np.any(self._refs[ids] != 0):
            raise RuntimeError("position-free allocator recycled a live page")
        self._nfree -= take
        self._high += fresh
        self._refs[ids] = 1
        self._written[:, ids] = False
        self._live += count
        return tuple(int(i) for i in ids)

    def reserve_additional(self, count: int) -> None:
        """Make room for ``count`` further allocations without growing later."""
        self._check_open()
        count = _count_arg(count, "reserve")
        self._grow(self._high + max(0, count - self._nfree))

    def _active(self, ids: np.ndarray) -> np.ndarray:
        ok = (ids >= 0) & (ids < self._high)
        ok[ok] = self._refs[ids[ok]] > 0
        return ok

    def retain(self, page_ids) -> None:
        """Add one reference per occurrence in ``page_ids`` (complete pages only)."""
        self._check_open()
        ids = _ids(page_ids)
        ok = self._active(ids)
        if not ok.all():
            raise ValueError(f"cannot retain inactive page {int(ids[~ok][0])}")
        complete = self._written[:, ids].all(axis=0)
        if not complete.all():
            raise ValueError(f"cannot share incomplete page {int(ids[~complete][0])}")
        np.add.at(self._refs, ids, 1)

    def release(self, page_ids) -> None:
        """Drop one reference per occurrence; pages left unreferenced are recycled."""
        if self._closed:
            return
        ids = _ids(page_ids)
        if ids.size == 0:
            return
        uniq, counts = np.unique(ids, return_counts=True)
        valid = (uniq >= 0) & (uniq < self._high)
        over = ~valid
        over[valid] = self._refs[uniq[valid]] < counts[valid]
        if over.any():
            raise RuntimeError(f"position-free page {int(uniq[over][0])} released twice")
        self._refs[uniq] -= counts
        gone = self._refs[uniq] == 0
        if gone.any():
            # freed in the order the reference's loop frees them: a page dies at
            # its last occurrence in page_ids (runtime/kv_cache.py:402-414)
            last = ids.size - 1 - np.unique(ids[::-1], return_index=True)[1]
            dead = uniq[gone][np.argsort(last[gone], kind="stable")]
            self._written[:, dead] = False
            self._stack[self._nfree:self._nfree + dead.size] = dead
            self._nfree += dead.size
            self._live -= int(dead.size)

    # ---- contents -----------------------------------------------------------------

    def write(self, layer: int, page_ids, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Write the newly allocated pages of one layer, once.

        ``keys`` / ``values`` [1, NKV, L, D]: unrotated K and ordinary V.
        """
        self._check_open()
        ids = _ids(page_ids)
        if (keys.dim() != 4 or values.shape != keys.shape or keys.shape[0] != 1
                or keys.shape[1] != self.num_kv_heads or keys.shape[2] != ids.size
                or keys.shape[3] != self.head_dim):
            raise ValueError("position-free K/V write shape mismatch")
        k_store, v_store = self._layer_storage(layer, keys.dtype)
        owned = self._active(ids)
        owned[owned] = self._refs[ids[owned]] == 1
        if not owned.all():
            raise ValueError(f"position-free page {int(ids[~owned][0])} is not exclusively "
                             "writable")
        again = self._written[layer, ids]
        if again.any():
            raise ValueError(f"position-free page {int(ids[again][0])} layer {layer} "
                             "written twice")
        if ids.size:
            idx = torch.from_numpy(ids).to(self.device)
            # [1, NKV, L, D] -> [L, NKV, 1, D]: one page per token
            k_store.index_copy_(0, idx, keys.permute(2, 1, 0, 3).contiguous().to(self.device))
            v_store.index_copy_(0, idx, values.permute(2, 1, 0, 3).contiguous().to(self.device))
            self._written[layer, ids] = True

    def pages(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_open()
        if not 0 <= layer < self.num_layers or self._storage[layer] is None:
            raise ValueError(f"position-free layer {layer} has no materialized pages")
        return self._storage[layer]

    def gather(self, layer: int, page_ids) -> tuple[torch.Tensor, torch.Tensor]:
        """Pages in logical order as ordinary [1, NKV, S, D] tensors (unrotated K)."""
        self._check_open()
        ids = _ids(page_ids)
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        if self._storage[layer] is None:
            raise ValueError(f"position-free layer {layer} has no pages")
        readable = self._active(ids)
        readable[readable] = self._written[layer, ids[readable]]
        if not readable.all():
            raise ValueError(f"position-free layer {layer} page {int(ids[~readable][0])} "
                             "is unreadable")
        keys, values = self._storage[layer]
        idx = torch.from_numpy(ids).to(self.device)
        return (keys.index_select(0, idx).permute(2, 1, 0, 3),
                values.index_select(0, idx).permute(2, 1, 0, 3))

    def key_positions(self, n: int) -> torch.Tensor:
        """Positions 0 .. n-1 as device int32, a view of one grow-only arange."""
        if self._positions is None or self._positions.numel() < n:
            size = max(n, 2 * (0 if self._positions is None else self._positions.numel()), 256)
            self._positions = torch.arange(size, dtype=torch.int32, device=self.device)
        return self._positions[:n]

    def rope(self, max_position: int, theta: float, denominators=None):
        """fp32 cos/sin tables [n >= max_position, D/2] for the kernel, cached per
        (theta, denominators) and regrown by doubling when a longer one is asked."""
        self._check_open()
        if max_position <= 0:
            raise ValueError("position-free RoPE length must be positive")
        key = (float(theta), None if denominators is None else
               np.asarray(denominators, dtype=np.float64).tobytes())
        have = self._tables.get(key)
        if have is not None and have[0].shape[0] >= max_position:
            return have
        n = max_position if have is None else max(max_position, 2 * have[0].shape[0])
        tables = ops.rope_cache(n, self.head_dim, theta, denominators=denominators,
                                device=self.device)
        self._tables[key] = tables
        return tables

    def bytes_per_page(self) -> int:
        itemsize = torch.empty((), dtype=self.dtype).element_size()
        return self.num_layers * 2 * self.num_kv_heads * self.head_dim * self.block_size * itemsize

    def live_nbytes(self) -> int:
        return self.live_pages * self.bytes_per_page()

    def allocated_nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for kv in self._storage if kv is not None
                   for t in kv)

    def close(self):
        self._storage = [None] * self.num_layers
        self._tables.clear()
        self._positions = None
        self._refs = np.zeros(0, dtype=np.int64)
        self._written = np.zeros((self.num_layers, 0), dtype=bool)
        self._stack = np.zeros(0, dtype=np.int64)
        self._nfree = self._high = self._live = 0
        self._closed = True


class PositionFreeKVCache:
    """One request's logical sequence of pages in a shared PositionFreePagePool."""

    position_free = True
    custom_attention_query_limit = 4

    def __init__(self, pool: PositionFreePagePool):
        self.pool = pool
        self.num_layers = pool.num_layers
        self._host = np.zeros(0, dtype=np.int32)  # page id of each position
        self._n = 0
        self._dev: torch.Tensor | None = None  # device copy of _host
        self._synced = 0  # positions already on the device
        self._lengths = np.zeros(pool.num_layers, dtype=np.int64)
        self._released = False

    # ---- state ----------------------------------------------------------------------

    @property
    def page_ids(self) -> tuple[int, ...]:
        return tuple(int(i) for i in self._host[:self._n])

    @property
    def offset(self) -> int:
        return self._n

    @property
    def is_complete(self) -> bool:
        return not self._released and bool((self._lengths == self._n).all())

    def _check_owned(self):
        if self._released:
            raise RuntimeError("position-free cache has been released")

    def _set_ids(self, ids) -> None:
        ids = np.asarray(ids, dtype=np.int32)
        self._host = ids.copy()
        self._n = ids.size
        self._synced = 0

    def _extend(self, ids) -> None:
        ids = np.asarray(ids, dtype=np.int32)
        need = self._n + ids.size
        if need > self._host.size:
            grown = np.zeros(max(need, 2 * self._host.size, 64), dtype=np.int32)
            grown[:self._n] = self._host[:self._n]
            self._host = grown
        self._host[self._n:need] = ids
        self._n = need

    def _truncate(self, n: int) -> None:
        self._n = n
        self._synced = min(self._synced, n)

    # ---- writes -----------------------------------------------------------------------

    def update_unrotated(self, layer: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append unrotated K and ordinary V [1, NKV, L, D] to a layer.  The
        first layer to reach a new span allocates its pages; every layer must
        append the same span."""
        self._check_owned()
        if not 0 <= layer < self.num_layers:
            raise IndexError(layer)
        width = int(keys.shape[2]) if keys.dim() == 4 else -1
        start = int(self._lengths[layer])
        if start == self._n and width >= 0:
            self._extend(self.pool.allocate(width))
        if width < 0 or start + width != self._n:
            raise ValueError("position-free layers must append the same complete token span")
        self.pool.write(layer, self._host[start:start + width], keys, values)
        self._lengths[layer] = start + width

    def reserve_growth(self, positions: int) -> None:
        """Make room in the pool for ``positions`` more tokens of this request."""
        self._check_owned()
        self.pool.reserve_additional(positions)

    @classmethod
    def from_pic_plan(cls, source: "PositionFreeKVCache", plan,
                      length: int) -> "PositionFreeKVCache":
        """A destination of ``length`` positions whose reused ranges share the
        source's pages by reference and whose selected positions own fresh
        pages, to be filled by ``write_selected`` once per layer.  On an
        invalid plan nothing stays allocated or retained."""
        source._check_owned()
        if not source.is_complete:
            raise ValueError("PIC source position-free cache is incomplete")
        selected = np.asarray([int(p) for p in plan.selected_positions], dtype=np.int64)
        if length <= 0 or selected.size <= 0:
            raise ValueError("PIC destination needs selected positions")
        pool = source.pool
        fresh = np.asarray(pool.allocate(int(selected.size)), dtype=np.int64)
        try:
            layout = np.full(int(length), -1, dtype=np.int64)
            if (selected.min() < 0 or selected.max() >= length
                    or np.unique(selected).size != selected.size):
                raise ValueError("invalid PIC selected position layout")
            layout[selected] = fresh
            shared = []
            for r in plan.reused:
                n = r.end - r.start
                if (not 0 <= r.start < r.end <= length or r.source_start < 0
                        or r.source_start + n > source.offset):
                    raise ValueError("invalid PIC reused position layout")
                span = layout[r.start:r.end]
                if (span >= 0).any():
                    raise ValueError("overlapping PIC destination layout")
                span[:] = source._host[r.source_start:r.source_start + n]
                shared.append(span.copy())
            if (layout < 0).any():
                raise ValueError("PIC destination layout has uncovered positions")
            if shared:
                pool.retain(np.concatenate(shared))
        except Exception:
            pool.release(fresh)
            raise
        dest = cls(pool)
        dest._set_ids(layout)
        return dest

    def write_selected(self, layer: int, positions, keys: torch.Tensor,
                       values: torch.Tensor) -> None:
        """Fill the selected (fresh) positions of a PIC destination in one layer,
        which completes the layer."""
        self._check_owned()
        pos = np.asarray([int(p) for p in positions], dtype=np.int64)
        if self._lengths[layer] != 0:
            raise ValueError(f"PIC layer {layer} was already completed")
        if keys.dim() != 4 or keys.shape[2] != pos.size:
            raise ValueError("PIC selected K/V shape mismatch")
        if pos.size and (pos.min() < 0 or pos.max() >= self._n):
            raise ValueError("PIC selected position is outside destination")
        self.pool.write(layer, self._host[pos], keys, values)
        self._lengths[layer] = self._n

    def trim(self, length: int) -> None:
        """Keep the first ``length`` positions; later pages lose this request's
        reference (and are recycled when nobody else holds them)."""
        self._check_owned()
        if isinstance(length, bool) or not isinstance(length, int):
            raise ValueError("position-free trim length must be an integer")
        if not 0 <= length <= self._n:
            raise ValueError("position-free trim cannot grow the cache")
        if length == self._n:
            return
        self.pool.release(self._host[length:self._n])
        self._truncate(length)
        np.minimum(self._lengths, length, out=self._lengths)
        dsa = getattr(self, "dsa", None)
        if dsa is not None:
            dsa.trim(length)

    @classmethod
    def share_prefix(cls, source: "PositionFreeKVCache", length: int) -> "PositionFreeKVCache":
        """A new request whose first ``length`` tokens are the source's pages,
        shared by reference (they must be complete in every layer)."""
        source._check_owned()
        if not 0 <= length <= source.offset:
            raise ValueError("shared prefix longer than the source")
        ids = source._host[:length].copy()
        source.pool.retain(ids)
        dest = cls(source.pool)
        dest._set_ids(ids)
        dest._lengths[:] = length
        return dest

    # ---- reads ------------------------------------------------------------------------

    def gather_unrotated(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        self._check_owned()
        if self._lengths[layer] != self._n:
            raise ValueError(f"position-free layer {layer} is incomplete")
        return self.pool.gather(layer, self._host[:self._n])

    def block_table(self) -> torch.Tensor:
        """The request's page ids as a device int32 vector [offset]; positions
        added since the last call are uploaded, earlier ones stay put."""
        self._check_owned()
        if self._dev is None or self._dev.numel() < self._n:
            size = max(self._host.size, self._n, 64)
            dev = torch.empty(size, dtype=torch.int32, device=self.pool.device)
            if self._dev is not None and self._synced:
                dev[:self._synced].copy_(self._dev[:self._synced])
            self._dev = dev
        if self._synced < self._n:
            src = torch.from_numpy(self._host[self._synced:self._n].copy())
            self._dev[self._synced:self._n].copy_(src)
            self._synced = self._n
        return self._dev[:self._n]

    def key_positions(self) -> torch.Tensor:
        self._check_owned()
        return self.pool.key_positions(self._n)

    def paged_attention(self, layer: int, queries: torch.Tensor, query_positions: torch.Tensor,
                        *, theta: float, denominators=None, scale: float) -> torch.Tensor:
        """Attention of rotated queries [B, NQ, TQ, D] over this request's pages
        (runtime/kv_cache.py:688-701)."""
        self._check_owned()
        if self._lengths[layer] != self._n:
            raise ValueError(f"position-free layer {layer} is incomplete")
        keys, values = self.pool.pages(layer)
        qpos = query_positions.to(device=self.pool.device, dtype=torch.int32).contiguous()
        n = max(self._n, int(qpos.max()) + 1 if qpos.numel() else 1)
        cos, sin = self.pool.rope(n, theta, denominators)
        return ops.position_free_paged_attention(
            queries.contiguous(), keys, values, self.block_table(), self.key_positions(), qpos,
            cos, sin, scale=scale)

    def nbytes(self) -> int:
        return self._n * self.pool.bytes_per_page()

    def allocated_nbytes(self) -> int:
        return self.nbytes()

    def release(self) -> None:
        if self._released:
            return
        self.pool.release(self._host[:self._n])
        self._truncate(0)
        self._lengths[:] = 0
        self._dev = None
        self._released = True

    def __del__(self):
        # a last resort only: owners release explicitly and see errors there
        try:
            self.release()
        except Exception:
            pass
