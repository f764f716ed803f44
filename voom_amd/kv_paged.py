"""PagedKVCache on MI355X: fixed-size KV pages in a device page pool, spilled
to pinned host memory as byte planes and reloaded through a side stream.

This keeps the reference's cache protocol (runtime/kv_paged.py:116-240):
``PagedKVCache(num_layers, max_bytes, spill_dir, page_positions=256,
resident_pages=1, compress_spill=False)`` with ``update(layer, k, v)``,
``offset``, ``nbytes()``, ``release()``, ``stats`` and the ``_pages``
introspection its tests use, and adds the explicit verbs of the paged path:

  append(layer, k, v)      slot write through the block table, no concatenation
  attend(layer, q, scale)  fused paged decode attention (HIP kernel); spilled
                           pages are reloaded on a side stream while the
                           resident pages are attended, then LSE-merged
  spill(pages)             byte-plane split on the GPU -> D2H into the arena
  reload(pages)            H2D -> byte-plane merge into fresh pool slots

Where the reference differs by platform:
  * Pages live in one device pool per layer (slot = one sequence's page) and
    are addressed through a per-layer block table, instead of per-layer lists
    of MLX arrays that are concatenated on every call (kv_paged.py:164-181).
  * The spill target is pinned host memory (the HBM <-> host boundary exists
    on MI355X; Apple unified memory has none), and a page is stored as its
    low-byte and high-byte planes (formats/packed.py:49-50).  With
    ``compress_spill`` the high plane is zstd level 1 compressed on the host,
    as vpack does; the low plane stays raw.
  * Budget accounting, page closing and the eviction order are the
    reference's (kv_paged.py:143-162, 187-194, 216-240).
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import ops
from . import zstd as _zstd
from .host_arena import HostArena, HostBlock
from .page_pool import DevicePagePool


@dataclass
class KVStats:
    """Counters of kv_paged.py:35-53 (same fields and summary text)."""

    spills: int = 0
    reloads: int = 0
    spill_s: float = 0.0
    reload_s: float = 0.0
    spill_bytes_raw: int = 0  # only tracked when compress_spill is on
    spill_bytes_compressed: int = 0

    def summary(self) -> str:
        base = (
            f"kv: {self.spills} pages spilled ({self.spill_s:.2f}s), "
            f"{self.reloads} page reloads ({self.reload_s:.2f}s)"
        )
        if self.spill_bytes_compressed:
            ratio = self.spill_bytes_raw / self.spill_bytes_compressed
            base += (f", compress {ratio:.2f}x ({self.spill_bytes_raw / 1e6:.1f}"
                     f"->{self.spill_bytes_compressed / 1e6:.1f}MB)")
        return base


class _SpillBlock:
    """Host copy of a batch of pages spilled together from one layer.

    Layout of ``block``: four parts, each ``n_pages * part_bytes`` long --
    K low plane, V low plane, K high plane, V high plane -- page j at offset
    ``j * part_bytes`` in each part.  ``ready`` is recorded after the D2H copy.
    """

    __slots__ = ("block", "n_pages", "part_bytes", "ready", "live", "compressed")

    def __init__(self, block: HostBlock, n_pages: int, part_bytes: int):
        self.block = block
        self.n_pages = n_pages
        self.part_bytes = part_bytes
        self.ready: torch.cuda.Event | None = None
        self.live = n_pages
        # per page: (k_hi_frame, v_hi_frame) when the hi plane is compressed
        self.compressed: list[tuple[np.ndarray, np.ndarray] | None] = [None] * n_pages

    def part(self, which: int, j: int, n: int = 1) -> torch.Tensor:
        off = which * self.n_pages * self.part_bytes + j * self.part_bytes
        return self.block.view[off:off + n * self.part_bytes]


class _Page:
    """One closed page of one layer: a pool slot per sequence, or a host copy."""

    __slots__ = ("cache", "layer", "index", "slots", "host", "host_j", "nbytes", "path",
                 "_compressed")

    def __init__(self, cache: "PagedKVCache", layer: int, index: int, slots: list[int],
                 nbytes: int):
        self.cache = cache
        self.layer = layer
        self.index = index
        self.slots: list[int] | None = slots
        self.host: _SpillBlock | None = None
        self.host_j = 0
        self.nbytes = nbytes
        self.path: Path | None = None
        self._compressed = False

    @property
    def resident(self) -> bool:
        return self.slots is not None

    def load(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The page's K and V as [B, NKV, page_positions, D] (bit-exact)."""
        return self.cache._page_tensors(self)


def budget_victims(pages: list[list], resident_pages: int, current_bytes: int,
                   max_bytes: int) -> list[tuple[int, int]]:
    """Pages to spill so resident bytes fall to ``max_bytes``.

    The reference's order (kv_paged.py:216-240): oldest page index first,
    round-robin over layers, never the newest ``resident_pages`` closed pages
    of a layer, stopping as soon as the total is within budget.  ``pages`` is
    a per-layer list of objects with ``resident`` and ``nbytes``.
    """
    if current_bytes <= max_bytes or not pages:
        return []
    out = []
    longest = max((len(p) for p in pages), default=0)
    for page_idx in range(longest):
        for layer, layer_pages in enumerate(pages):
            if page_idx >= len(layer_pages) - resident_pages:
                continue
            page = layer_pages[page_idx]
            if not page.resident:
                continue
            out.append((layer, page_idx))
            current_bytes -= page.nbytes
            if current_bytes <= max_bytes:
                return out
    return out


class PagedKVCache:
    """Drop-in for the reference PagedKVCache, backed by device page pools."""

    def __init__(self, num_layers: int, max_bytes: int, spill_dir: str | Path | None = None,
                 page_positions: int = 256, resident_pages: int = 1,
                 compress_spill: bool = False, *, device=None, initial_slots: int = 0,
                 arena: HostArena | None = None):
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if page_positions <= 0 or page_positions & (page_positions - 1):
            raise ValueError("page_positions must be a power of two")
        self.num_layers = num_layers
        self.max_bytes = max_bytes
        self.page_positions = page_positions
        self.resident_pages = resident_pages
        self.compress_spill = compress_spill
        # The spill target is the pinned host arena; spill_dir is kept for
        # interface compatibility and created when given.
        self.spill_dir = Path(spill_dir) if spill_dir is not None else None
        if self.spill_dir is not None:
            self.spill_dir.mkdir(parents=True, exist_ok=True)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.initial_slots = initial_slots
        self.arena = arena if arena is not None else HostArena()
        self._own_arena = arena is None
        self.stats = KVStats()
        self._copy_stream: torch.cuda.Stream | None = None
        self._reset_state()

    # ---- state ------------------------------------------------------------

    def _reset_state(self):
        L = self.num_layers
        self._pages: list[list[_Page]] = [[] for _ in range(L)]
        # slots of allocated pages that are not closed yet (page index -> slots)
        self._open_slots: list[dict[int, list[int]]] = [{} for _ in range(L)]
        self._len = [0] * L
        self._offset = 0
        self._pools: list[DevicePagePool | None] = [None] * L
        self._stage_pools: list[DevicePagePool | None] = [None] * L
        self._tables: list[torch.Tensor | None] = [None] * L
        self._tables_host: list[np.ndarray | None] = [None] * L
        self._geom: tuple[int, int, int] | None = None  # (B, NKV, D)

    def _init_geometry(self, k: torch.Tensor):
        if k.dim() != 4:
            raise ValueError("k/v must be [B, num_kv_heads, L, head_dim]")
        B, NKV, _, D = k.shape
        if self._geom is None:
            if k.dtype != torch.bfloat16:
                raise ValueError("PagedKVCache stores bfloat16 K/V")
            self._geom = (B, NKV, D)
        elif self._geom != (B, NKV, D):
            raise ValueError(f"K/V geometry changed: {self._geom} -> {(B, NKV, D)}")

    def _pool(self, layer: int) -> DevicePagePool:
        pool = self._pools[layer]
        if pool is None:
            B, NKV, D = self._geom
            pool = DevicePagePool(NKV, D, self.page_positions, capacity=self.initial_slots,
                                  device=self.device)
            self._pools[layer] = pool
        return pool

    def _stage_pool(self, layer: int) -> DevicePagePool:
        pool = self._stage_pools[layer]
        if pool is None:
            B, NKV, D = self._geom
            pool = DevicePagePool(NKV, D, self.page_positions, device=self.device, min_grow=16)
            self._stage_pools[layer] = pool
        return pool

    def _stream(self) -> torch.cuda.Stream:
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=self.device)
        return self._copy_stream

    @property
    def page_nbytes(self) -> int:
        B, NKV, D = self._geom
        return B * NKV * self.page_positions * D * 2 * 2

    def _token_nbytes(self) -> int:
        B, NKV, D = self._geom
        return B * NKV * D * 2 * 2

    def _set_table_cols(self, layer: int, cols: dict[int, list[int] | None]) -> None:
        """Set block-table columns (page index -> B slots, or None = not resident)."""
        B = self._geom[0]
        host = self._tables_host[layer]
        need = max(cols) + 1
        if host is None or need > host.shape[1]:
            cap = max(16, need * 2)
            new = np.full((B, cap), -1, dtype=np.int32)
            if host is not None:
                new[:, :host.shape[1]] = host
            self._tables_host[layer] = host = new
            self._tables[layer] = torch.from_numpy(new).to(self.device)
            for page, slots in cols.items():
                host[:, page] = -1 if slots is None else np.asarray(slots, np.int32)
            self._tables[layer].copy_(torch.from_numpy(host))
            return
        for page, slots in cols.items():
            host[:, page] = -1 if slots is None else np.asarray(slots, np.int32)
        lo, hi = min(cols), max(cols) + 1
        self._tables[layer][:, lo:hi].copy_(torch.from_numpy(np.ascontiguousarray(host[:, lo:hi])))

    def _set_table(self, layer: int, page_idx: int, slots) -> None:
        self._set_table_cols(layer, {page_idx: slots})

    # ---- reference protocol -------------------------------------------------

    @property
    def offset(self) -> int:
        return self._offset

    def layer_length(self, layer: int) -> int:
        return self._len[layer]

    def nbytes(self) -> int:
        """Resident bytes: resident closed pages plus open-page tokens (kv_paged.py:187-194)."""
        if self._geom is None:
            return 0
        total = 0
        tok = self._token_nbytes()
        for layer in range(self.num_layers):
            total += sum(p.nbytes for p in self._pages[layer] if p.resident)
            total += (self._len[layer] - len(self._pages[layer]) * self.page_positions) * tok
        return total

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write k, v [B, NKV, L, D] after the layer's current tokens (slot writes).

        Pages that fill up are closed (kv_paged.py:150-158); after the last
        layer the offset advances and the budget is enforced (:160-162).
        """
        self._init_geometry(k)
        if v.shape != k.shape:
            raise ValueError("k and v shapes differ")
        L = k.shape[2]
        B = self._geom[0]
        pool = self._pool(layer)
        start = self._len[layer]
        end = start + L
        PT = self.page_positions
        new_pages = range(-(-start // PT), -(-end // PT))
        if len(new_pages):
            slots = pool.allocate(B * len(new_pages))
            cols = {}
            for j, page in enumerate(new_pages):
                cols[page] = slots[j * B:(j + 1) * B]
                self._open_slots[layer][page] = cols[page]
            self._set_table_cols(layer, cols)
        if L:
            pos = torch.full((B,), start, dtype=torch.int32, device=self.device)
            ops.append_kv(k.contiguous(), v.contiguous(), pool.k, pool.v, self._tables[layer],
                          pos)
        self._len[layer] = end
        pages = self._pages[layer]
        while (len(pages) + 1) * PT <= end:
            idx = len(pages)
            pages.append(_Page(self, layer, idx, self._open_slots[layer].pop(idx),
                               self.page_nbytes))
        if layer == self.num_layers - 1:
            self._offset += L
            self._enforce_budget()

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        """Append, then return the layer's full K/V [B, NKV, S, D] (kv_paged.py:143-181).

        Spilled pages are reloaded transiently for this call, as the
        reference does; prefer ``attend`` on the decode path.
        """
        self.append(layer, k, v)
        return self.gather(layer)

    def gather(self, layer: int):
        """Logical K/V [B, NKV, S, D] of a layer, spilled pages reloaded transiently."""
        S = self._len[layer]
        pool = self._pool(layer)
        spilled = [p for p in self._pages[layer] if not p.resident]
        if not spilled:
            return ops.gather_kv(pool.k, pool.v, self._tables[layer], S)
        stage, slots = self._transient_reload(layer, spilled)
        table = self._tables[layer].clone()
        # Point spilled pages at their staging slots (a second pool): gather
        # resident and staged pages separately and interleave by page.
        k_res, v_res = ops.gather_kv(pool.k, pool.v, self._resident_table(layer, table), S)
        B, NKV, D = self._geom
        PT = self.page_positions
        st_table = torch.full_like(table, -1)
        for j, p in enumerate(spilled):
            st_table[:, p.index] = torch.tensor(slots[j * B:(j + 1) * B], dtype=torch.int32,
                                                device=self.device)
        torch.cuda.current_stream().wait_stream(self._stream())
        k_st, v_st = ops.gather_kv(stage.k, stage.v, st_table, S)
        mask = torch.zeros(S, dtype=torch.bool, device=self.device)
        for p in spilled:
            mask[p.index * PT:(p.index + 1) * PT] = True
        k_all = torch.where(mask[None, None, :, None], k_st, k_res)
        v_all = torch.where(mask[None, None, :, None], v_st, v_res)
        self._release_stage(layer, slots)
        return k_all, v_all

    def _resident_table(self, layer: int, table: torch.Tensor) -> torch.Tensor:
        t = table.clone()
        for p in self._pages[layer]:
            if not p.resident:
                t[:, p.index] = -1
        return t

    def release(self) -> None:
        """Free device slots and host copies; offset and nbytes return to 0."""
        if self._own_arena:
            self.arena.close()
        else:
            seen = set()
            for pages in self._pages:
                for p in pages:
                    if p.host is not None and id(p.host) not in seen:
                        seen.add(id(p.host))
                        self.arena.free(p.host.block)
        paths = {p.path for pages in self._pages for p in pages if p.path is not None}
        self._reset_state()
        for path in paths:
            try:
                path.unlink()
            except FileNotFoundError:
                pass

    # ---- spilling -----------------------------------------------------------

    def _enforce_budget(self) -> None:
        victims = budget_victims(self._pages, self.resident_pages, self.nbytes(), self.max_bytes)
        if victims:
            self.spill([self._pages[l][i] for l, i in victims])

    def spill(self, pages=None) -> int:
        """Spill pages (``_Page`` objects or (layer, index) pairs) to the host arena.

        ``None`` applies the budget policy.  Returns the number of pages spilled.
        """
        if pages is None:
            before = self.stats.spills
            self._enforce_budget()
            return self.stats.spills - before
        pages = [self._pages[p[0]][p[1]] if isinstance(p, tuple) else p for p in pages]
        pages = [p for p in pages if p.resident]
        by_layer: dict[int, list[_Page]] = {}
        for p in pages:
            by_layer.setdefault(p.layer, []).append(p)
        t0 = time.perf_counter()
        for layer, lp in by_layer.items():
            self._spill_layer(layer, lp)
        if self.compress_spill:
            self._compress_spilled(pages)
        self.stats.spills += len(pages)
        self.stats.spill_s += time.perf_counter() - t0
        return len(pages)

    def _spill_layer(self, layer: int, pages: list[_Page]) -> None:
        B = self._geom[0]
        pool = self._pool(layer)
        part = B * pool.slot_bytes // 2            # bytes of one plane of K (or V) of a page
        n = len(pages)
        block = self.arena.alloc(4 * n * part)
        sb = _SpillBlock(block, n, part)
        slots = [s for p in pages for s in p.slots]
        main = torch.cuda.current_stream()
        copy = self._stream()
        slot_t = torch.tensor(slots, dtype=torch.int32, device=self.device)
        staging = torch.empty(4 * n * part, dtype=torch.uint8, device=self.device)
        # Split on the main stream (ordered after the writes of the pages), copy
        # to the host on the side stream.
        lo_k, lo_v = staging[0:n * part], staging[n * part:2 * n * part]
        hi_k, hi_v = staging[2 * n * part:3 * n * part], staging[3 * n * part:]
        if ops.slot_codec_supported(pool.k):
            ops.byteplane_split_slots(pool.k, slot_t, lo_k, hi_k)
            ops.byteplane_split_slots(pool.v, slot_t, lo_v, hi_v)
        else:
            idx = slot_t.long()
            ops.byteplane_split(pool.k.index_select(0, idx).contiguous(), lo_k, hi_k)
            ops.byteplane_split(pool.v.index_select(0, idx).contiguous(), lo_v, hi_v)
        split_done = torch.cuda.Event()
        split_done.record(main)
        copy.wait_event(split_done)
        with torch.cuda.stream(copy):
            block.view.copy_(staging, non_blocking=True)
            staging.record_stream(copy)
        sb.ready = torch.cuda.Event()
        sb.ready.record(copy)
        for j, p in enumerate(pages):
            pool.release(p.slots)
            p.slots = None
            p.host = sb
            p.host_j = j
        self._set_table_cols(layer, {p.index: None for p in pages})

    def _compress_spilled(self, pages: list[_Page]) -> None:
        for p in pages:
            sb = p.host
            sb.ready.synchronize()
            k_hi = sb.part(2, p.host_j).numpy()
            v_hi = sb.part(3, p.host_j).numpy()
            kz, vz = _zstd.compress(k_hi, 1), _zstd.compress(v_hi, 1)
            sb.compressed[p.host_j] = (kz, vz)
            p._compressed = True
            self.stats.spill_bytes_raw += p.nbytes
            self.stats.spill_bytes_compressed += 2 * sb.part_bytes + kz.nbytes + vz.nbytes

    def _host_planes(self, p: _Page, stage: torch.Tensor | None = None):
        """Pinned (lo_k, lo_v, hi_k, hi_v) host tensors of a spilled page."""
        sb = p.host
        parts = [sb.part(w, p.host_j) for w in range(4)]
        comp = sb.compressed[p.host_j]
        if comp is not None:
            for w, frame in ((2, comp[0]), (3, comp[1])):
                out = torch.empty(sb.part_bytes, dtype=torch.uint8,
                                  pin_memory=self.arena.pin)
                _zstd.decompress_into(frame, out.numpy())
                parts[w] = out
        return parts

    def _upload_planes(self, pages: list[_Page], staging: torch.Tensor, part: int) -> None:
        """H2D the planes of ``pages`` into staging laid out [lo_k | lo_v | hi_k | hi_v]."""
        n = len(pages)
        j = 0
        while j < n:
            p = pages[j]
            sb = p.host
            # extend a run of consecutive pages of the same spill block
            r = 1
            while (j + r < n and pages[j + r].host is sb and pages[j + r].host_j == p.host_j + r
                   and sb.compressed[p.host_j + r] is None and sb.compressed[p.host_j] is None):
                r += 1
            if sb.compressed[p.host_j] is None:
                for w in range(4):
                    src = sb.part(w, p.host_j, r)
                    staging[w * n * part + j * part: w * n * part + (j + r) * part].copy_(
                        src, non_blocking=True)
            else:
                parts = self._host_planes(p)
                for w in range(4):
                    staging[w * n * part + j * part: w * n * part + (j + 1) * part].copy_(
                        parts[w], non_blocking=True)
            j += r

    def _merge_into(self, pool: DevicePagePool, staging: torch.Tensor, n: int, part: int,
                    slots: list[int]) -> None:
        slot_t = torch.tensor(slots, dtype=torch.int32, device=self.device)
        lo_k, lo_v = staging[0:n * part], staging[n * part:2 * n * part]
        hi_k, hi_v = staging[2 * n * part:3 * n * part], staging[3 * n * part:]
        if ops.slot_codec_supported(pool.k):
            ops.byteplane_merge_slots(lo_k, hi_k, pool.k, slot_t)
            ops.byteplane_merge_slots(lo_v, hi_v, pool.v, slot_t)
        else:
            idx = slot_t.long()
            kb = torch.empty((len(slots),) + tuple(pool.k.shape[1:]), dtype=pool.k.dtype,
                             device=self.device)
            vb = torch.empty((len(slots),) + tuple(pool.v.shape[1:]), dtype=pool.v.dtype,
                             device=self.device)
            ops.byteplane_merge(lo_k, hi_k, kb)
            ops.byteplane_merge(lo_v, hi_v, vb)
            pool.k.index_copy_(0, idx, kb)
            pool.v.index_copy_(0, idx, vb)

    def _transient_reload(self, layer: int, pages: list[_Page]):
        """Stage spilled pages in the layer's staging pool on the side stream.

        Returns (staging pool, slots); the side stream holds the work, so the
        caller waits on it before reading the slots.
        """
        B = self._geom[0]
        stage = self._stage_pool(layer)
        t0 = time.perf_counter()
        slots = stage.allocate(B * len(pages))
        part = B * stage.slot_bytes // 2
        copy = self._stream()
        copy.wait_stream(torch.cuda.current_stream())
        for sb in {id(p.host): p.host for p in pages}.values():
            copy.wait_event(sb.ready)
        with torch.cuda.stream(copy):
            staging = torch.empty(4 * len(pages) * part, dtype=torch.uint8, device=self.device)
            self._upload_planes(pages, staging, part)
            self._merge_into(stage, staging, len(pages), part, slots)
        self.stats.reloads += len(pages)
        self.stats.reload_s += time.perf_counter() - t0
        return stage, slots

    def _release_stage(self, layer: int, slots: list[int]) -> None:
        # Later staging writes go through the side stream, which first waits
        # for the main stream (see _transient_reload), so the slots can be
        # recycled as soon as the reading kernels are enqueued.
        self._stage_pools[layer].release(slots)

    def reload(self, pages=None, stream: torch.cuda.Stream | None = None) -> int:
        """Make spilled pages resident again in fresh pool slots; returns the count.

        The copies and merges run on ``stream`` (default: the cache's side
        stream); the current stream waits for them before returning.
        """
        if pages is None:
            pages = [p for layer in self._pages for p in layer if not p.resident]
        pages = [self._pages[p[0]][p[1]] if isinstance(p, tuple) else p for p in pages]
        pages = [p for p in pages if not p.resident]
        if not pages:
            return 0
        t0 = time.perf_counter()
        B = self._geom[0]
        side = stream if stream is not None else self._stream()
        side.wait_stream(torch.cuda.current_stream())
        by_layer: dict[int, list[_Page]] = {}
        for p in pages:
            by_layer.setdefault(p.layer, []).append(p)
        for layer, lp in by_layer.items():
            pool = self._pool(layer)
            slots = pool.allocate(B * len(lp))
            part = B * pool.slot_bytes // 2
            for sb in {id(p.host): p.host for p in lp}.values():
                side.wait_event(sb.ready)
            with torch.cuda.stream(side):
                staging = torch.empty(4 * len(lp) * part, dtype=torch.uint8, device=self.device)
                self._upload_planes(lp, staging, part)
                self._merge_into(pool, staging, len(lp), part, slots)
            for j, p in enumerate(lp):
                p.slots = slots[j * B:(j + 1) * B]
                self._drop_host(p)
            self._set_table_cols(layer, {p.index: p.slots for p in lp})
        torch.cuda.current_stream().wait_stream(side)
        self.stats.reloads += len(pages)
        self.stats.reload_s += time.perf_counter() - t0
        return len(pages)

    def _drop_host(self, p: _Page) -> None:
        sb = p.host
        p.host = None
        p._compressed = False
        sb.live -= 1
        if sb.live == 0:
            sb.ready.synchronize()
            self.arena.free(sb.block)

    def _page_tensors(self, p: _Page):
        B, NKV, D = self._geom
        pool = self._pool(p.layer)
        if p.resident:
            idx = torch.tensor(p.slots, dtype=torch.long, device=self.device)
            return (pool.k.index_select(0, idx),
                    pool.v.index_select(0, idx).transpose(2, 3).contiguous())
        stage, slots = self._transient_reload(p.layer, [p])
        torch.cuda.current_stream().wait_stream(self._stream())
        idx = torch.tensor(slots, dtype=torch.long, device=self.device)
        k = stage.k.index_select(0, idx)
        v = stage.v.index_select(0, idx).transpose(2, 3).contiguous()
        self._release_stage(p.layer, slots)
        return k, v

    # ---- fused decode attention --------------------------------------------

    def attend(self, layer: int, q: torch.Tensor, scale: float | None = None) -> torch.Tensor:
        """Decode attention of q [B, NQ, 1, D] over the layer's pages.

        Replaces kv.update + mx.fast.scaled_dot_product_attention at
        runtime/layer_runner.py:158,179-180 with one paged kernel; spilled
        pages are reloaded on the side stream while the resident pages are
        attended, and the two partial results are merged by log-sum-exp.
        """
        B, NKV, D = self._geom
        S = self._len[layer]
        pool = self._pool(layer)
        if scale is None:
            scale = D ** -0.5
        spilled = [p for p in self._pages[layer] if not p.resident]
        if not spilled:
            ctx = torch.full((B,), S, dtype=torch.int32, device=self.device)
            return ops.paged_gqa_decode(q, pool.k, pool.v, self._tables[layer], ctx, scale=scale)
        PT = self.page_positions
        stage, slots = self._transient_reload(layer, spilled)
        # Resident pages in logical order, the open page last (attention over
        # one query token is order-free; only the partial page must be last).
        host = self._tables_host[layer]
        res_cols = [p.index for p in self._pages[layer] if p.resident]
        open_len = S - len(self._pages[layer]) * PT
        if open_len > 0:
            res_cols.append(len(self._pages[layer]))
        res_ctx = (len(res_cols) - (1 if open_len > 0 else 0)) * PT + max(open_len, 0)
        outs = []
        if res_cols:
            t_res = torch.from_numpy(np.ascontiguousarray(host[:, res_cols])).to(self.device)
            c_res = torch.full((B,), res_ctx, dtype=torch.int32, device=self.device)
            outs.append(ops.paged_gqa_decode(q, pool.k, pool.v, t_res, c_res, scale=scale,
                                             return_lse=True))
        t_sp = torch.tensor(np.asarray(slots, np.int32).reshape(len(spilled), B).T.copy(),
                            device=self.device)
        c_sp = torch.full((B,), len(spilled) * PT, dtype=torch.int32, device=self.device)
        torch.cuda.current_stream().wait_stream(self._stream())
        outs.append(ops.paged_gqa_decode(q, stage.k, stage.v, t_sp, c_sp, scale=scale,
                                         return_lse=True))
        self._release_stage(layer, slots)
        if len(outs) == 1:
            return outs[0][0]
        (o1, l1), (o2, l2) = outs
        return ops.merge_attn_states(o1, l1, o2, l2)[0]
