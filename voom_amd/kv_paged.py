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
  attend_prefill(layer, q) causal attention of a prompt through the same kernel
  append_latent / update_latent / attend_mla
                           the absorbed-MLA latent cache (runtime/glm.py:265-330)
  spill(pages)             byte-plane split on the GPU -> D2H into the arena
  reload(pages)            H2D -> byte-plane merge into fresh pool slots

Where the reference differs by platform:
  * Pages live in one device pool per layer (slot = one sequence's page) and
    are addressed through a per-layer block table, instead of per-layer lists
    of MLX arrays that are concatenated on every call (kv_paged.py:164-181).
  * The first spill tier is pinned host memory (the HBM <-> host boundary
    exists on MI355X; Apple unified memory has none), and a page is stored as
    its low-byte and high-byte planes (formats/packed.py:49-50).  With
    ``compress_spill`` the high plane is zstd level 1 compressed on the host,
    as vpack does; the low plane stays raw.
  * With ``spill_dir`` a spilled page is also written to
    ``spill_dir/kv_l{L}_p{P}.vt`` (vpack framing, voom_amd/page_file.py) and
    ``page.path`` names it, as in the reference; ``host_max_bytes`` then caps
    the host copies, and a page whose host copy was dropped reloads from its
    file.  ``release()`` deletes the files.
  * Budget accounting, page closing and the eviction order are the
    reference's (kv_paged.py:143-162, 187-194, 216-240).
"""

from __future__ import annotations

import os
import threading
import time
from collections import OrderedDict, deque
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import ops
from . import page_file
from . import zstd as _zstd
from .host_arena import HostArena, HostBlock
from .page_pool import DevicePagePool, v_pages_to_tokens


# A high plane is kept zstd-compressed only when it shrinks by at least this
# factor; one that barely compresses is stored raw and costs no decompression
# (the admission rule of runtime/warm_tier.py:56,79-81).
MIN_COMPRESS_RATIO = 1.15


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


class KVIntegrityError(RuntimeError):
    """Spilled bytes did not come back as they left: a page checksum did not
    match on reload, a page file is malformed or truncated, or a compressed
    plane does not decompress to its size."""


class _SpillBlock:
    """Host copy of a batch of pages spilled together from one layer.

    ``parts[t]`` is the byte size of one byte plane of slot tensor t for one
    page (B slots).  The block is a sequence of records of up to ``chunk``
    pages (the staging ring's chunk).  A record of m pages is contiguous and
    laid out as the low planes of every tensor, then the high planes, each
    ``m * parts[t]`` long, page i of the record at ``i * parts[t]`` inside its
    part, then (when ``nsum`` > 0) the pages' checksums as int32 [T, m * B],
    page i's B slots at ``i * B`` of each tensor's row.  A record therefore
    moves in one copy each way, exactly as it sits in a staging buffer, and
    is the unit of voom_spill_record / voom_reload_record.  Records start
    ``rec_stride`` bytes apart (a multiple of 256).  ``ready`` is recorded
    after the block's last record is written, ``last_use`` after the last
    kernel that reads the block.
    """

    __slots__ = ("block", "n_pages", "parts", "chunk", "ready", "rec_ready", "live", "pages",
                 "nsum", "jobs", "last_use", "_where", "ready_at")

    def __init__(self, block: HostBlock, n_pages: int, parts: list[int], chunk: int,
                 nsum: int = 0):
        self.pages: list = []
        self.block = block
        self.n_pages = n_pages
        self.parts = list(parts)
        self.chunk = chunk
        self.nsum = nsum  # checksum words per page (T * B), 0 = none
        self.ready: torch.cuda.Event | None = None  # after the block's last record landed
        self.rec_ready: dict[int, torch.cuda.Event] = {}  # after each record landed
        self.last_use: torch.cuda.Event | None = None  # after the last direct reload from it
        self._where: tuple | None = None  # see where()
        # (stream handle, sequence number) of ``ready``: events of one stream
        # complete in the order they were recorded
        self.ready_at: tuple[int, int] | None = None
        self.live = n_pages
        # host work queued on the spill (compression, page files), per page group
        self.jobs: list[Future] = []

    def wait_jobs(self) -> None:
        """Wait for the block's queued host work and re-raise its first error."""
        jobs, self.jobs = self.jobs, []
        for job in jobs:
            job.result()

    def where(self) -> tuple:
        """(host address, address of its pinned slab, chunk, pages, record
        stride): what the staged upload needs to place this block's pages,
        found once (a block never moves)."""
        if self._where is None:
            view = self.block.view
            self._where = (view.data_ptr(), view.untyped_storage().data_ptr(), self.chunk,
                           self.n_pages, self.rec_stride)
        return self._where

    @property
    def page_bytes(self) -> int:
        return record_page_bytes(self.parts, self.nsum)

    def record_pages(self, r: int) -> int:
        return min(self.chunk, self.n_pages - r * self.chunk)

    @property
    def rec_stride(self) -> int:
        return record_stride(self.chunk, self.page_bytes)

    def record(self, r: int) -> torch.Tensor:
        off = r * self.rec_stride
        return self.block.view[off:off + self.record_pages(r) * self.page_bytes]

    def part(self, which: int, j: int) -> torch.Tensor:
        """Plane ``which`` (low planes 0..T-1, then high planes) of page j."""
        r, i = divmod(j, self.chunk)
        m = self.record_pages(r)
        off = r * self.rec_stride + part_offset(self.parts, m, which) + \
            i * self.parts[which % len(self.parts)]
        return self.block.view[off:off + self.parts[which % len(self.parts)]]

    def sums(self, j: int) -> torch.Tensor:
        """Checksums of page j: int32 [T, B] (a strided view of its record)."""
        r, i = divmod(j, self.chunk)
        m = self.record_pages(r)
        T = len(self.parts)
        B = self.nsum // T
        rec = self.record(r)
        return sums_view(rec, self.parts, m, self.nsum)[:, i * B:(i + 1) * B]


def record_page_bytes(parts: list[int], nsum: int) -> int:
    """Bytes one page takes in a record: both planes of every tensor plus its
    ``nsum`` int32 checksums."""
    return 2 * sum(parts) + 4 * nsum


def record_stride(chunk: int, page_bytes: int) -> int:
    """Distance between the starts of consecutive records of a spill block:
    one full record rounded up to 256 bytes, so every record is aligned for
    the record kernels' 16-byte accesses."""
    return -(-chunk * page_bytes // 256) * 256


def block_bytes(n_pages: int, chunk: int, page_bytes: int) -> int:
    """Host bytes of a spill block of ``n_pages`` pages in records of ``chunk``."""
    full, last = divmod(n_pages, chunk)
    if last == 0:
        full, last = full - 1, chunk
    return full * record_stride(chunk, page_bytes) + last * page_bytes


def sums_view(buf: torch.Tensor, parts: list[int], m: int, nsum: int) -> torch.Tensor:
    """The int32 [T, m * B] checksum block of an m-page record/staging buffer."""
    T = len(parts)
    off = 2 * sum(parts) * m
    return buf[off:off + 4 * nsum * m].view(torch.int32).view(T, (nsum // T) * m)


def part_offset(parts: list[int], m: int, which: int) -> int:
    """Offset of plane ``which`` inside an m-page record/staging buffer."""
    T = len(parts)
    lo = sum(parts[:which % T]) * m
    return lo + (sum(parts) * m if which >= T else 0)


def _planes(buf: torch.Tensor, parts: list[int], m: int, t: int):
    """(low, high) plane views of tensor t inside an m-page record/staging buffer."""
    T = len(parts)
    lo = part_offset(parts, m, t)
    hi = part_offset(parts, m, T + t)
    return buf[lo:lo + m * parts[t]], buf[hi:hi + m * parts[t]]


# A run of consecutive record pages this large or larger is reloaded by the
# record kernel; shorter runs go through the staging ring.  One record-kernel
# launch costs ~30 us however little it moves (measured: 100 one-page runs of
# 256 KiB took 3.25 ms, one 100-page run 0.65 ms); 2 MiB is ~36 us at the
# host link's rate.
_RECORD_RUN_BYTES = 2 << 20


def _record_runs(pages: list) -> list:
    """[block, record, pages] runs of consecutive pages of one host record,
    in the given order (every page must have a host copy)."""
    runs: list = []
    for p in pages:
        sb, j = p.host, p.host_j
        r = j // sb.chunk
        last = runs[-1] if runs else None
        if last is not None and last[0] is sb and last[1] == r and last[2][-1].host_j + 1 == j:
            last[2].append(p)
        else:
            runs.append([sb, r, [p]])
    return runs


def _side_stream_off_queue(device: torch.device, tries: int = 8) -> torch.cuda.Stream:
    """A new stream whose work does not queue behind the current stream's.

    HIP maps a process's streams onto a few hardware queues (four by default),
    so a new stream can share the current stream's queue; its copies then run
    only after every kernel enqueued before them there, and everything the
    current stream enqueues after a copy waits for that copy.  The uploads
    that overlap attention depend on the opposite (measured on config 4: 4.5
    ms per step on a shared queue, 3.8 ms on its own).  Which stream lands
    where depends on how many streams the process made before, so each
    candidate is checked: a marker recorded on it must complete before about
    0.1 ms of fills enqueued earlier on the current stream have finished."""
    if torch.cuda.is_current_stream_capturing():
        return torch.cuda.Stream(device=device)  # no waits while a graph is captured
    main = torch.cuda.current_stream(device)
    scratch = torch.empty(16 << 20, dtype=torch.int32, device=device)
    cand = None
    for _ in range(tries):
        cand = torch.cuda.Stream(device=device)
        start, busy_end, marker = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        start.record(main)
        for _ in range(12):
            scratch.fill_(1)
        busy_end.record(main)
        marker.record(cand)
        marker.synchronize()
        busy_end.synchronize()
        if start.elapsed_time(marker) < 0.5 * start.elapsed_time(busy_end):
            break
    del scratch
    return cand


class _Page:
    """One closed page of one layer: a pool slot per sequence, or a host copy."""

    __slots__ = ("cache", "layer", "index", "_slots", "host", "host_j", "nbytes", "_path",
                 "_compressed")

    def __init__(self, cache: "PagedKVCache", layer: int, index: int, slots: list[int],
                 nbytes: int):
        self.cache = cache
        self.layer = layer
        self.index = index
        self.slots = slots
        self.host: _SpillBlock | None = None
        self.host_j = 0
        self.nbytes = nbytes
        self._path: Path | None = None
        self._compressed = False

    @property
    def slots(self) -> list[int] | None:
        """Pool slots (one per sequence) while resident, None while spilled."""
        return self._slots

    @slots.setter
    def slots(self, value) -> None:
        self._slots = value
        self.cache._mark(self.layer, self.index, value is not None)

    @property
    def resident(self) -> bool:
        return self._slots is not None

    @property
    def path(self) -> Path | None:
        """The page file of a spilled page (spill_dir), once it is written: a
        file still being written in the background is waited for."""
        if self.host is not None and self.host.jobs:
            self.host.wait_jobs()
        return self._path

    def load(self):
        """The page's contents, bit-exact: (K, V) as [B, NKV, page_positions, D],
        or (latent,) as [B, page_positions, latent_dim] for a latent cache."""
        return self.cache._page_tensors(self)


class _StagingRing:
    """Persistent device staging buffers reused round-robin.

    Each buffer carries the event after which it may be overwritten; the
    stream that writes it next waits on that event, so the H2D/D2H copies on
    the side stream and the split/merge kernels on the main stream pipeline
    without host synchronisation or allocator churn.  Buffers are large
    (2 x 256 MiB): every copy and every cross-stream event costs on the order
    of 0.1 ms of engine idle time on MI355X, so fewer, larger transfers keep
    the host link saturated.

    A buffer is *held* from ``acquire`` until ``release`` (or ``abandon``):
    ``next_free`` never returns a held buffer, so an upload that landed ahead
    of its merge keeps its buffer until the merge has been enqueued.
    """

    def __init__(self, device: torch.device, nbuf: int = 2, nbytes: int = 256 << 20):
        self.device = device
        self.nbytes = nbytes
        self.bufs: list[torch.Tensor | None] = [None] * nbuf
        self.free_ev: list[torch.cuda.Event | None] = [None] * nbuf
        self.held: set[int] = set()
        self.i = 0

    def next_free(self) -> int | None:
        """The next buffer in round-robin order that nobody holds, or None."""
        n = len(self.bufs)
        for k in range(n):
            idx = (self.i + k) % n
            if idx not in self.held:
                return idx
        return None

    def acquire(self, writer: torch.cuda.Stream, nbytes: int, idx: int | None = None):
        if idx is None:
            idx = self.next_free()
        if idx is None or idx in self.held:
            raise RuntimeError("staging ring: every buffer is held")
        self.i = (idx + 1) % len(self.bufs)
        self.held.add(idx)
        buf = self.bufs[idx]
        if buf is None or buf.numel() < nbytes:
            if self.free_ev[idx] is not None:
                self.free_ev[idx].synchronize()
            buf = torch.empty(max(nbytes, self.nbytes), dtype=torch.uint8, device=self.device)
            self.bufs[idx] = buf
        elif self.free_ev[idx] is not None:
            writer.wait_event(self.free_ev[idx])
        return idx, buf[:nbytes]

    def release(self, idx: int, last_user: torch.cuda.Stream) -> None:
        ev = torch.cuda.Event()
        ev.record(last_user)
        self.free_ev[idx] = ev
        self.held.discard(idx)

    def abandon(self, idx: int, last_use: torch.cuda.Event) -> None:
        """Give a held buffer back; the next writer waits for ``last_use``."""
        self.free_ev[idx] = last_use
        self.held.discard(idx)


class _PinnedUploads:
    """Small host-to-device index lists through one persistent pinned buffer.

    Allocating pinned memory per list (``pin_memory()``) can stall the host
    for milliseconds; the buffer here is carved round-robin instead, and a
    region is rewritten only after the work that last read it has completed.
    ``upload`` copies a list to the device; ``stage`` leaves it in the pinned
    buffer for a kernel that reads host memory itself, and ``settle`` names
    the event after which the staged regions may be reused.
    """

    def __init__(self, device: torch.device, pin: bool, words: int = 1 << 20):
        self.device = device
        self.pin = pin
        self.buf = torch.empty(words, dtype=torch.int32, pin_memory=pin)
        self.np = self.buf.numpy()
        self.pos = 0
        # regions whose readers may still be running, oldest first: [lo, hi,
        # event or None while staged and not yet settled].  A region still
        # pending from an earlier lap of the ring can sit ahead of the ones a
        # new region overlaps, so every pending region is checked.
        self.inflight: deque = deque()
        self._own: list = []  # (event or None, dedicated buffer) of oversized lists

    def _region(self, arr: np.ndarray) -> tuple[int, int]:
        n = arr.size
        if self.pos + n > self.buf.numel():
            self.pos = 0
        lo, hi = self.pos, self.pos + n
        q = self.inflight
        while q and q[0][2] is not None and q[0][2].query():  # finished readers
            q.popleft()
        keep: deque = deque()
        for region in q:
            if region[0] < hi and region[1] > lo:
                if region[2] is None:
                    raise RuntimeError("pinned list ring: a staged region was never settled")
                region[2].synchronize()  # its reader must be done before the rewrite
            else:
                keep.append(region)
        self.inflight = keep
        self.np[lo:hi] = arr.reshape(-1)
        self.pos = hi
        return lo, hi

    def upload(self, arr: np.ndarray) -> torch.Tensor:
        n = arr.size
        if n > self.buf.numel() // 2:  # rare: a dedicated buffer
            host = torch.from_numpy(arr)
            return (host.pin_memory() if self.pin else host).to(self.device, non_blocking=True)
        lo, hi = self._region(arr)
        dev = torch.empty(arr.shape, dtype=torch.int32, device=self.device)
        dev.view(-1).copy_(self.buf[lo:hi], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.inflight.append([lo, hi, ev])
        return dev

    def stage(self, arr: np.ndarray) -> torch.Tensor:
        """The int32 list in pinned host memory, for a kernel to read; the
        region stays reserved until the event given to the next ``settle``."""
        if arr.size > self.buf.numel() // 2:
            own = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.int32).reshape(-1))
            own = own.pin_memory() if self.pin else own
            self._own.append([None, own])
            return own
        lo, hi = self._region(arr)
        self.inflight.append([lo, hi, None])
        return self.buf[lo:hi]

    def settle(self, ev: torch.cuda.Event) -> None:
        """Every staged region is free once ``ev`` has passed."""
        for region in self.inflight:
            if region[2] is None:
                region[2] = ev
        for entry in self._own:
            if entry[0] is None:
                entry[0] = ev
        self._own = [e for e in self._own if not e[0].query()]


def budget_victims_fast(resident: np.ndarray, lengths, resident_pages: int, page_nbytes: int,
                        current_bytes: int, max_bytes: int) -> tuple[np.ndarray, np.ndarray]:
    """``budget_victims`` for pages of one size, on a resident mask.

    ``resident`` [L, cap] bool (page i of layer l is resident), ``lengths``
    the closed-page count per layer.  Returns (layers, page indices) of the
    victims in the reference's order (oldest page index first, round-robin
    over layers, never the newest ``resident_pages`` of a layer), as many as
    bring ``current_bytes`` within ``max_bytes``.
    """
    if current_bytes <= max_bytes or resident.size == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    need = -(-(current_bytes - max_bytes) // page_nbytes)
    L, cap = resident.shape
    limit = np.asarray(lengths, dtype=np.int64) - resident_pages
    eligible = resident & (np.arange(cap)[None, :] < limit[:, None])
    flat = np.flatnonzero(eligible.T.reshape(-1))[:need]  # page index major, layer minor
    return flat % L, flat // L


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
                 arena: HostArena | None = None, prefetch: bool = True,
                 host_max_bytes: int | None = None, verify_spills: bool = True):
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if page_positions <= 0 or page_positions & (page_positions - 1):
            raise ValueError("page_positions must be a power of two")
        self.num_layers = num_layers
        self.max_bytes = max_bytes
        self.page_positions = page_positions
        self.resident_pages = resident_pages
        self.compress_spill = compress_spill
        # Spilled pages live in the pinned host arena; with spill_dir they are
        # also written to page files, and host_max_bytes bounds the host copies.
        self.spill_dir = Path(spill_dir) if spill_dir is not None else None
        self.host_max_bytes = host_max_bytes
        if host_max_bytes is not None and self.spill_dir is None:
            raise ValueError("host_max_bytes needs a spill_dir to hold the evicted copies")
        if self.spill_dir is not None:
            self.spill_dir.mkdir(parents=True, exist_ok=True)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.initial_slots = initial_slots
        self.arena = arena if arena is not None else HostArena()
        self._own_arena = arena is None
        self._stats = KVStats()
        self._stats_lock = threading.Lock()
        # host work of spills (zstd of the high planes, page files) runs on
        # worker threads: the caller never waits for a D2H copy to land
        self._workers: ThreadPoolExecutor | None = None
        self._zstd_scratch = threading.local()
        self._copy_stream: torch.cuda.Stream | None = None
        self._ring = _StagingRing(self.device)
        self._i32_cache: OrderedDict = OrderedDict()
        self._uploads: _PinnedUploads | None = None
        # attend(layer) starts the upload of the next layer's first spilled
        # chunk, so host-link time overlaps the compute in between
        self.prefetch = prefetch
        self.prefetch_hits = 0
        self._prefetched: dict = {}
        # Spill integrity: every spilled page carries per-slot checksums made
        # by the split kernel; the merge recomputes them and a verify kernel
        # counts mismatches into a sticky device status, which the host reads
        # after reload() and, without blocking, at later calls.
        self.verify_spills = verify_spills
        self._status: torch.Tensor | None = None
        self._status_host: torch.Tensor | None = None
        self._status_ev: torch.cuda.Event | None = None
        self._sum_scratch: torch.Tensor | None = None
        # spill records move between pool slots and the pinned arena through
        # the record kernels (the split writes host memory, the merge reads
        # it); False takes the staging ring and copy-engine path instead
        self.direct_host = True
        # a reload takes the record kernels for runs of consecutive record
        # pages of at least this many bytes, the staging ring for the rest
        self.record_run_bytes = _RECORD_RUN_BYTES
        self._ready_seq = 0  # sequence of spill ready events (see _SpillBlock.ready_at)
        self._ready_done: dict[int, int] = {}  # stream -> newest sequence known complete
        self._pending_frees: list = []  # (event, host block) freed once the event passed
        self._tags: OrderedDict = OrderedDict()  # tag -> (layer, page indices)
        self._next_tag = 1
        self._reset_state()

    # ---- state ------------------------------------------------------------

    def _reset_state(self):
        L = self.num_layers
        self._pages: list[list[_Page]] = [[] for _ in range(L)]
        # slots of allocated pages that are not closed yet (page index -> slots)
        self._open_slots: list[dict[int, list[int]]] = [{} for _ in range(L)]
        self._len = [0] * L
        self._offset = 0
        self._resident_closed = 0  # closed pages held in device slots, all layers
        # _res[layer, i]: closed page i of the layer is resident (the budget
        # scan reads this mask instead of the page objects)
        self._res = np.zeros((L, 64), dtype=bool)
        # host blocks, oldest first (keyed by id: removal and lookup in O(1)
        # however many one-page records a long decode leaves)
        self._spill_blocks: dict[int, _SpillBlock] = {}
        self._pools: list[DevicePagePool | None] = [None] * L
        # one transient staging pool shared by all layers: every transient
        # merge and every read of it is ordered on the main stream
        self._stage: DevicePagePool | None = None
        self._drop_prefetch()
        self._tables: list[torch.Tensor | None] = [None] * L
        self._tables_host: list[np.ndarray | None] = [None] * L
        # ("kv", B, NKV, D) or ("latent", B, latent_dim), fixed by the first write
        self._geom: tuple | None = None

    @property
    def stats(self) -> KVStats:
        """Spill and reload counters (KVStats); compression counters include
        every spill so far (queued host work is waited for)."""
        self._wait_host_work()
        return self._stats

    def _wait_host_work(self) -> None:
        for sb in list(getattr(self, "_spill_blocks", {}).values()):
            if sb.jobs:
                sb.wait_jobs()

    def _mark(self, layer: int, index: int, resident: bool) -> None:
        if index >= self._res.shape[1]:
            grown = np.zeros((self.num_layers, max(2 * self._res.shape[1], index + 1)),
                             dtype=bool)
            grown[:, :self._res.shape[1]] = self._res
            self._res = grown
        self._res[layer, index] = resident

    def _set_geometry(self, geom: tuple, dtype: torch.dtype) -> None:
        if self._geom is None:
            if dtype != torch.bfloat16:
                raise ValueError("PagedKVCache stores bfloat16 pages")
            self._geom = geom
            if self.direct_host and self.arena.pin:
                ops.record_prepare()  # the first spill then pays no kernel setup
        elif self._geom != geom:
            raise ValueError(f"cache geometry changed: {self._geom} -> {geom}")

    def _init_geometry(self, k: torch.Tensor):
        if k.dim() != 4:
            raise ValueError("k/v must be [B, num_kv_heads, L, head_dim]")
        B, NKV, _, D = k.shape
        self._set_geometry(("kv", B, NKV, D), k.dtype)

    def _init_latent(self, lat: torch.Tensor):
        if lat.dim() != 3:
            raise ValueError("latent must be [B, L, latent_dim]")
        B, _, R = lat.shape
        self._set_geometry(("latent", B, R), lat.dtype)

    @property
    def _batch(self) -> int:
        return self._geom[1]

    @property
    def compressed_mla(self) -> bool:
        """True for a latent (absorbed-MLA) cache (the reference's kv.compressed_mla)."""
        return self._geom is not None and self._geom[0] == "latent"

    def _new_pool(self, **kw) -> DevicePagePool:
        if self._geom[0] == "kv":
            _, _, NKV, D = self._geom
            return DevicePagePool.kv(NKV, D, self.page_positions, device=self.device, **kw)
        return DevicePagePool.rows(self.page_positions, self._geom[2], device=self.device, **kw)

    def _pool(self, layer: int) -> DevicePagePool:
        pool = self._pools[layer]
        if pool is None:
            pool = self._new_pool(capacity=self.initial_slots)
            self._pools[layer] = pool
        return pool

    def _stage_pool(self, layer: int) -> DevicePagePool:
        if self._stage is None:
            self._stage = self._new_pool(min_grow=16)
        return self._stage

    def _stream(self) -> torch.cuda.Stream:
        if self._copy_stream is None:
            self._copy_stream = _side_stream_off_queue(self.device)
        return self._copy_stream

    def _dev_i32(self, values, cache: bool = False) -> torch.Tensor:
        """Int32 device tensor through a pinned buffer (asynchronous, no host stall).

        With ``cache`` the tensor is memoised by value: index tensors that
        repeat every decode step (staging-slot tables, the resident page
        table) are uploaded once.
        """
        arr = np.ascontiguousarray(values, dtype=np.int32)
        if cache:
            key = (arr.shape, arr.tobytes())
            hit = self._i32_cache.get(key)
            if hit is not None:
                self._i32_cache.move_to_end(key)
                return hit
        if self._uploads is None:
            self._uploads = _PinnedUploads(self.device, self.arena.pin)
        dev = self._uploads.upload(arr)
        if cache:
            self._i32_cache[key] = dev
            if len(self._i32_cache) > 256:
                self._i32_cache.popitem(last=False)
        return dev

    def _host_i32(self, values) -> torch.Tensor:
        """Int32 list staged in pinned host memory for a kernel that reads it
        there (no upload); call ``_uploads.settle`` with an event recorded
        after that kernel."""
        if self._uploads is None:
            self._uploads = _PinnedUploads(self.device, self.arena.pin)
        return self._uploads.stage(np.ascontiguousarray(values, dtype=np.int32))

    def _token_nbytes(self) -> int:
        """Bytes one token adds to a layer across the batch (K+V, or one latent row)."""
        if self._geom[0] == "kv":
            _, B, NKV, D = self._geom
            return B * NKV * D * 2 * 2
        _, B, R = self._geom
        return B * R * 2

    @property
    def page_nbytes(self) -> int:
        return self._token_nbytes() * self.page_positions

    def _set_table_cols(self, layer: int, cols: dict[int, list[int] | None]) -> None:
        """Set block-table columns (page index -> B slots, or None = not resident)."""
        B = self._batch
        host = self._tables_host[layer]
        need = max(cols) + 1
        if host is None or need > host.shape[1]:
            cap = max(16, need * 2)
            new = np.full((B, cap), -1, dtype=np.int32)
            if host is not None:
                new[:, :host.shape[1]] = host
            self._tables_host[layer] = host = new
            self._fill_cols(host, cols)
            self._tables[layer] = self._dev_i32(host)
            return
        self._fill_cols(host, cols)
        lo, hi = min(cols), max(cols) + 1
        self._tables[layer][:, lo:hi].copy_(self._dev_i32(host[:, lo:hi]))

    @staticmethod
    def _fill_cols(host: np.ndarray, cols: dict) -> None:
        """Write table columns in two vectorised assignments (cleared, set)."""
        cleared = [page for page, slots in cols.items() if slots is None]
        if cleared:
            host[:, cleared] = -1
        filled = [page for page, slots in cols.items() if slots is not None]
        if filled:
            host[:, filled] = np.asarray([cols[page] for page in filled], np.int32).T

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
        tok = self._token_nbytes()
        total = self._resident_closed * self.page_nbytes
        for layer in range(self.num_layers):
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

        def write(pool, pos):
            ops.append_kv(k.contiguous(), v.contiguous(), pool.k, pool.v, self._tables[layer],
                          pos)

        self._append(layer, k.shape[2], write)

    def append_latent(self, layer: int, lat: torch.Tensor) -> None:
        """Write latent rows lat [B, L, latent_dim] ([c_kv | k_rope]) after the
        layer's current tokens: the append of KVCache.update_latent
        (runtime/kv_cache.py:99-105) as a slot write into the latent pool."""
        self._init_latent(lat)

        def write(pool, pos):
            ops.append_rows(lat.contiguous(), pool.lat, self._tables[layer], pos)

        self._append(layer, lat.shape[1], write)

    def _append(self, layer: int, L: int, write) -> None:
        B = self._batch
        pool = self._pool(layer)
        start = self._len[layer]
        end = start + L
        PT = self.page_positions
        new_pages = [p for p in range(-(-start // PT), -(-end // PT))
                     if p not in self._open_slots[layer]]  # reserve() may have opened them
        if len(new_pages):
            slots = pool.allocate(B * len(new_pages))
            cols = {}
            for j, page in enumerate(new_pages):
                cols[page] = slots[j * B:(j + 1) * B]
                self._open_slots[layer][page] = cols[page]
            self._set_table_cols(layer, cols)
        if L:
            write(pool, torch.full((B,), start, dtype=torch.int32, device=self.device))
        self._len[layer] = end
        pages = self._pages[layer]
        while (len(pages) + 1) * PT <= end:
            idx = len(pages)
            pages.append(_Page(self, layer, idx, self._open_slots[layer].pop(idx),
                               self.page_nbytes))
            self._resident_closed += 1
        if layer == self.num_layers - 1:
            self._offset += L
            self._enforce_budget()

    # ---- decode steps that a HIP graph can capture ------------------------------

    def reserve(self, total_len: int) -> None:
        """Open pool slots and block-table entries now for every page up to
        ``total_len`` tokens in every layer, and create the device position
        counters of ``append_at`` / ``attend_at``.

        After it, appends up to ``total_len`` allocate nothing and the pools
        and tables keep their device addresses -- what a captured decode step
        needs.  Nothing may spill meanwhile: raises if the reserved pages do
        not fit ``max_bytes``.
        """
        if self._geom is None:
            raise ValueError("reserve() needs the page geometry: append once first")
        PT = self.page_positions
        B = self._batch
        total_pages = -(-int(total_len) // PT)
        spilled = sum(1 for pages in self._pages for p in pages if not p.resident)
        if spilled:
            # a spilled page's table column is -1; the captured step reads the
            # table as it is, so every page must be resident first
            raise ValueError(f"reserve(): {spilled} pages are spilled; reload() them first")
        if total_pages * self.page_nbytes * self.num_layers > self.max_bytes:
            raise ValueError(f"{total_len} tokens exceed max_bytes={self.max_bytes}; "
                             "reserve() cannot spill")
        for layer in range(self.num_layers):
            first = -(-self._len[layer] // PT)
            pages = [p for p in range(first, total_pages) if p not in self._open_slots[layer]]
            if not pages:
                continue
            slots = self._pool(layer).allocate(B * len(pages))
            cols = {}
            for j, page in enumerate(pages):
                cols[page] = slots[j * B:(j + 1) * B]
                self._open_slots[layer][page] = cols[page]
            self._set_table_cols(layer, cols)
        self._reserved = int(total_len)
        # one [2, B] tensor, so a step advances both counters in one launch
        self._counters_dev = torch.tensor([[self._offset] * B, [self._offset + 1] * B],
                                          dtype=torch.int32, device=self.device)
        self._pos_dev = self._counters_dev[0]
        self._ctx_dev = self._counters_dev[1]

    def append_at(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write one token's k, v [B, NKV, 1, D] at the device position counter
        (no host bookkeeping; ``advance`` does it after the step)."""
        pool = self._pool(layer)
        ops.append_kv(k.contiguous(), v.contiguous(), pool.k, pool.v, self._tables[layer],
                      self._pos_dev)

    def project_append_at(self, layer: int, h: torch.Tensor, w_qkv: torch.Tensor,
                          cos: torch.Tensor, sin: torch.Tensor, num_q_heads: int,
                          **norm) -> torch.Tensor:
        """One token of one sequence: the fused qkv projection of h, its RoPE
        and the K/V write at the device position counter in one launch;
        returns q [1, NQ, 1, D] (``append_at`` with the projection and rotation
        folded in).  ``norm`` (ln_weight, eps, delta, x_out) puts the
        residual-add + RMSNorm of h in front, as in ``ops.qkv_rope_append``."""
        pool = self._pool(layer)
        _, NKV, _, D = pool.k.shape
        return ops.qkv_rope_append(h, w_qkv, cos, sin, pool.k, pool.v, self._tables[layer],
                                   self._pos_dev, num_q_heads, NKV, D, **norm)

    def attend_at(self, layer: int, q: torch.Tensor, scale: float) -> torch.Tensor:
        """Decode attention of q [B, NQ, 1, D] over the device context counter
        (all pages resident, as ``reserve`` guarantees)."""
        pool = self._pool(layer)
        return ops.paged_gqa_decode(q, pool.k, pool.v, self._tables[layer], self._ctx_dev,
                                    scale=scale)

    def step_counters(self) -> None:
        """Advance the device position counters by one token (the end of a
        captured step)."""
        self._counters_dev.add_(1)

    def advance(self, L: int = 1) -> None:
        """Host bookkeeping of ``L`` tokens written by ``append_at`` in every
        layer: lengths, closed pages, the offset."""
        PT = self.page_positions
        end = self._offset + L
        if end > getattr(self, "_reserved", 0):
            raise ValueError(f"advance past the reserved {getattr(self, '_reserved', 0)} tokens")
        for layer in range(self.num_layers):
            self._len[layer] = end
            pages = self._pages[layer]
            while (len(pages) + 1) * PT <= end:
                idx = len(pages)
                pages.append(_Page(self, layer, idx, self._open_slots[layer].pop(idx),
                                   self.page_nbytes))
                self._resident_closed += 1
        self._offset = end

    # ---- rollback ---------------------------------------------------------------

    def layer_lengths(self) -> tuple[int, ...]:
        """Each layer's token count (KVCache.layer_lengths, runtime/kv_cache.py:139-151)."""
        return tuple(self._len)

    def trim(self, length: int) -> None:
        """Roll every layer back to its first ``length`` positions
        (KVCache.trim, runtime/kv_cache.py:107-137); layers already shorter are
        left alone, and an attached ``dsa`` state is trimmed with the cache."""
        if isinstance(length, bool) or not isinstance(length, int) or length < 0:
            raise ValueError("trim length must be a non-negative integer")
        self._trim_to([min(n, length) for n in self._len])
        dsa = getattr(self, "dsa", None)
        if dsa is not None:
            dsa.trim(length)

    def trim_layer_lengths(self, lengths) -> None:
        """Roll each layer back to its own checkpointed length
        (KVCache.trim_layer_lengths, runtime/kv_cache.py:153-179)."""
        targets = tuple(int(n) for n in lengths)
        if len(targets) != self.num_layers or any(n < 0 for n in targets):
            raise ValueError("invalid per-layer KV rollback lengths")
        if any(t > n for t, n in zip(targets, self._len)):
            raise ValueError("cannot grow KV during rollback")
        self._trim_to(list(targets))

    def _trim_to(self, targets: list[int]) -> None:
        """Cut layer l to targets[l] tokens.

        Closed pages past the cut become open pages again: a resident page
        keeps its slots and table column (so a reserved, captured decode
        step still finds them), the page that now holds the last partial
        tokens is reloaded first if it was spilled, and any other spilled
        page past the cut drops its host copy and page file.
        """
        PT = self.page_positions
        self._drop_prefetch()
        for layer, n in enumerate(targets):
            if n >= self._len[layer]:
                continue
            pages = self._pages[layer]
            keep = n // PT  # pages wholly below the cut stay closed
            partial = keep if n % PT else None  # page that holds the last tokens
            cut = pages[keep:]
            again = [p for p in cut if p.index == partial and not p.resident]
            if again:
                self.reload(again)
            del pages[keep:]
            for p in cut:
                if p.resident:
                    self._open_slots[layer][p.index] = p.slots
                    p.slots = None
                    self._resident_closed -= 1
                else:
                    self._drop_host(p)
            self._len[layer] = n
        self._offset = targets[0] if targets else 0
        if getattr(self, "_counters_dev", None) is not None:
            B = self._batch
            self._counters_dev.copy_(torch.tensor(
                [[self._offset] * B, [self._offset + 1] * B], dtype=torch.int32))

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        """Append, then return the layer's full K/V [B, NKV, S, D] (kv_paged.py:143-181).

        Spilled pages are reloaded transiently for this call, as the
        reference does; prefer ``attend`` on the decode path.
        """
        self.append(layer, k, v)
        return self.gather(layer)

    def update_latent(self, layer: int, lat: torch.Tensor) -> torch.Tensor:
        """Append latent rows, then return the layer's latent [B, S, latent_dim]
        (KVCache.update_latent, runtime/kv_cache.py:99-105); prefer
        ``attend_mla`` on the decode path."""
        self.append_latent(layer, lat)
        return self.gather_latent(layer)

    def gather(self, layer: int):
        """Logical K/V [B, NKV, S, D] of a layer, spilled pages reloaded transiently."""
        self._require_kind(layer, "kv")
        S = self._len[layer]
        pool = self._pool(layer)
        k_all, v_all = ops.gather_kv(pool.k, pool.v, self._tables[layer], S)
        PT = self.page_positions

        def place(p, idx, stage):
            k_all[:, :, p.index * PT:(p.index + 1) * PT] = stage.k.index_select(0, idx)
            v_all[:, :, p.index * PT:(p.index + 1) * PT] = \
                v_pages_to_tokens(stage.v.index_select(0, idx))

        self._place_spilled(layer, place)
        return k_all, v_all

    def gather_latent(self, layer: int) -> torch.Tensor:
        """Logical latent [B, S, latent_dim] of a layer, spilled pages reloaded transiently."""
        self._require_kind(layer, "latent")
        S = self._len[layer]
        lat_all = ops.gather_rows(self._pool(layer).lat, self._tables[layer], S)
        PT = self.page_positions

        def place(p, idx, stage):
            lat_all[:, p.index * PT:(p.index + 1) * PT] = stage.lat.index_select(0, idx)

        self._place_spilled(layer, place)
        return lat_all

    def _require_kind(self, layer: int, kind: str) -> None:
        if self._geom is None or self._geom[0] != kind:
            have = "empty" if self._geom is None else self._geom[0]
            raise ValueError(f"layer {layer}: this call needs a {kind} cache, the cache is {have}")

    def _place_spilled(self, layer: int, place) -> None:
        """Stream a layer's spilled pages through staging slots, calling
        ``place(page, slot_index_tensor, stage_pool)`` for each landed page."""
        self.check_integrity(wait=False)
        spilled = [p for p in self._pages[layer] if not p.resident]
        if not spilled:
            return
        stage = self._stage_pool(layer)
        B = self._batch

        def consume(chunk, slots):
            for j, p in enumerate(chunk):
                place(p, self._dev_i32(slots[j * B:(j + 1) * B], cache=True).long(), stage)

        self._stream_in(layer, spilled, stage, consume, transient=True)

    def release(self) -> None:
        """Free device slots and host copies; offset and nbytes return to 0."""
        self._wait_host_work()
        # uploads started ahead still read host copies and write staging buffers
        if self._copy_stream is not None:
            self._copy_stream.synchronize()
        # no kernel may still touch the host copies once they are given back
        # (the spills' events: one host wait per recording stream)
        self._sync_ready(self._spill_blocks.values())
        # a reload stamps one event on every block it read: each once
        for ev in {id(sb.last_use): sb.last_use for sb in self._spill_blocks.values()
                   if sb.last_use is not None}.values():
            ev.synchronize()
        self._reap_frees(wait=True)
        if self._own_arena:
            self.arena.close()
        else:
            seen = set()
            for pages in self._pages:
                for p in pages:
                    if p.host is not None and id(p.host) not in seen:
                        seen.add(id(p.host))
                        self.arena.free(p.host.block)
        paths = {p._path for pages in self._pages for p in pages if p._path is not None}
        self._reset_state()
        for path in paths:
            try:
                path.unlink()
            except FileNotFoundError:
                pass

    # ---- spilling -----------------------------------------------------------

    def _enforce_budget(self) -> None:
        """Spill in the reference's order until resident bytes fit max_bytes
        (kv_paged.py:216-240; every page of a cache has the same size, so the
        order is found on the resident mask by budget_victims_fast)."""
        current = self.nbytes()
        if current <= self.max_bytes:
            return
        layers, idx = budget_victims_fast(self._res, [len(p) for p in self._pages],
                                          self.resident_pages, self.page_nbytes, current,
                                          self.max_bytes)
        if layers.size:
            def groups():  # layer by layer, so the first layer spills while the rest are listed
                for layer in np.unique(layers).tolist():
                    pages = self._pages[layer]
                    yield layer, [pages[i] for i in idx[layers == layer].tolist()]

            self._spill_groups(groups())

    def spill(self, pages=None) -> int:
        """Spill pages (``_Page`` objects or (layer, index) pairs) to the host arena.

        ``None`` applies the budget policy.  Returns the number of pages spilled.
        """
        if pages is None:
            before = self._stats.spills
            self._enforce_budget()
            return self._stats.spills - before
        groups: dict[int, list[_Page]] = {}
        for p in pages:
            if isinstance(p, tuple):
                p = self._pages[p[0]][p[1]]
            if p.resident:
                groups.setdefault(p.layer, []).append(p)
        return self._spill_groups(groups.items())

    def _spill_groups(self, by_layer) -> int:
        """Spill resident pages given as (layer, pages) pairs.  Each layer's
        records are enqueued as soon as the layer is planned, so the first
        transfer starts while later layers are still being listed and planned."""
        t0 = time.perf_counter()
        issue = self._spill_issuer()
        done = []
        for layer, lp in by_layer:
            direct = self._direct_ok(self._pool(layer))
            for item in self._spill_plan(layer, lp):
                if direct:
                    self._spill_record(item)
                else:
                    issue(item)
            done.append((layer, lp))
        issue(None)
        pages = [p for _, lp in done for p in lp]
        for layer, lp in done:
            pool = self._pool(layer)
            pool.release([s for p in lp for s in p.slots])
            for p in lp:
                p.slots = None
            self._resident_closed -= len(lp)
            self._set_table_cols(layer, {p.index: None for p in lp})
        if self.compress_spill or self.spill_dir is not None:
            self._queue_host_work(pages)
        if self.spill_dir is not None:
            self._evict_host()
        self._stats.spills += len(pages)
        self._stats.spill_s += time.perf_counter() - t0
        return len(pages)

    def _plane_parts(self, pool: DevicePagePool) -> list[int]:
        """Bytes of one byte plane of each pool tensor for one page (B slots)."""
        return [self._batch * pool.tensor_slot_bytes(t) // 2 for t in range(len(pool.tensors))]

    def _nsum(self, pool: DevicePagePool) -> int:
        """Checksum words per page (one per slot of each pool tensor), or 0 when
        spills are not verified (verification needs the slot codec kernels)."""
        if not self.verify_spills or not all(ops.slot_codec_supported(t) for t in pool.tensors):
            return 0
        return self._batch * len(pool.tensors)

    def _spill_plan(self, layer: int, pages: list[_Page]):
        """One host block for the layer's pages; returns its chunk work items."""
        pool = self._pool(layer)
        parts = self._plane_parts(pool)
        nsum = self._nsum(pool)
        page_bytes = record_page_bytes(parts, nsum)
        n = len(pages)
        per_chunk = max(1, self._ring.nbytes // page_bytes)
        self._reap_frees(wait=True)
        sb = _SpillBlock(self.arena.alloc(block_bytes(n, per_chunk, page_bytes)), n, parts,
                         per_chunk, nsum)
        sb.pages = list(pages)
        self._spill_blocks[id(sb)] = sb
        for j, p in enumerate(pages):
            p.host = sb
            p.host_j = j
        return [(pool, pages[c0:c0 + per_chunk], sb, c0 // per_chunk)
                for c0 in range(0, n, per_chunk)]

    def _direct_ok(self, pool: DevicePagePool) -> bool:
        """Whether spill records move between this pool and the arena through
        the record kernels (pinned arena, slots of whole 64-byte lines)."""
        return (self.direct_host and self.arena.pin and len(pool.tensors) <= 4
                and all(ops.slot_codec_supported(t) for t in pool.tensors))

    def _spill_record(self, item) -> None:
        """Spill one record with voom_spill_record: the split kernel reads the
        slot list from pinned memory and writes the planes and checksums
        straight into the pinned record, on the current stream (which holds
        the pages' writes), with no staging buffer and no copy."""
        pool, cp, sb, rec = item
        slots = self._host_i32([s for p in cp for s in p.slots])
        ops.spill_record(pool.tensors, slots, sb.record(rec), sums=sb.nsum > 0)
        ev = torch.cuda.Event()
        ev.record()
        self._uploads.settle(ev)
        self._set_ready(sb, rec, ev, torch.cuda.current_stream())

    def _spill_issuer(self):
        """A function taking spill work items (pool, pages, block, record) one
        at a time (None flushes): the byte-plane split of each (main stream,
        ordered after the pages' writes) into a staging buffer, then the D2H
        of the staged record (side stream).

        Items are issued in windows of ring size; within a window every split
        is enqueued before any copy, so copies run back to back even when the
        two streams share a hardware queue.
        """
        main = torch.cuda.current_stream()
        copy = self._stream()
        nbuf = len(self._ring.bufs)
        staged = []

        def flush():
            for idx, buf, sb, rec, ev in staged:
                copy.wait_event(ev)
                with torch.cuda.stream(copy):
                    sb.record(rec).copy_(buf, non_blocking=True)
                self._ring.release(idx, copy)
                ev = torch.cuda.Event()
                ev.record(copy)
                self._set_ready(sb, rec, ev, copy)
            staged.clear()

        def issue(item) -> None:
            if item is None:
                flush()
                return
            pool, cp, sb, rec = item
            m = len(cp)
            slot_t = self._dev_i32([s for p in cp for s in p.slots])
            idx, buf = self._acquire(main, m * sb.page_bytes)
            sums = None
            if sb.nsum:
                sums = sums_view(buf, sb.parts, m, sb.nsum)
                sums.zero_()
            for t, tensor in enumerate(pool.tensors):
                lo, hi = _planes(buf, sb.parts, m, t)
                if ops.slot_codec_supported(tensor):
                    ops.byteplane_split_slots(tensor, slot_t, lo, hi,
                                              sums=None if sums is None else sums[t])
                else:
                    ops.byteplane_split(tensor.index_select(0, slot_t.long()).contiguous(),
                                        lo, hi)
            ev = torch.cuda.Event()
            ev.record(main)
            staged.append((idx, buf, sb, rec, ev))
            if len(staged) == nbuf:
                flush()

        return issue

    # pages per background job: small enough to spread one record over the
    # workers, large enough that a job is milliseconds of zstd
    _HOST_JOB_PAGES = 64

    def _queue_host_work(self, pages: list[_Page]) -> None:
        """Queue the host side of a spill on worker threads: per group of pages
        of one record, wait for that record's D2H copy, zstd level 1 each high
        plane (low planes stay raw, formats/packed.py:49-50) and, with
        spill_dir, write the page files.  Nothing here blocks the caller; the
        raw planes stay in the arena, so reloads never decompress them."""
        if self._workers is None:
            try:
                n = len(os.sched_getaffinity(0))
            except AttributeError:  # pragma: no cover
                n = os.cpu_count() or 1
            self._workers = ThreadPoolExecutor(max_workers=max(1, min(16, n)),
                                               thread_name_prefix="voom-spill")
        groups: dict[tuple, list[_Page]] = {}
        for p in pages:
            groups.setdefault((id(p.host), p.host_j // p.host.chunk), []).append(p)
        for (_, rec), group in groups.items():
            sb = group[0].host
            ev = sb.rec_ready[rec]
            meta = self._tensor_meta(group[0].layer) if self.spill_dir is not None else None
            for g0 in range(0, len(group), self._HOST_JOB_PAGES):
                part = group[g0:g0 + self._HOST_JOB_PAGES]
                sb.jobs.append(self._workers.submit(self._host_job, sb, ev, part, meta))

    def _host_job(self, sb: _SpillBlock, landed: torch.cuda.Event, pages: list[_Page],
                  meta) -> None:
        """One background job of _queue_host_work (runs on a worker thread).

        The record is viewed once as a numpy array and each high plane is
        compressed straight from it into a per-thread buffer, so the thread
        holds the GIL only for slicing and bookkeeping, not for copies."""
        while not landed.query():  # sleeping releases the GIL
            time.sleep(50e-6)
        T = len(sb.parts)
        r = pages[0].host_j // sb.chunk
        m = sb.record_pages(r)
        rec = sb.record(r).numpy()
        lo_off = [part_offset(sb.parts, m, t) for t in range(T)]
        hi_off = [part_offset(sb.parts, m, T + t) for t in range(T)]
        scratch = None
        if self.compress_spill:
            local = self._zstd_scratch
            scratch = getattr(local, "buf", None)
            need = _zstd.compress_bound(max(sb.parts))
            if scratch is None or scratch.nbytes < need:
                scratch = local.buf = np.empty(need, dtype=np.uint8)
        raw = comp = 0
        for p in pages:
            i = p.host_j - r * sb.chunk
            his = [rec[hi_off[t] + i * sb.parts[t]:hi_off[t] + (i + 1) * sb.parts[t]]
                   for t in range(T)]
            planes = his
            packed = [False] * T
            if scratch is not None:
                planes = []
                for t in range(T):
                    n = _zstd.compress_into(his[t], scratch, 1)
                    if n * MIN_COMPRESS_RATIO <= sb.parts[t]:
                        comp += n
                        packed[t] = True
                        # only a page file keeps the frame
                        planes.append(scratch[:n].copy() if meta is not None else None)
                    else:
                        # a plane that barely compresses stays raw
                        comp += sb.parts[t]
                        planes.append(his[t])
                comp += sum(sb.parts)  # the raw low planes
                raw += p.nbytes
                p._compressed = True
            if meta is not None:
                los = [rec[lo_off[t] + i * sb.parts[t]:lo_off[t] + (i + 1) * sb.parts[t]]
                       for t in range(T)]
                path = page_file.page_path(self.spill_dir, p.layer, p.index)
                sums = sb.sums(p.host_j).tolist() if sb.nsum else None
                page_file.write(path, p.layer, p.index, meta, los, planes, packed, sums=sums)
                p._path = path
        if raw:
            with self._stats_lock:
                self._stats.spill_bytes_raw += raw
                self._stats.spill_bytes_compressed += comp

    def _tensor_meta(self, layer: int) -> list[dict]:
        """Name, dtype and page shape ([B, ...slot shape]) of each pool tensor."""
        pool = self._pool(layer)
        names = ["k", "v_t"] if self._geom[0] == "kv" else ["latent"]
        return [{"name": n, "dtype": "BF16", "shape": (self._batch,) + shp}
                for n, shp in zip(names, pool.slot_shapes)]

    def _evict_host(self) -> None:
        """Drop host copies, oldest block first, while they exceed host_max_bytes;
        only blocks whose pages all have page files are dropped."""
        if self.host_max_bytes is None:
            return
        for sb in list(self._spill_blocks.values()):
            if self.arena.used_bytes <= self.host_max_bytes:
                break
            sb.wait_jobs()
            live = [p for p in sb.pages if p.host is sb]
            if any(p._path is None for p in live):
                continue
            for p in live:
                p.host = None
            self._release_block(sb)

    def _set_ready(self, sb: _SpillBlock, rec: int, ev: torch.cuda.Event,
                   stream: torch.cuda.Stream) -> None:
        """Record ``ev`` (just recorded on ``stream``) as the moment record
        ``rec`` of ``sb``, and so the block so far, has been written."""
        self._ready_seq += 1
        sb.rec_ready[rec] = ev
        sb.ready = ev
        sb.ready_at = (int(stream.cuda_stream), self._ready_seq)

    @staticmethod
    def _newest_ready(blocks) -> list:
        """(stream, sequence, event) of the ready events that cover ``blocks``:
        per recording stream only the newest, which completes after every
        earlier one of that stream (the streams outlive the spills recorded
        on them)."""
        newest: dict[int, tuple[int, torch.cuda.Event]] = {}
        for sb in blocks:
            if sb.ready is None:
                continue
            st, seq = sb.ready_at
            if st not in newest or seq > newest[st][0]:
                newest[st] = (seq, sb.ready)
        return [(st, seq, ev) for st, (seq, ev) in newest.items()]

    def _wait_ready(self, stream: torch.cuda.Stream, blocks) -> None:
        """Make ``stream`` wait until the spills of ``blocks`` have landed (one
        event wait per recording stream, however many blocks)."""
        for _, _, ev in self._newest_ready(blocks):
            stream.wait_event(ev)

    def _sync_ready(self, blocks) -> None:
        """Wait on the host until the spills of ``blocks`` have landed; events
        known to have completed (a later one of their stream was waited for)
        are not waited for again."""
        for st, seq, ev in self._newest_ready(blocks):
            if self._ready_done.get(st, 0) >= seq:
                continue
            ev.synchronize()
            self._ready_done[st] = seq

    def _release_block(self, sb: _SpillBlock) -> None:
        """Give a spill block's host memory back.  Kernels still reading it
        (a direct reload just enqueued) keep it until they are done: it is
        freed once ``last_use`` has passed (at the next spill or release)."""
        sb.wait_jobs()
        self._sync_ready([sb])
        del self._spill_blocks[id(sb)]
        if sb.last_use is not None and not sb.last_use.query():
            self._pending_frees.append((sb.last_use, sb.block))
        else:
            self.arena.free(sb.block)

    def _reap_frees(self, wait: bool = False) -> None:
        """Free the host blocks whose last reader has finished (all of them,
        waiting, with ``wait``)."""
        keep = []
        for ev, block in self._pending_frees:
            if wait:
                ev.synchronize()
            if wait or ev.query():
                self.arena.free(block)
            else:
                keep.append((ev, block))
        self._pending_frees = keep

    def _file_data(self, p: _Page):
        """Planes (low planes, then high planes) and checksums ([T, B] int32 or
        None) of a page that has no host copy, read from its page file into
        pinned buffers."""
        parts = self._plane_parts(self._pool(p.layer))
        bufs = [torch.empty(n, dtype=torch.uint8, pin_memory=self.arena.pin)
                for n in parts + parts]
        T = len(parts)
        try:
            head = page_file.read(p._path, [b.numpy() for b in bufs[:T]],
                                  [b.numpy() for b in bufs[T:]])
        except (OSError, ValueError, RuntimeError) as exc:
            raise KVIntegrityError(f"layer {p.layer} page {p.index}: {exc}") from exc
        sums = head.get("sums")
        if sums is not None:
            sums = torch.tensor(sums, dtype=torch.int32)
            if self.arena.pin:
                sums = sums.pin_memory()
        return bufs, sums

    def _host_data(self, p: _Page):
        """Pinned host tensors of a spilled page's planes (low planes of every
        pool tensor, then high planes, decompressed when compressed) and its
        checksums ([T, B] int32, or None when it has none)."""
        if p.host is None:
            return self._file_data(p)
        sb = p.host
        T = len(sb.parts)
        planes = [sb.part(w, p.host_j) for w in range(2 * T)]
        return planes, (sb.sums(p.host_j) if sb.nsum else None)

    def _upload_planes(self, pages: list[_Page], staging: torch.Tensor,
                       parts: list[int], nsum: int = 0) -> None:
        """H2D the planes of ``pages`` into staging, laid out as a host record
        (low planes of every tensor, then high planes, page-major inside each,
        then the checksums when ``nsum`` > 0).

        A chunk that is exactly one host record, in order, moves in a single
        copy.  Otherwise the pages go in runs: consecutive pages of one pinned
        slab whose planes (and checksum rows) lie at a constant host stride
        from one page to the next -- consecutive pages of one record (the
        stride is the plane's page size, so each plane of the run is one
        contiguous range), or one-page records spaced evenly in the arena, as
        the budget's spills of one page at a time leave them.  Each plane and
        checksum row of a run moves as one strided transfer
        (``ops.copy_rows``).  Pages outside any run (page files) are
        assembled page by page.
        """
        n = len(pages)
        p0 = pages[0]
        sb = p0.host
        if (sb is not None and sb.nsum == nsum and p0.host_j % sb.chunk == 0
                and n == sb.record_pages(p0.host_j // sb.chunk)
                and all(p.host is sb and p.host_j == p0.host_j + j
                        for j, p in enumerate(pages))):
            staging.copy_(sb.record(p0.host_j // sb.chunk), non_blocking=True)
            return
        T = len(parts)
        B = nsum // T if nsum else 0
        dst = sums_view(staging, parts, n, nsum) if nsum else None
        # Per column c (each plane, then each checksum row) the host address of
        # page q is base(q) + m(q) * at_m[c] + i(q) * width[c]: base = its
        # record's start, m = the record's page count, i = q's place in it.
        width = [parts[w % T] for w in range(2 * T)] + ([4 * B] * T if nsum else [])
        at_m = [part_offset(parts, 1, w) for w in range(2 * T)] + \
            [2 * sum(parts) + 4 * t * B for t in range(T if nsum else 0)]
        K = len(width)
        # per page: block address, slab, chunk, pages, record stride, host_j
        # (zeros and chunk 1 for a page that goes page by page)
        none = (0, 0, 1, 0, 0)
        rows: list[tuple] = []
        okl: list[bool] = []
        parts_l = list(parts)
        for q in pages:
            h = q.host
            e = None
            if h is not None:
                if nsum and not h.nsum:
                    raise KVIntegrityError(f"layer {q.layer} page {q.index}: no checksums "
                                           "were stored with the spilled page")
                if h.parts == parts_l and (not nsum or h.nsum == nsum):
                    e = h.where()
            okl.append(e is not None)
            rows.append((*(e if e is not None else none), q.host_j if e is not None else 0))
        ptr, slab, chunk, npages, stride, hj = np.array(rows, dtype=np.int64).T
        ok = np.array(okl, dtype=bool)
        r = hj // chunk
        i = hj - r * chunk
        m = np.minimum(chunk, npages - r * chunk)
        A = (ptr + r * stride)[:, None] + m[:, None] * np.asarray(at_m, dtype=np.int64)[None, :] \
            + i[:, None] * np.asarray(width, dtype=np.int64)[None, :]
        D = np.diff(A, axis=0)
        # pair (q, q + 1) may share a run: both have host rows in one slab
        pair = (ok[:-1] & ok[1:] & (slab[:-1] == slab[1:])).tolist()
        wide = np.all(D >= np.asarray(width, dtype=np.int64)[None, :], axis=1).tolist()
        same = [False] + np.all(D[1:] == D[:-1], axis=1).tolist()
        rows_at, steps = A.tolist(), D.tolist()

        stream = torch.cuda.current_stream()
        stage0 = staging.data_ptr()
        sums0 = dst.data_ptr() if dst is not None else 0
        j = 0
        while j < n:
            if not okl[j]:
                self._upload_page(pages[j], staging, parts, n, j, dst)
                j += 1
                continue
            k = j + 1
            if k < n and pair[j] and wide[j]:
                k = j + 2
                while k < n and pair[k - 1] and same[k - 1]:
                    k += 1
            run = k - j
            first = rows_at[j]
            pitch = steps[j] if run > 1 else width
            for c in range(K):
                if c < 2 * T:
                    to = stage0 + part_offset(parts, n, c) + j * width[c]
                else:
                    to = sums0 + 4 * ((c - 2 * T) * n * B + j * B)
                ops.copy_rows(to, width[c], first[c], pitch[c], width[c], run, stream=stream)
            j = k

    def _upload_page(self, p: _Page, staging: torch.Tensor, parts: list[int], n: int, j: int,
                     dst: torch.Tensor | None) -> None:
        """Page j of an n-page staging buffer, plane by plane (see _upload_planes)."""
        T = len(parts)
        planes, sums = self._host_data(p)
        for w, plane in enumerate(planes):
            off = part_offset(parts, n, w) + j * parts[w % T]
            staging[off:off + parts[w % T]].copy_(plane, non_blocking=True)
        if dst is not None:
            if sums is None:
                raise KVIntegrityError(f"layer {p.layer} page {p.index}: no checksums "
                                       "were stored with the spilled page")
            B = dst.shape[1] // n
            for t in range(T):
                dst[t, j * B:(j + 1) * B].copy_(sums[t], non_blocking=True)

    def _merge_into(self, pool: DevicePagePool, staging: torch.Tensor, n: int,
                    parts: list[int], slots: list[int], cache: bool = False,
                    tag: int = 0) -> None:
        """Byte-plane merge of an n-page staged record into pool slots; with
        checksums, the merged words are summed and compared with the record's
        sums, mismatches counted into the status under ``tag``."""
        slot_t = self._dev_i32(slots, cache=cache)
        nsum = self._nsum(pool) if tag else 0
        got = None
        if nsum:
            if self._sum_scratch is None or self._sum_scratch.numel() < nsum * n:
                self._sum_scratch = torch.empty(max(nsum * n, 4096), dtype=torch.int32,
                                                device=self.device)
            got = self._sum_scratch[:nsum * n].view(len(pool.tensors), -1)
            got.zero_()
        for t, tensor in enumerate(pool.tensors):
            lo, hi = _planes(staging, parts, n, t)
            if ops.slot_codec_supported(tensor):
                ops.byteplane_merge_slots(lo, hi, tensor, slot_t,
                                          sums=None if got is None else got[t])
            else:
                staged = torch.empty((len(slots),) + tuple(tensor.shape[1:]), dtype=tensor.dtype,
                                     device=self.device)
                ops.byteplane_merge(lo, hi, staged)
                tensor.index_copy_(0, slot_t.long(), staged)

        if got is not None:
            if self._status is None:
                self._status = torch.zeros(2, dtype=torch.int32, device=self.device)
            ops.page_sums_verify(sums_view(staging, parts, n, nsum), got, tag, self._status)

    # ---- spill integrity -------------------------------------------------------

    def _tag(self, layer: int, pages: list[_Page]) -> int:
        """A non-zero tag naming a verified chunk in the status (the last 4096
        are remembered for the error message)."""
        tag = self._next_tag
        self._next_tag = tag % 0x7FFFFFFE + 1
        self._tags[tag] = (layer, [p.index for p in pages])
        if len(self._tags) > 4096:
            self._tags.popitem(last=False)
        return tag

    def _publish_status(self) -> None:
        """Queue a copy of the device status to host memory after the merges."""
        if self._status is None:
            return
        if self._status_host is None:
            self._status_host = torch.zeros(2, dtype=torch.int32, pin_memory=self.arena.pin)
        self._status_host.copy_(self._status, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._status_ev = ev

    def check_integrity(self, wait: bool = True) -> None:
        """Raise KVIntegrityError if a spilled page came back changed.

        Every merge of spilled bytes is checked on the device against the
        checksums the split made.  ``reload()`` and ``load()`` call this and
        wait; attention and gathers poll it without waiting at their next call,
        so a mismatch found during one of them is raised by a later call (or
        here).  The count is cleared when it is raised."""
        ev = self._status_ev
        if ev is None or (not wait and not ev.query()):
            return
        ev.synchronize()
        self._status_ev = None
        bad, tag = (int(v) for v in self._status_host.tolist())
        if bad:
            self._status.zero_()
            where = self._tags.get(tag)
            first = (f"layer {where[0]}, pages {where[1]}" if where is not None
                     else "an earlier reload")
            raise KVIntegrityError(f"{bad} spilled page slot(s) failed their checksum on "
                                   f"reload (first in {first})")

    @staticmethod
    def _chunk_sig(pages: list[_Page]) -> tuple:
        return tuple((id(p.host), p.host_j, p._path) for p in pages)

    def _acquire(self, writer: torch.cuda.Stream, nbytes: int):
        """Next staging buffer nobody holds.  When uploads started ahead hold
        every buffer, the oldest one not yet claimed by a reload is given up
        (the writer then waits for that copy to land)."""
        if self._ring.next_free() is None:
            for layer, (_, (pidx, _buf, ev)) in list(self._prefetched.items()):
                del self._prefetched[layer]
                self._ring.abandon(pidx, ev)
                break
        return self._ring.acquire(writer, nbytes)

    def _drop_prefetch(self) -> None:
        """Forget uploads started ahead; their buffers free once the copy lands."""
        for _, (idx, _buf, ev) in getattr(self, "_prefetched", {}).values():
            self._ring.abandon(idx, ev)
        self._prefetched = {}

    def _take_prefetch(self, layer: int, pages: list[_Page]):
        """(ring idx, buffer, landed event) of an upload of exactly ``pages``
        started ahead for this layer, or None (a stale one is dropped)."""
        hit = self._prefetched.pop(layer, None)
        if hit is None:
            return None
        sig, landed = hit
        if sig == self._chunk_sig(pages):
            self.prefetch_hits += 1
            return landed
        self._ring.abandon(landed[0], landed[2])
        return None

    def _prefetch(self, layer: int) -> None:
        """Start uploading the first chunk of ``layer``'s spilled pages into a
        staging buffer on the side stream; the layer's next transient reload
        (attend, gather, load) merges it instead of uploading again.  Spilled
        pages are immutable while spilled, and any spill or reload in between
        changes the chunk, which discards the upload."""
        if not self.prefetch or layer in self._prefetched or self._geom is None:
            return
        spilled = [p for p in self._pages[layer] if not p.resident]
        if not spilled:
            return
        stage = self._stage_pool(layer)
        parts = self._plane_parts(stage)
        nsum = self._nsum(stage)
        rec = record_page_bytes(parts, nsum)
        per_chunk = max(1, self._ring.nbytes // rec)
        cp = spilled[:per_chunk]
        copy = self._stream()
        self._wait_ready(copy, [p.host for p in cp if p.host is not None])
        idx, buf = self._acquire(copy, len(cp) * rec)
        self._guarded_upload(copy, idx, buf, cp, parts, nsum)
        ev = torch.cuda.Event()
        ev.record(copy)
        self._prefetched[layer] = (self._chunk_sig(cp), (idx, buf, ev))

    def _guarded_upload(self, copy: torch.cuda.Stream, idx: int, buf: torch.Tensor,
                        pages: list[_Page], parts: list[int], nsum: int) -> None:
        """_upload_planes on the side stream; if it raises (a page that cannot
        be read back), the staging buffer is given back before the error
        propagates, after whatever copies were already queued into it."""
        try:
            with torch.cuda.stream(copy):
                self._upload_planes(pages, buf, parts, nsum)
        except BaseException:
            self._ring.release(idx, copy)
            raise

    def _stream_in(self, layer: int, pages: list[_Page], target: DevicePagePool, consume,
                   transient: bool) -> None:
        """Bring spilled pages of one layer into ``target``, chunk by chunk."""
        self._pipeline_in([(layer, pages, target, consume, transient)])

    def _pipeline_in(self, jobs) -> None:
        """Upload spilled pages and merge them into device slots.

        ``jobs``: (layer, pages, target pool, consume(chunk_pages, slots),
        transient).  Each job is cut into staging-ring chunks.  Per window of
        ring size: every H2D copy of the window is enqueued on the side stream
        first, then on the main stream, per chunk, a wait for its copy, the
        byte-plane merge into target slots, and ``consume``.  Copies thus run
        back to back and chunk i is merged and consumed while chunk i+1 is in
        flight.  Transient jobs land in fixed staging slots per ring buffer,
        so the index tensors of a steady decode loop repeat (and stay cached);
        the slots are reused safely because merges and the consumers' reads
        are all on the main stream.
        """
        B = self._batch
        main = torch.cuda.current_stream()
        copy = self._stream()
        nbuf = len(self._ring.bufs)
        t0 = time.perf_counter()
        n_pages = 0
        verified = False
        window: list = []

        def run_window():
            landed = []
            for layer, cp, target, consume, transient, parts, nsum, per_chunk, ahead in window:
                if ahead is not None:
                    landed.append(ahead)
                    continue
                idx, buf = self._acquire(copy, len(cp) * record_page_bytes(parts, nsum))
                try:
                    self._guarded_upload(copy, idx, buf, cp, parts, nsum)
                except KVIntegrityError:
                    for held, _, _ in landed:  # this window's other buffers
                        self._ring.release(held, copy)
                    raise
                ev = torch.cuda.Event()
                ev.record(copy)
                landed.append((idx, buf, ev))
            for (layer, cp, target, consume, transient, parts, nsum, per_chunk, _), \
                    (idx, buf, ev) in zip(window, landed):
                main.wait_event(ev)
                m = len(cp)
                if transient:
                    base = idx * per_chunk * B
                    slots = list(range(base, base + m * B))
                else:
                    slots = target.allocate(B * m)
                self._merge_into(target, buf, m, parts, slots, cache=transient,
                                 tag=self._tag(layer, cp) if nsum else 0)
                self._ring.release(idx, main)
                consume(cp, slots)
            window.clear()

        # chunks are produced job by job and issued a window at a time, so the
        # first copy starts before later jobs are even looked at
        for layer, pages, target, consume, transient in jobs:
            if not transient and self._direct_ok(target):
                # runs of at least record_run_bytes go to the record kernel;
                # shorter ones (pages spilled a few at a time) would each cost
                # a launch that moves too little, and take the staged path,
                # whose strided transfers move any number of them at once
                held = [p for p in pages if p.host is not None]
                page_bytes = held[0].host.page_bytes if held else 0
                direct = [p for _, _, run in _record_runs(held)
                          if len(run) * page_bytes >= self.record_run_bytes for p in run]
                if direct:
                    verified |= self._reload_records(layer, direct, target, consume)
                    n_pages += len(direct)
                    ids = {id(p) for p in direct}
                    pages = [p for p in pages if id(p) not in ids]
                    if not pages:
                        continue
            parts = self._plane_parts(target)
            nsum = self._nsum(target)
            verified |= nsum > 0
            per_chunk = max(1, self._ring.nbytes // record_page_bytes(parts, nsum))
            if transient:
                target.ensure_capacity(nbuf * per_chunk * B)
            self._wait_ready(copy, [p.host for p in pages if p.host is not None])
            for c0 in range(0, len(pages), per_chunk):
                cp = pages[c0:c0 + per_chunk]
                ahead = self._take_prefetch(layer, cp) if transient and c0 == 0 else None
                window.append((layer, cp, target, consume, transient, parts, nsum, per_chunk,
                               ahead))
                if len(window) == nbuf:
                    run_window()
            n_pages += len(pages)
        if window:
            run_window()
        if verified:
            self._publish_status()
        self._stats.reloads += n_pages
        self._stats.reload_s += time.perf_counter() - t0

    def _reload_records(self, layer: int, pages: list[_Page], target: DevicePagePool,
                        consume) -> bool:
        """Merge pages held in the arena back into fresh ``target`` slots with
        voom_reload_record, one launch per run of consecutive pages of one
        record, on the current stream: the kernel reads the pinned record
        itself and checks each slot's checksum.  Returns whether checksums
        were compared."""
        B = self._batch
        nsum = self._nsum(target)
        for p in pages:
            if nsum and not p.host.nsum:
                raise KVIntegrityError(f"layer {p.layer} page {p.index}: no checksums were "
                                       "stored with the spilled page")
        runs = _record_runs(pages)
        main = torch.cuda.current_stream()
        blocks = {id(sb): sb for sb, _, _ in runs}
        self._wait_ready(main, blocks.values())
        if nsum and self._status is None:
            self._status = torch.zeros(2, dtype=torch.int32, device=self.device)
        slots = target.allocate(B * len(pages))
        k = 0
        for sb, r, run in runs:
            mine = slots[k:k + B * len(run)]
            k += len(mine)
            tag = self._tag(layer, run) if nsum else 0
            ops.reload_record(sb.record(r), target.tensors, self._host_i32(mine),
                              rec_slots=sb.record_pages(r) * B,
                              first=(run[0].host_j - r * sb.chunk) * B, tag=tag,
                              status=self._status if tag else None)
            consume(run, mine)
        done = torch.cuda.Event()
        done.record(main)
        self._uploads.settle(done)
        for sb in blocks.values():
            sb.last_use = done
        return nsum > 0

    def reload(self, pages=None, stream: torch.cuda.Stream | None = None) -> int:
        """Make spilled pages resident again in fresh pool slots; returns the count.

        Pages held in the pinned arena are merged by the record kernel, which
        reads host memory itself, on the current stream.  Pages that live only
        in page files are read (and decompressed) on the host, uploaded on the
        cache's side stream (or ``stream``) and merged on the current stream.
        The host waits at the end for the pages' checksums (KVIntegrityError
        when a page came back changed).
        """
        self.check_integrity(wait=False)
        if pages is None:
            # every spilled page, found layer by layer from the resident mask
            # while the first layers' uploads are already running
            def layer_lists():
                for layer, lp in enumerate(self._pages):
                    idx = np.flatnonzero(~self._res[layer, :len(lp)])
                    if idx.size:
                        yield layer, [lp[i] for i in idx.tolist()]
        else:
            by_layer: dict[int, list[_Page]] = {}
            for p in pages:
                if isinstance(p, tuple):
                    p = self._pages[p[0]][p[1]]
                if not p.resident:
                    by_layer.setdefault(p.layer, []).append(p)

            def layer_lists():
                yield from by_layer.items()
        if stream is not None:
            self._copy_stream = stream
        B = self._batch
        done: dict[int, list[_Page]] = {}

        def jobs():
            for layer, lp in layer_lists():
                done[layer] = []

                def adopt(chunk, slots, acc=done[layer]):
                    for j, p in enumerate(chunk):
                        p.slots = slots[j * B:(j + 1) * B]
                        acc.append(p)
                    self._resident_closed += len(chunk)

                yield layer, lp, self._pool(layer), adopt, False

        self._pipeline_in(jobs())
        n = 0
        self._sync_ready({id(p.host): p.host for lp in done.values() for p in lp
                          if p.host is not None}.values())
        for layer, lp in done.items():
            self._set_table_cols(layer, {p.index: p.slots for p in lp})
            for p in lp:
                self._drop_host(p)
            n += len(lp)
        if n:
            self.check_integrity()
        return n

    def _drop_host(self, p: _Page) -> None:
        """Forget the spilled copies of a page that is resident again."""
        sb = p.host
        if sb is not None and sb.jobs:
            sb.wait_jobs()  # its page file may still be being written
        p.host = None
        p._compressed = False
        if p._path is not None:
            try:
                p._path.unlink()
            except FileNotFoundError:
                pass
            p._path = None
        if sb is None:
            return
        sb.live -= 1
        if sb.live == 0 and id(sb) in self._spill_blocks:
            self._release_block(sb)

    def _slot_contents(self, pool: DevicePagePool, idx: torch.Tensor):
        if self._geom[0] == "kv":
            return (pool.k.index_select(0, idx),
                    v_pages_to_tokens(pool.v.index_select(0, idx)).contiguous())
        return (pool.lat.index_select(0, idx),)

    def _page_tensors(self, p: _Page):
        if p.resident:
            return self._slot_contents(self._pool(p.layer), self._dev_i32(p.slots).long())
        stage = self._stage_pool(p.layer)
        out = []

        def grab(chunk, slots):
            out.extend(self._slot_contents(stage, self._dev_i32(slots).long()))

        self._stream_in(p.layer, [p], stage, grab, transient=True)
        self.check_integrity()
        return tuple(out)

    # ---- fused decode attention --------------------------------------------

    def attend(self, layer: int, q: torch.Tensor, scale: float | None = None) -> torch.Tensor:
        """Decode attention of q [B, NQ, 1, D] over the layer's pages.

        Replaces kv.update + mx.fast.scaled_dot_product_attention at
        runtime/layer_runner.py:158,179-180 with the paged kernel.  Spilled
        pages (reloaded for every call, as the reference does) stream in on
        the side stream chunk by chunk while the resident pages are attended;
        each landed chunk is attended in turn and the partial results are
        merged by log-sum-exp, so only the last chunk's attention is exposed
        after the transfer.
        """
        self._require_kind(layer, "kv")
        D = self._geom[3]
        if scale is None:
            scale = D ** -0.5

        def run(pool, table, ctx, lse):
            return ops.paged_gqa_decode(q, pool.k, pool.v, table, ctx, scale=scale,
                                        return_lse=lse)

        return self._attend_pages(layer, run)

    def attend_prefill(self, layer: int, q: torch.Tensor,
                       scale: float | None = None) -> torch.Tensor:
        """Causal attention of the layer's newest L tokens: q [B, NQ, L, D] holds
        the queries of positions S-L .. S-1, whose K/V were just appended.

        The reference masks a multi-token window explicitly (k_pos <= q_pos,
        runtime/layer_runner.py:166-177).  Here every query row becomes its own
        entry of one paged decode call -- the same block-table row, with the
        context cut at its own position + 1 -- so a prompt runs through the
        paged kernel in one launch per 1024 query rows.  Spilled pages of the
        layer are made resident first.
        """
        self._require_kind(layer, "kv")
        B, NQ, L, D = q.shape
        S = self._len[layer]
        if L > S:
            raise ValueError(f"{L} queries but the layer holds {S} tokens")
        if scale is None:
            scale = D ** -0.5
        spilled = [p for p in self._pages[layer] if not p.resident]
        if spilled:
            self.reload(spilled)
        pool = self._pool(layer)
        rows_q = q.permute(0, 2, 1, 3).reshape(B * L, NQ, D).contiguous()
        table = self._tables[layer].repeat_interleave(L, dim=0)
        ctx = (torch.arange(S - L + 1, S + 1, dtype=torch.int32, device=self.device)
               .repeat(B))
        out = torch.empty_like(rows_q)
        step = 1024  # rows per launch (the kernel's batch limit)
        for r0 in range(0, B * L, step):
            r1 = min(B * L, r0 + step)
            out[r0:r1] = ops.paged_gqa_decode(rows_q[r0:r1], pool.k, pool.v,
                                              table[r0:r1].contiguous(), ctx[r0:r1].contiguous(),
                                              scale=scale)
        return out.reshape(B, L, NQ, D).permute(0, 2, 1, 3)

    def attend_mla(self, layer: int, q_nope: torch.Tensor, q_rope: torch.Tensor,
                   w_uk, w_uv_t, scale: float,
                   return_weighted_c: bool = False, selection=None):
        """Absorbed-MLA decode over the layer's latent pages (runtime/glm.py:78-202).

        q_nope [B, H, dn], q_rope [B, H, 64] bf16 (one query token); W_UK
        [H, dn, 512] and W_UV^T [H, 512, dv] as from ops.split_kv_b (tensors,
        or ops.HeadWeights packed once, which saves a packing pass per call); ``scale``
        is the reference's (dn + dr) ** -0.5.  q_lat = [q_nope . W_UK | q_rope]
        is contracted with the paged latent in the HIP kernel (resident pages
        first, spilled pages chunk by chunk as they land, LSE-merged), and
        weighted_c . W_UV gives the per-head output [B, H, dv] before o_proj.

        ``selection``: the DSA top-k of this step (runtime/glm.py:280-289) --
        ascending positions [B, k] int32 (or [B, 1, k] as DSAState returns
        them), optionally with their counts as ``(sel, sel_lens)``.  The
        contraction then runs over those rows only, read straight from the
        pages; spilled pages that the selection touches are reloaded first.
        """
        self._require_kind(layer, "latent")
        q_lat = ops.mla_absorb_query(q_nope, q_rope, w_uk)
        if selection is not None:
            wc = self._attend_selected(layer, q_lat, selection, scale)
            out = ops.mla_project_out(wc, w_uv_t)
            return (out, wc) if return_weighted_c else out

        def run(pool, table, ctx, lse):
            return ops.mla_latent_decode(q_lat, pool.lat, table, ctx, scale=scale,
                                         return_lse=lse)

        wc = self._attend_pages(layer, run)
        out = ops.mla_project_out(wc, w_uv_t)
        return (out, wc) if return_weighted_c else out

    def attend_mla_prefill(self, layer: int, q_nope: torch.Tensor, q_rope: torch.Tensor,
                           w_uk, w_uv_t, scale: float, return_weighted_c: bool = False):
        """Causal absorbed-MLA attention of the layer's newest L tokens.

        q_nope [B, H, L, dn] and q_rope [B, H, L, dr] hold the queries of
        positions S-L .. S-1, whose latent rows were just appended: the L > 1
        branch of _mla_absorbed_attention (runtime/glm.py:142-153), where key
        t' is visible to query t iff t' <= offset + t, with the dense path's
        cast points (fp32 scores, bf16 P, bf16 weighted_c; :157-164).  As in
        ``attend_prefill``, every query row becomes its own entry of the paged
        latent kernel -- the same block-table row with the context cut at its
        own position + 1 -- and the absorption products run on the decode
        kernels, 16 rows per launch, so L = 1 gives ``attend_mla``'s bits.
        Spilled pages of the layer are made resident first.  Returns the
        per-head output [B, H, L, dv] (and weighted_c [B, H, L, 512]).
        """
        self._require_kind(layer, "latent")
        if q_nope.dim() != 4 or q_rope.dim() != 4:
            raise ValueError("q_nope [B, H, L, dn] and q_rope [B, H, L, dr]")
        B, H, L, dn = q_nope.shape
        dr = q_rope.shape[-1]
        if tuple(q_rope.shape[:3]) != (B, H, L) or B != self._batch:
            raise ValueError(f"q_rope must be [{self._batch}, {H}, {L}, dr]")
        S = self._len[layer]
        if L > S:
            raise ValueError(f"{L} queries but the layer holds {S} tokens")
        spilled = [p for p in self._pages[layer] if not p.resident]
        if spilled:
            self.reload(spilled)
        pool = self._pool(layer)
        w_uk = ops.pack_head_weights(w_uk)
        w_uv = ops.pack_head_weights(w_uv_t)
        R = B * L
        rows_n = q_nope.permute(0, 2, 1, 3).reshape(R, H, dn).contiguous()
        rows_r = q_rope.permute(0, 2, 1, 3).reshape(R, H, dr).contiguous()
        q_lat = torch.empty((R, H, w_uk.n + dr), dtype=torch.bfloat16, device=self.device)
        for r0 in range(0, R, 16):  # the head products take at most 16 rows
            r1 = min(R, r0 + 16)
            q_lat[r0:r1] = ops.mla_absorb_query(rows_n[r0:r1], rows_r[r0:r1], w_uk)
        table = self._tables[layer].repeat_interleave(L, dim=0)
        ctx = (torch.arange(S - L + 1, S + 1, dtype=torch.int32, device=self.device)
               .repeat(B))
        wc = torch.empty((R, H, w_uk.n), dtype=torch.bfloat16, device=self.device)
        step = 256  # query rows per latent launch (bounds the range partials)
        for r0 in range(0, R, step):
            r1 = min(R, r0 + step)
            wc[r0:r1] = ops.mla_latent_decode(q_lat[r0:r1], pool.lat, table[r0:r1].contiguous(),
                                              ctx[r0:r1].contiguous(), scale=scale)
        out = torch.empty((R, H, w_uv.n), dtype=torch.bfloat16, device=self.device)
        for r0 in range(0, R, 16):
            r1 = min(R, r0 + 16)
            out[r0:r1] = ops.mla_project_out(wc[r0:r1], w_uv)
        out = out.reshape(B, L, H, w_uv.n).permute(0, 2, 1, 3)
        if return_weighted_c:
            return out, wc.reshape(B, L, H, w_uk.n).permute(0, 2, 1, 3)
        return out

    def _attend_selected(self, layer: int, q_lat: torch.Tensor, selection, scale: float):
        if isinstance(selection, tuple):
            sel, sel_lens = selection
        else:
            sel, sel_lens = selection, None
        if sel.dim() == 3:
            sel = sel[:, 0]
        sel = sel.to(device=self.device, dtype=torch.int32).contiguous()
        B, k = sel.shape
        if sel_lens is None:
            sel_lens = torch.full((B,), min(k, self._len[layer]), dtype=torch.int32,
                                  device=self.device)
        else:
            sel_lens = sel_lens.to(device=self.device, dtype=torch.int32).contiguous()
        spilled = {p.index: p for p in self._pages[layer] if not p.resident}
        if spilled:
            # the pages this selection reads must be resident (one host sync,
            # only when the layer has spilled pages)
            used = sel.cpu().numpy()
            counts = sel_lens.cpu().numpy()
            need = set()
            for b in range(B):
                need.update((used[b, :counts[b]] // self.page_positions).tolist())
            pages = [spilled[i] for i in sorted(need) if i in spilled]
            if pages:
                self.reload(pages)
        return ops.mla_sparse_decode(q_lat, self._pool(layer).lat, self._tables[layer], sel,
                                     sel_lens, scale=scale)

    def _attend_pages(self, layer: int, run) -> torch.Tensor:
        """Drive ``run(pool, block_table, ctx_lens, return_lse)`` over a layer:
        one call over the block table when every page is resident, else one
        over the resident pages plus one per landed chunk of spilled pages,
        folded by log-sum-exp merges."""
        B = self._batch
        S = self._len[layer]
        pool = self._pool(layer)
        spilled = [p for p in self._pages[layer] if not p.resident]
        self.check_integrity(wait=False)
        if not spilled:
            ctx = torch.full((B,), S, dtype=torch.int32, device=self.device)
            out = run(pool, self._tables[layer], ctx, False)
            self._prefetch((layer + 1) % self.num_layers)
            return out
        # the first chunk's upload goes first, ahead of the resident attention
        self._prefetch(layer)
        PT = self.page_positions
        # Resident pages, the open page last (attention of one query token is
        # order-free; only a partial page has to be the last one).
        res_cols = [p.index for p in self._pages[layer] if p.resident]
        open_len = S - len(self._pages[layer]) * PT
        if open_len > 0:
            res_cols.append(len(self._pages[layer]))
        res_ctx = (len(res_cols) - (1 if open_len > 0 else 0)) * PT + max(open_len, 0)
        # fp32 running (o, lse): each part's bf16 output is folded in without
        # re-rounding the running sum, so the error does not grow with the
        # number of chunks; one rounding to bf16 at the end
        state: list[torch.Tensor] = []

        def fold(o_l):
            o, lse = o_l
            if not state:
                state.extend((torch.empty(o.shape, dtype=torch.float32, device=o.device),
                              torch.empty(lse.shape, dtype=torch.float32, device=o.device)))
                ops.fold_attn_state(state[0], state[1], o, lse, init=True)
            else:
                ops.fold_attn_state(state[0], state[1], o, lse)

        if res_cols:
            t_res = self._dev_i32(self._tables_host[layer][:, res_cols], cache=True)
            c_res = torch.full((B,), res_ctx, dtype=torch.int32, device=self.device)
            fold(run(pool, t_res, c_res, True))
        stage = self._stage_pool(layer)

        def attend_chunk(chunk, slots):
            m = len(chunk)
            t = self._dev_i32(np.asarray(slots, np.int32).reshape(m, B).T, cache=True)
            c = torch.full((B,), m * PT, dtype=torch.int32, device=self.device)
            fold(run(stage, t, c, True))

        self._stream_in(layer, spilled, stage, attend_chunk, transient=True)
        self._prefetch((layer + 1) % self.num_layers)
        return state[0].to(torch.bfloat16)
