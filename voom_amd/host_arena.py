"""Pinned host memory arena for spilled page planes.

Spilled KV lives in page-locked host memory so that spill (D2H) and reload
(H2D) run as asynchronous copies on a side stream.  Pinned allocations are
slow (page locking), so memory is taken in large slabs up front (``reserve``)
and carved with a first-fit free list; a block is a ``torch.uint8`` view of
its slab.  Slabs are never returned to the system before ``close``.
"""

from __future__ import annotations

import bisect
import weakref
from dataclasses import dataclass

import torch

ALIGN = 256

# every open arena, so that process teardown can release the pinned slabs
# before the runtime's own finalisers run
_LIVE: "weakref.WeakSet[HostArena]" = weakref.WeakSet()


@dataclass
class HostBlock:
    slab: int
    offset: int
    nbytes: int
    view: torch.Tensor  # uint8 pinned view of exactly nbytes


# Slab size: 256 MiB of page planes plus 1 MiB for what rides along with them
# (checksum words, 256-byte record alignment), so that blocks of a power-of-two
# plane size (64 MiB = one config-3 layer's spilled half) pack four to a slab
# instead of three.
SLAB_BYTES = (256 + 1) << 20


class HostArena:
    def __init__(self, slab_bytes: int = SLAB_BYTES, pin: bool | None = None):
        self.slab_bytes = int(slab_bytes)
        # Page-locked whenever a device exists (asynchronous copies need it);
        # plain host memory otherwise, which keeps the allocator testable.
        self.pin = torch.cuda.is_available() if pin is None else bool(pin)
        self._slabs: list[torch.Tensor] = []
        # per slab: sorted list of (offset, size) free extents
        self._free: list[list[tuple[int, int]]] = []
        self.used_bytes = 0
        _LIVE.add(self)

    @property
    def capacity(self) -> int:
        return sum(s.numel() for s in self._slabs)

    def _add_slab(self, nbytes: int) -> int:
        size = max(self.slab_bytes, -(-nbytes // ALIGN) * ALIGN)
        slab = torch.empty(size, dtype=torch.uint8, pin_memory=self.pin)
        self._slabs.append(slab)
        self._free.append([(0, size)])
        return len(self._slabs) - 1

    def reserve(self, nbytes: int, warm: bool = True) -> None:
        """Ensure at least ``nbytes`` of free pinned memory exist, in slabs of
        ``slab_bytes``.  (One slab of the whole amount was tried: a copy into
        the part of a multi-GiB pinned allocation past its first 2 GiB ran at
        a quarter of the link rate on MI355X boxes; 256 MiB slabs do not.)
        With ``warm`` each new slab is read once by the copy engine (see
        _warm), so that the first upload from it runs at the link rate."""
        free = sum(sz for ext in self._free for _, sz in ext)
        while free < nbytes:
            idx = self._add_slab(min(self.slab_bytes, nbytes - free))
            free += self._slabs[idx].numel()
            if warm:
                self._warm(self._slabs[idx])

    def _warm(self, slab: torch.Tensor) -> None:
        """One host-to-device pass of the copy engine over a new pinned slab,
        waited for.  The engine's first read of freshly pinned pages is slow
        (a 210 MB record: 10.9 ms on first read, 3.67 ms on every later one
        from the same memory, even after the GPU has written it again), so
        reserving ahead pays that here rather than in the first reload."""
        if not (self.pin and torch.cuda.is_available()):
            return
        piece = 64 << 20
        scratch = torch.empty(min(piece, slab.numel()), dtype=torch.uint8, device="cuda")
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            for off in range(0, slab.numel(), piece):
                n = min(piece, slab.numel() - off)
                scratch[:n].copy_(slab[off:off + n], non_blocking=True)
        stream.synchronize()

    def alloc(self, nbytes: int) -> HostBlock:
        need = -(-max(int(nbytes), 1) // ALIGN) * ALIGN
        for si, ext in enumerate(self._free):
            for k, (off, sz) in enumerate(ext):
                if sz >= need:
                    if sz == need:
                        ext.pop(k)
                    else:
                        ext[k] = (off + need, sz - need)
                    self.used_bytes += need
                    return HostBlock(si, off, need, self._slabs[si][off:off + int(nbytes)])
        si = self._add_slab(need)
        return self.alloc(nbytes)

    def free(self, block: HostBlock) -> None:
        ext = self._free[block.slab]
        i = bisect.bisect_left(ext, (block.offset, 0))
        ext.insert(i, (block.offset, block.nbytes))
        # coalesce with neighbours
        if i + 1 < len(ext) and ext[i][0] + ext[i][1] == ext[i + 1][0]:
            ext[i] = (ext[i][0], ext[i][1] + ext[i + 1][1])
            ext.pop(i + 1)
        if i > 0 and ext[i - 1][0] + ext[i - 1][1] == ext[i][0]:
            ext[i - 1] = (ext[i - 1][0], ext[i - 1][1] + ext[i][1])
            ext.pop(i)
        self.used_bytes -= block.nbytes

    def close(self) -> None:
        self._slabs.clear()
        self._free.clear()
        self.used_bytes = 0


def close_all() -> None:
    """Close every open arena (process teardown)."""
    for arena in list(_LIVE):
        arena.close()
