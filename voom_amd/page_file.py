"""On-disk page files of the spill tier: ``kv_l{layer}_p{page}.vt``.

The framing is vpack's (formats/packed.py:8-11, 57-59): an 8-byte
little-endian header length, a JSON header, then per tensor its high byte
plane (zstd level 1 when compressed, raw otherwise) followed by its raw low
byte plane.  A page file holds every tensor of one page of one layer (K and
V^T blocks, or the latent rows) in the device page layout, B slots after each
other:

    {"format": "voom-kv-page", "version": 3, "layer": L, "page": P,
     "tensors": [{"name": "k", "dtype": "BF16", "shape": [B, NKV, PT, D],
                  "lo": n, "hi": n, "hi_z": m | null},
                 {"name": "v", "dtype": "BF16", "shape": [B, NKV, PT/VB, D, VB], ...}],
     "sums": [[c_0, ..., c_{B-1}] per tensor] | null}

Version 2 stored V as V^T blocks of VB = min(PT, 32) tokens (version 1 held
one [D, PT] V^T per page); version 3 adds ``sums``, the per-slot checksums the
spill kernel made (int32 values), which the reload verifies on the device.

``hi_z`` is the compressed length of the high plane, or null when it is
stored raw (``hi`` bytes).  Writing goes through a temporary name and an
atomic rename, so a file that exists is complete.
"""

from __future__ import annotations

import json
import os
import struct
from pathlib import Path

import numpy as np

from . import zstd as _zstd

FORMAT = "voom-kv-page"
VERSION = 3


def page_path(spill_dir: Path, layer: int, page: int) -> Path:
    """File name of a spilled page (the reference's kv_l{L}_p{P}, runtime/kv_paged.py:231)."""
    return Path(spill_dir) / f"kv_l{layer}_p{page}.vt"


def write(path: Path, layer: int, page: int, tensors: list[dict],
          lo_planes: list, hi_planes: list, hi_compressed: list[bool],
          sums: list | None = None) -> int:
    """Write one page file; returns its size in bytes.

    ``tensors``: [{"name", "dtype", "shape"}] per tensor; ``lo_planes`` /
    ``hi_planes``: bytes-like planes (a zstd frame where ``hi_compressed``);
    ``sums``: per tensor, the page's per-slot checksums (or None).
    """
    entries = []
    for meta, lo, hi, z in zip(tensors, lo_planes, hi_planes, hi_compressed):
        lo_n = memoryview(lo).nbytes
        hi_n = memoryview(hi).nbytes
        entries.append({"name": meta["name"], "dtype": meta["dtype"],
                        "shape": [int(d) for d in meta["shape"]], "lo": lo_n,
                        "hi": lo_n, "hi_z": hi_n if z else None})
        if not z and hi_n != lo_n:
            raise ValueError("raw byte planes of one tensor must be the same size")
    if sums is not None:
        sums = [[int(c) for c in row] for row in sums]
        if len(sums) != len(entries):
            raise ValueError("one checksum row per tensor")
    head = json.dumps({"format": FORMAT, "version": VERSION, "layer": int(layer),
                       "page": int(page), "tensors": entries, "sums": sums}).encode()
    tmp = path.with_name(path.name + ".tmp")
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(head)))
        f.write(head)
        for lo, hi in zip(lo_planes, hi_planes):
            f.write(memoryview(hi))
            f.write(memoryview(lo))
    os.replace(tmp, path)
    return 8 + len(head) + sum(e["lo"] + (e["hi_z"] or e["hi"]) for e in entries)


def read(path: Path, lo_out: list, hi_out: list) -> dict:
    """Read a page file into preallocated uint8 arrays (one per tensor and
    plane, exact sizes); returns the header.  Raises on a malformed file."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: truncated header length")
        (n,) = struct.unpack("<Q", raw)
        text = f.read(n)
        if len(text) != n:
            raise ValueError(f"{path}: truncated header")
        try:
            head = json.loads(text)
        except ValueError as exc:
            raise ValueError(f"{path}: malformed header: {exc}") from exc
        if head.get("format") != FORMAT or head.get("version") != VERSION:
            raise ValueError(f"{path}: not a {FORMAT} v{VERSION} file")
        ents = head["tensors"]
        if len(ents) != len(lo_out) or len(ents) != len(hi_out):
            raise ValueError(f"{path}: {len(ents)} tensors, expected {len(lo_out)}")
        for e, lo, hi in zip(ents, lo_out, hi_out):
            if e["lo"] != lo.nbytes or e["hi"] != hi.nbytes:
                raise ValueError(f"{path}: plane sizes {e['lo']}/{e['hi']} do not match the page")
            if e["hi_z"] is None:
                _readinto(f, hi, path)
            else:
                frame = np.frombuffer(f.read(e["hi_z"]), dtype=np.uint8)
                if frame.nbytes != e["hi_z"]:
                    raise ValueError(f"{path}: truncated zstd frame ({frame.nbytes} of "
                                     f"{e['hi_z']} bytes)")
                try:
                    _zstd.decompress_into(frame, hi)
                except RuntimeError as exc:
                    raise ValueError(f"{path}: {exc}") from exc
            _readinto(f, lo, path)
        if f.read(1):
            raise ValueError(f"{path}: trailing bytes after the planes")
    return head


def _readinto(f, arr: np.ndarray, path: Path) -> None:
    view = memoryview(arr).cast("B")
    got = f.readinto(view)
    if got != arr.nbytes:
        raise ValueError(f"{path}: truncated plane ({got} of {arr.nbytes} bytes)")
