"""Bench-only calibration probes (libvoom_calibrate.so, include/voom_calibrate.h).

Probe kernels that bench.py times to give floors for the kernels of the
paged-KV library: a plain streaming read, a row gather, and the MLA latent
kernel's data movement.  They are not on the paged-KV path, nothing under
voom_amd imports this module, and the product library does not export them.
No counterpart in the reference.
"""

from __future__ import annotations

import threading
from ctypes import CDLL, c_int, c_size_t, c_void_p

import torch

from . import _lib
from ._build import CALIB_LIB_PATH
from .ops import _ptr, _require, _require_device, _stream

_P = c_void_p
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "voom_stream_read": (c_int, [_P, c_size_t, _P, c_int, _P]),
    "voom_gather_read": (c_int, [_P, _P, c_size_t, c_int, _P, c_int, _P, c_int, _P]),
    "voom_tile_read": (c_int, [_P, c_int, _P, _P, c_int, c_int, c_int, c_int, c_int, _P, _P, _P]),
}

_lock = threading.Lock()
_handle: CDLL | None = None


def lib() -> CDLL:
    """Load (once) the calibration library, after the paged-KV library it links to."""
    global _handle
    if _handle is None:
        with _lock:
            if _handle is None:
                _lib.lib()
                if not CALIB_LIB_PATH.exists():
                    raise _lib.VoomLibraryError(
                        f"{CALIB_LIB_PATH} is not built; run __graft_entry__.build() first")
                h = CDLL(str(CALIB_LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(h, name)
                    fn.restype = res
                    fn.argtypes = args
                _handle = h
    return _handle


def _call(name: str, *args) -> None:
    _lib.check(getattr(lib(), name)(*args), name)


def stream_read(src: torch.Tensor, sink: torch.Tensor, workgroups: int = 512,
                stream: torch.cuda.Stream | None = None) -> None:
    """One launch reading all of ``src`` (device, contiguous, 16-byte multiple):
    the calibration kernel bench.py uses for the single-launch streaming floor.
    ``sink`` is a device int32 tensor of at least ``workgroups`` entries."""
    _require_device(src, sink)
    nbytes = src.numel() * src.element_size()
    _require(sink.dtype == torch.int32 and sink.numel() >= workgroups, "sink too small")
    _call("voom_stream_read", _ptr(src), nbytes, _ptr(sink), int(workgroups), _stream(stream))


def gather_read(base: torch.Tensor, idx: torch.Tensor, sink: torch.Tensor,
                base2: torch.Tensor | None = None, workgroups: int = 512,
                stream: torch.cuda.Stream | None = None) -> None:
    """One launch reading rows ``base[idx[i]]`` (base [rows, ...], each row 1-4
    KiB), and the same rows of ``base2`` (same shape) when given -- the
    calibration kernel for the floor of a page gather."""
    _require_device(base, idx, sink, base2)
    row_bytes = base[0].numel() * base.element_size()
    _require(base2 is None or (base2.shape == base.shape and base2.dtype == base.dtype),
             "base2 must have base's shape and dtype")
    _require(idx.dtype == torch.int32 and idx.dim() == 1, "idx must be 1-D int32")
    _require(sink.dtype == torch.int32 and sink.numel() >= workgroups, "sink too small")
    _call("voom_gather_read", _ptr(base), _ptr(base2), row_bytes, base.shape[0], _ptr(idx),
              idx.numel(), _ptr(sink), int(workgroups), _stream(stream))


def tile_read(pool: torch.Tensor, table: torch.Tensor, ctx: int, ranges: int, groups: int,
              rows: torch.Tensor, sink: torch.Tensor, q: torch.Tensor | None = None,
              stream: torch.cuda.Stream | None = None) -> None:
    """One launch with the data movement of the MLA latent kernel and no
    arithmetic: ``table.shape[0] * ranges * groups`` workgroups stream the
    64-token tiles of ``pool`` ([slots, 64, 576] bf16) for their token range
    (and their 64 rows of ``q`` [B, 64 groups, 576] when given) through LDS
    and write 64 x 512 fp16 of ``rows`` each -- the calibration kernel for the
    floor of the latent contraction's loads."""
    _require_device(pool, table, rows, sink, q)
    _require(pool.dim() == 3 and tuple(pool.shape[1:]) == (64, 576) and pool.dtype == torch.bfloat16,
             "pool must be [slots, 64, 576] bf16")
    _require(table.dtype == torch.int32 and table.dim() == 2, "table must be [B, max_pages] int32")
    batch = table.shape[0]
    grid = batch * ranges * groups
    _require(rows.numel() * rows.element_size() >= grid * 64 * 512 * 2, "rows too small")
    _require(sink.dtype == torch.int32 and sink.numel() >= grid, "sink too small")
    _require(q is None or (q.dtype == torch.bfloat16 and q.numel() >= batch * groups * 64 * 576),
             "q must hold [B, 64 groups, 576] bf16")
    _call("voom_tile_read", _ptr(pool), pool.shape[0], _ptr(table), _ptr(q), batch,
              table.shape[1], int(ctx), int(ranges), int(groups), _ptr(rows), _ptr(sink),
              _stream(stream))


