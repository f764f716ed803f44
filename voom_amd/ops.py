"""Torch-facing wrappers over the libvoom_hip.so C ABI.

Every function validates shapes/dtypes/devices on the host, passes raw device
pointers plus the current HIP stream, and raises on any non-zero return.  There
is no CPU path: tensors must live on a ROCm device and the library must be
built.

Pool layouts (per layer):
  k_pool  [slots, num_kv_heads, page_tokens, head_dim]  bf16, token-major
  v_pool  [slots, num_kv_heads, page_tokens/VB, head_dim, VB]  bf16, V^T in blocks
          of VB = min(page_tokens, 32) tokens (page_pool.v_slot_shape)
"""

from __future__ import annotations

import ctypes
import os

import torch

from . import _lib
from .page_pool import v_slot_shape

_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


# The current stream's raw handle straight from torch (0.2 us against 2.8 us
# through torch.cuda.current_stream(), called for every launch); the public
# route where this torch build does not expose it.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_CUR_DEVICE = getattr(torch._C, "_cuda_getDevice", None)


def _stream(stream: torch.cuda.Stream | None) -> int:
    if stream is not None:
        return int(stream.cuda_stream)
    if _RAW_STREAM is not None and _CUR_DEVICE is not None:
        return int(_RAW_STREAM(_CUR_DEVICE()))
    return int(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        _require(t.is_cuda, "voom_amd ops need ROCm device tensors (no CPU fallback exists)")
        _require(t.is_contiguous(), "voom_amd ops need contiguous tensors")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


def _side_stream(stream: torch.cuda.Stream | None) -> torch.cuda.Stream | None:
    """``stream`` when it is not the current stream (work enqueued there reads
    tensors the current stream made), else None."""
    if stream is None or stream == torch.cuda.current_stream():
        return None
    return stream


def _used_on(stream: torch.cuda.Stream | None, *tensors: torch.Tensor | None) -> None:
    """Tensors allocated on the current stream but read or written by work on a
    side stream: the caching allocator must not hand their memory out again
    before that work has run (record_stream)."""
    if stream is None:
        return
    for t in tensors:
        if t is not None:
            t.record_stream(stream)


def workspace(device: torch.device, nbytes: int, tag: int = 0) -> torch.Tensor:
    """Per-device cached uint8 scratch tensor of at least ``nbytes`` bytes,
    zeroed when it is allocated: the DSA top-k keeps arrival counters in its
    workspace, which must start at zero (each call leaves them zero)."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), tag)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


# ---- debug bounds checks ------------------------------------------------------
# Off by default (each check costs a launch and a host synchronisation).  When
# on, every attention call first counts the slot / page ids and positions its
# kernel would read out of range and raises ValueError instead of attending:
# the kernels themselves read slot 0 for a bad id and clamp a bad position.
_BOUNDS_CHECKS = os.environ.get("VOOM_BOUNDS_CHECK", "") not in ("", "0")


def set_bounds_checks(enabled: bool) -> None:
    """Turn the debug bounds checks of the attention calls on or off (also
    VOOM_BOUNDS_CHECK=1 in the environment)."""
    global _BOUNDS_CHECKS
    _BOUNDS_CHECKS = bool(enabled)


def bounds_checks_enabled() -> bool:
    return _BOUNDS_CHECKS


def check_block_table(block_table: torch.Tensor, ctx_lens: torch.Tensor, num_slots: int,
                      page_tokens: int, *, stream: torch.cuda.Stream | None = None) -> None:
    """Raise ValueError if a slot id inside some sequence's context lies outside
    [0, num_slots) (a spilled column's -1 included) or a context length does
    not fit the table."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("bounds checks synchronise and cannot run under graph capture")
    B, max_pages = block_table.shape
    status = torch.zeros(4, dtype=torch.int32, device=block_table.device)
    _lib.call("voom_check_block_table", _ptr(block_table), _ptr(ctx_lens), _ptr(status), B,
              max_pages, int(page_tokens), int(num_slots), _stream(stream))
    bad = status.cpu().tolist()
    if bad[1]:
        raise ValueError(f"{bad[1]} context lengths lie outside [0, {max_pages * page_tokens}]")
    if bad[0]:
        raise ValueError(f"block table holds {bad[0]} slot ids outside [0, {num_slots}) "
                         "inside the context")


def check_selection(sel: torch.Tensor, sel_lens: torch.Tensor, block_table: torch.Tensor,
                    num_slots: int, page_tokens: int, *,
                    stream: torch.cuda.Stream | None = None) -> None:
    """Raise ValueError if a used selected position lies outside the block
    table, reads a slot id outside [0, num_slots), or a selection count lies
    outside [0, k]."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("bounds checks synchronise and cannot run under graph capture")
    B, k = sel.shape
    max_pages = block_table.shape[1]
    status = torch.zeros(4, dtype=torch.int32, device=sel.device)
    _lib.call("voom_check_selection", _ptr(sel), _ptr(sel_lens), _ptr(block_table),
              _ptr(status), B, k, max_pages, int(page_tokens), int(num_slots), _stream(stream))
    bad = status.cpu().tolist()
    if bad[3]:
        raise ValueError(f"{bad[3]} selection counts lie outside [0, {k}]")
    if bad[2]:
        raise ValueError(f"selection holds {bad[2]} positions outside the block table")
    if bad[0]:
        raise ValueError(f"selection reads {bad[0]} slot ids outside [0, {num_slots})")


def check_position_free_pages(block_table: torch.Tensor, key_positions: torch.Tensor,
                              block_size: int, num_pages: int, max_position: int,
                              *, stream: torch.cuda.Stream | None = None) -> None:
    """Raise ValueError if a key's page id lies outside [0, num_pages) or a key
    position outside the RoPE cache [0, max_position)."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("bounds checks synchronise and cannot run under graph capture")
    TK = key_positions.numel()
    if TK == 0:
        return
    status = torch.zeros(4, dtype=torch.int32, device=key_positions.device)
    _lib.call("voom_check_position_free_pages", _ptr(block_table), _ptr(key_positions),
              _ptr(status), TK, int(block_size), int(num_pages), int(max_position), _stream(stream))
    bad = status.cpu().tolist()
    if bad[0]:
        raise ValueError(f"block table holds {bad[0]} page ids outside [0, {num_pages})")
    if bad[1]:
        raise ValueError(f"{bad[1]} key positions lie outside the RoPE cache [0, {max_position})")


def default_splits() -> int:
    return int(_lib.lib().voom_paged_gqa_default_splits())


def gqa_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                        num_splits: int) -> int:
    return int(_lib.lib().voom_paged_gqa_workspace_bytes(batch, num_q_heads, num_kv_heads,
                                                        head_dim, num_splits))


def _check_v_pool(v_pool, slots, NKV, D, PT):
    want = (slots,) + v_slot_shape(NKV, D, PT)
    _require(tuple(v_pool.shape) == want,
             f"v_pool must be [slots, NKV, PT/VB, D, VB] = {want}, got {tuple(v_pool.shape)}")


def _gqa_plan(q, k_pool, v_pool, block_table, ctx_lens, out, scale, num_splits, ws):
    """Validate a paged GQA decode call; returns (q3, dims tuple, scale, splits, ws, need)."""
    if q.dim() == 4:
        _require(q.shape[2] == 1, "paged_gqa_decode handles one query token per sequence")
        q = q.reshape(q.shape[0], q.shape[1], q.shape[3])
    _require(q.dim() == 3, "q must be [B, NQ, D]")
    dev = _require_device(q, k_pool, v_pool, block_table, ctx_lens, out)
    B, NQ, D = q.shape
    _require(k_pool.dim() == 4, "k_pool must be [slots, NKV, PT, D]")
    slots, NKV, PT, Dk = k_pool.shape
    _require(Dk == D, f"k_pool head_dim {Dk} != q head_dim {D}")
    _check_v_pool(v_pool, slots, NKV, D, PT)
    _require(q.dtype == k_pool.dtype == v_pool.dtype == torch.bfloat16,
             "q and pools must be bfloat16")
    _require(block_table.dtype == torch.int32 and ctx_lens.dtype == torch.int32,
             "block_table and ctx_lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == B,
             "block_table must be [B, max_pages]")
    _require(tuple(ctx_lens.shape) == (B,), "ctx_lens must be [B]")
    _require(NQ % NKV == 0, "num_q_heads must be a multiple of num_kv_heads")
    max_pages = block_table.shape[1]
    if scale is None:
        scale = D ** -0.5
    if num_splits is None:
        # the library's choice: short block tables take the one-launch segment
        # kernel, longer ones split-K over the default number of wavefronts
        num_splits = 0
    need = gqa_workspace_bytes(B, NQ, NKV, D, num_splits)
    if ws is None:
        ws = workspace(dev, need, tag=1)
    _require(ws.numel() * ws.element_size() >= need, "workspace too small")
    return q, (B, NQ, NKV, D, PT, max_pages, slots), float(scale), int(num_splits), ws, need


def paged_gqa_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     block_table: torch.Tensor, ctx_lens: torch.Tensor, *,
                     scale: float | None = None, out: torch.Tensor | None = None,
                     return_lse: bool = False, num_splits: int | None = None,
                     ws: torch.Tensor | None = None,
                     stream: torch.cuda.Stream | None = None):
    """Decode attention of one query token per sequence over paged K/V.

    q [B, NQ, D] (or [B, NQ, 1, D]) bf16; pools as in the module docstring;
    block_table [B, max_pages] int32; ctx_lens [B] int32.  Returns out with q's
    shape (and the fp32 natural-log LSE [B, NQ] when ``return_lse``).
    Mirrors softmax(q.K^T*scale).V over the concatenated pages
    (runtime/kv_paged.py:164-181, runtime/layer_runner.py:179-180).
    """
    q_shape = q.shape
    q, (B, NQ, NKV, D, PT, max_pages, slots), scale, num_splits, ws, need = _gqa_plan(
        q, k_pool, v_pool, block_table, ctx_lens, out, scale, num_splits, ws)
    if _BOUNDS_CHECKS:
        check_block_table(block_table, ctx_lens, slots, PT, stream=stream)
    if out is None:
        out = torch.empty((B, NQ, D), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, NQ), dtype=torch.float32, device=q.device) if return_lse else None
    _lib.call("voom_paged_gqa_decode", _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
              _ptr(ctx_lens), _ptr(out), _ptr(lse), _ptr(ws), need, B, NQ, NKV, D, PT,
              max_pages, slots, scale, num_splits, _stream(stream))
    out = out.reshape(q_shape)
    return (out, lse) if return_lse else out


def paged_gqa_partials(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       block_table: torch.Tensor, ctx_lens: torch.Tensor, *,
                       scale: float | None = None, num_splits: int | None = None,
                       ws: torch.Tensor | None = None,
                       stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """First half of paged_gqa_decode: the page-streaming kernel, leaving the
    partial softmax states in ``ws`` (returned).  Pair with paged_gqa_combine
    using the same geometry, num_splits and workspace."""
    q, (B, NQ, NKV, D, PT, max_pages, slots), scale, num_splits, ws, need = _gqa_plan(
        q, k_pool, v_pool, block_table, ctx_lens, None, scale, num_splits, ws)
    _lib.call("voom_paged_gqa_partials", _ptr(q), _ptr(k_pool), _ptr(v_pool),
              _ptr(block_table), _ptr(ctx_lens), _ptr(ws), need, B, NQ, NKV, D, PT, max_pages,
              slots, scale, num_splits, _stream(stream))
    return ws


def paged_gqa_combine(ctx_lens: torch.Tensor, out: torch.Tensor, ws: torch.Tensor, *,
                      num_kv_heads: int, page_tokens: int, max_pages: int, num_splits: int,
                      lse: torch.Tensor | None = None,
                      stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Second half of paged_gqa_decode: merge the partial states in ``ws`` into
    out [B, NQ, D] bf16 (and lse [B, NQ] fp32 when given)."""
    _require_device(ctx_lens, out, ws, lse)
    B, NQ, D = out.shape
    need = gqa_workspace_bytes(B, NQ, num_kv_heads, D, num_splits)
    _require(ws.numel() * ws.element_size() >= need, "workspace too small")
    _lib.call("voom_paged_gqa_combine", _ptr(ctx_lens), _ptr(out), _ptr(lse), _ptr(ws), need, B,
              NQ, num_kv_heads, D, page_tokens, max_pages, num_splits, _stream(stream))
    return out


def merge_attn_states(o_a: torch.Tensor, lse_a: torch.Tensor, o_b: torch.Tensor,
                      lse_b: torch.Tensor, *, stream: torch.cuda.Stream | None = None):
    """Combine two attention results over disjoint key sets (LSE merge)."""
    dev = _require_device(o_a, lse_a, o_b, lse_b)
    _require(o_a.shape == o_b.shape and o_a.dtype == o_b.dtype == torch.bfloat16,
             "o_a/o_b must be equal-shaped bf16")
    D = o_a.shape[-1]
    rows = o_a.numel() // D
    _require(lse_a.numel() == rows == lse_b.numel(), "lse must have one entry per row")
    _require(lse_a.dtype == lse_b.dtype == torch.float32, "lse must be float32")
    out = torch.empty_like(o_a)
    lse = torch.empty(lse_a.shape, dtype=torch.float32, device=dev)
    _lib.call("voom_merge_attn_states", _ptr(o_a), _ptr(lse_a), _ptr(o_b), _ptr(lse_b),
              _ptr(out), _ptr(lse), rows, D, _stream(stream))
    return out, lse


def fold_attn_state(o_acc: torch.Tensor, lse_acc: torch.Tensor, o_b: torch.Tensor,
                    lse_b: torch.Tensor, *, init: bool = False,
                    stream: torch.cuda.Stream | None = None) -> None:
    """Fold a bf16 result (o_b, lse_b) over a disjoint key set into the fp32
    running state (o_acc, lse_acc) in place (``init`` sets the state to it).

    The running output stays fp32 however many chunks are folded, as the
    reference's online key tiles keep fp32 (max, sum, acc) (runtime/glm.py:165-196).
    """
    _require_device(o_acc, lse_acc, o_b, lse_b)
    _require(o_acc.dtype == torch.float32 and lse_acc.dtype == torch.float32,
             "the running state must be float32")
    _require(o_b.dtype == torch.bfloat16 and lse_b.dtype == torch.float32,
             "o_b must be bf16 and lse_b float32")
    _require(o_acc.numel() == o_b.numel(), "o_acc and o_b sizes differ")
    D = o_b.shape[-1]
    rows = o_b.numel() // D
    _require(lse_acc.numel() == rows == lse_b.numel(), "lse must have one entry per row")
    _lib.call("voom_fold_attn_state", _ptr(o_acc), _ptr(lse_acc), _ptr(o_b), _ptr(lse_b),
              rows, D, int(bool(init)), _stream(stream))


def append_kv(k_new: torch.Tensor, v_new: torch.Tensor, k_pool: torch.Tensor,
              v_pool: torch.Tensor, block_table: torch.Tensor, positions: torch.Tensor, *,
              stream: torch.cuda.Stream | None = None) -> None:
    """Write k_new/v_new [B, NKV, L, D] at logical positions positions[b] + t."""
    _require_device(k_new, v_new, k_pool, v_pool, block_table, positions)
    B, NKV, L, D = k_new.shape
    slots, NKVp, PT, Dp = k_pool.shape
    _require(v_new.shape == k_new.shape, "k_new and v_new shapes differ")
    _require(NKVp == NKV and Dp == D, "pool geometry does not match new K/V")
    _check_v_pool(v_pool, slots, NKV, D, PT)
    _require(k_new.dtype == v_new.dtype == k_pool.dtype == v_pool.dtype == torch.bfloat16,
             "K/V and pools must be bfloat16")
    _require(block_table.dtype == torch.int32 and positions.dtype == torch.int32,
             "block_table and positions must be int32")
    _require(block_table.shape[0] == B and tuple(positions.shape) == (B,),
             "block_table/positions batch mismatch")
    _lib.call("voom_append_kv", _ptr(k_new), _ptr(v_new), _ptr(k_pool), _ptr(v_pool),
              _ptr(block_table), _ptr(positions), B, NKV, L, D, PT, block_table.shape[1],
              slots, _stream(stream))


def gather_kv(k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
              seq_len: int, *, stream: torch.cuda.Stream | None = None):
    """Materialise logical K/V [B, NKV, seq_len, D] from the pools."""
    dev = _require_device(k_pool, v_pool, block_table)
    slots, NKV, PT, D = k_pool.shape
    B = block_table.shape[0]
    _check_v_pool(v_pool, slots, NKV, D, PT)
    _require(block_table.dtype == torch.int32, "block_table must be int32")
    k = torch.empty((B, NKV, seq_len, D), dtype=k_pool.dtype, device=dev)
    v = torch.empty_like(k)
    _lib.call("voom_gather_kv", _ptr(k_pool), _ptr(v_pool), _ptr(block_table), _ptr(k), _ptr(v),
              B, NKV, seq_len, D, PT, block_table.shape[1], slots, _stream(stream))
    return k, v


def _u16_view(t: torch.Tensor) -> torch.Tensor:
    _require(t.element_size() == 2, "byte-plane codec needs a 16-bit dtype")
    return t


def byteplane_split(src: torch.Tensor, lo: torch.Tensor | None = None,
                    hi: torch.Tensor | None = None, *,
                    stream: torch.cuda.Stream | None = None):
    """Split 16-bit elements into (lo, hi) uint8 planes of src.numel() bytes each."""
    _u16_view(src)
    dev = _require_device(src, lo, hi)
    n = src.numel()
    lo = torch.empty(n, dtype=torch.uint8, device=dev) if lo is None else lo
    hi = torch.empty(n, dtype=torch.uint8, device=dev) if hi is None else hi
    _require(lo.numel() >= n and hi.numel() >= n and lo.dtype == hi.dtype == torch.uint8,
             "planes must be uint8 with >= numel bytes")
    _lib.call("voom_byteplane_split", _ptr(src), _ptr(lo), _ptr(hi), n, _stream(stream))
    return lo, hi


def byteplane_merge(lo: torch.Tensor, hi: torch.Tensor, out: torch.Tensor, *,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Interleave planes back into the 16-bit tensor ``out`` (bit-exact)."""
    _u16_view(out)
    _require_device(lo, hi, out)
    n = out.numel()
    _require(lo.numel() >= n and hi.numel() >= n and lo.dtype == hi.dtype == torch.uint8,
             "planes must be uint8 with >= numel bytes")
    _lib.call("voom_byteplane_merge", _ptr(lo), _ptr(hi), _ptr(out), n, _stream(stream))
    return out


def byteplane_split_slots(pool: torch.Tensor, slots: torch.Tensor, lo: torch.Tensor,
                          hi: torch.Tensor, *, sums: torch.Tensor | None = None,
                          stream: torch.cuda.Stream | None = None) -> None:
    """Gather pool[slots[i]] and split it into plane chunk i (slot_bytes/2 bytes each).

    ``sums`` (int32 [n], zeroed by the caller): each listed slot's checksum is
    added in (see voom_byteplane_split_slots)."""
    _u16_view(pool)
    _require_device(pool, slots, lo, hi, sums)
    _require(slots.dtype == torch.int32 and slots.dim() == 1, "slots must be 1-D int32")
    num_slots = pool.shape[0]
    slot_bytes = pool[0].numel() * 2
    n = slots.numel()
    _require(lo.numel() >= n * slot_bytes // 2 and hi.numel() >= n * slot_bytes // 2,
             "plane buffers too small")
    _check_sums(sums, n)
    _lib.call("voom_byteplane_split_slots", _ptr(pool), _ptr(slots), n, slot_bytes, num_slots,
              _ptr(lo), _ptr(hi), _ptr(sums), _stream(stream))


def byteplane_merge_slots(lo: torch.Tensor, hi: torch.Tensor, pool: torch.Tensor,
                          slots: torch.Tensor, *, sums: torch.Tensor | None = None,
                          stream: torch.cuda.Stream | None = None) -> None:
    """Merge plane chunk i back into pool[slots[i]] (scatter, bit-exact); with
    ``sums`` the checksum of each slot's merged words is added into sums[i]."""
    _u16_view(pool)
    _require_device(pool, slots, lo, hi, sums)
    _require(slots.dtype == torch.int32 and slots.dim() == 1, "slots must be 1-D int32")
    num_slots = pool.shape[0]
    slot_bytes = pool[0].numel() * 2
    n = slots.numel()
    _require(lo.numel() >= n * slot_bytes // 2 and hi.numel() >= n * slot_bytes // 2,
             "plane buffers too small")
    _check_sums(sums, n)
    _lib.call("voom_byteplane_merge_slots", _ptr(lo), _ptr(hi), _ptr(pool), _ptr(slots), n,
              slot_bytes, num_slots, _ptr(sums), _stream(stream))


def _check_sums(sums: torch.Tensor | None, n: int) -> None:
    if sums is not None:
        _require(sums.dtype == torch.int32 and sums.numel() >= n,
                 "sums must be int32 with one entry per listed slot")


def page_sums_verify(expected: torch.Tensor, got: torch.Tensor, tag: int,
                     status: torch.Tensor, *, stream: torch.cuda.Stream | None = None) -> None:
    """Count the checksums in ``got`` that differ from ``expected`` into
    status[0] and, for the first mismatch, store ``tag`` in status[1]."""
    _require_device(expected, got, status)
    _require(expected.dtype == got.dtype == status.dtype == torch.int32,
             "checksums and status must be int32")
    _require(expected.numel() == got.numel() and status.numel() >= 2, "checksum sizes differ")
    _require(tag != 0, "tag must be non-zero")
    _lib.call("voom_page_sums_verify", _ptr(expected), _ptr(got), expected.numel(), int(tag),
              _ptr(status), _stream(stream))


def copy_rows(dst: int, dst_pitch: int, src: int, src_pitch: int, width: int, rows: int, *,
              stream: torch.cuda.Stream | None = None) -> None:
    """Enqueue one transfer of ``rows`` rows of ``width`` bytes, row r from
    address src + r * src_pitch to dst + r * dst_pitch (``voom_copy_rows``;
    pinned host or device memory on either side).  The addresses are raw
    integers: the caller keeps both ranges alive until the stream has passed
    the copy."""
    _require(width >= 0 and rows >= 0, "width and rows must be non-negative")
    _lib.call("voom_copy_rows", int(dst), int(dst_pitch), int(src), int(src_pitch), int(width),
              int(rows), _stream(stream))


def record_bytes(pools: list[torch.Tensor], rec_slots: int, sums: bool) -> int:
    """Bytes of a spill record of ``rec_slots`` slots of every tensor in
    ``pools``: both byte planes of each slot, plus int32 [T, rec_slots]
    checksums with ``sums``."""
    slot = sum(p[0].numel() * 2 for p in pools)
    return rec_slots * slot + (4 * len(pools) * rec_slots if sums else 0)


def _record_call_args(pools: list[torch.Tensor], slots: torch.Tensor, record: torch.Tensor,
                      rec_slots: int, first: int, sums: bool):
    _require(1 <= len(pools) <= 4, "a record holds 1 to 4 pool tensors")
    for p in pools:
        _u16_view(p)
        _require(slot_codec_supported(p), "pool slots must be whole 64-byte lines")
    _require_device(*pools)
    _require(slots.dtype == torch.int32 and slots.dim() == 1 and slots.is_contiguous(),
             "slots must be 1-D contiguous int32")
    _require(slots.device == pools[0].device or (slots.device.type == "cpu" and slots.is_pinned()),
             "slots must be on the pools' device or in pinned host memory")
    _require(record.dtype == torch.uint8 and record.dim() == 1 and record.is_contiguous(),
             "record must be a contiguous 1-D uint8 tensor")
    _require(record.is_cuda or record.is_pinned(),
             "record must be pinned host memory or device memory")
    _require(0 <= first and first + slots.numel() <= rec_slots,
             "listed slots run past the record")
    _require(record.numel() >= record_bytes(pools, rec_slots, sums), "record too small")
    n = len(pools)
    ptrs = (ctypes.c_void_p * n)(*[p.data_ptr() for p in pools])
    sbytes = (ctypes.c_size_t * n)(*[p[0].numel() * 2 for p in pools])
    counts = (ctypes.c_int * n)(*[p.shape[0] for p in pools])
    return ptrs, sbytes, counts


def record_prepare() -> None:
    """Set the spill-record kernels up on the current device ahead of the first
    spill (their one-time launch setup costs about a millisecond each)."""
    _lib.call("voom_record_prepare")


def spill_record(pools: list[torch.Tensor], slots: torch.Tensor, record: torch.Tensor, *,
                 rec_slots: int | None = None, first: int = 0, sums: bool = False,
                 stream: torch.cuda.Stream | None = None) -> None:
    """Byte-plane split of pool slots ``slots`` (of every tensor in ``pools``)
    straight into ``record`` (pinned host memory, or device memory), as record
    slots first .. first + len(slots) - 1, with their checksums when ``sums``.
    ``slots`` may be pinned host memory, read by the kernel itself (keep it
    unchanged until the call has run).  The record layout is the one
    voom_spill_record documents."""
    rec_slots = slots.numel() if rec_slots is None else int(rec_slots)
    ptrs, sbytes, counts = _record_call_args(pools, slots, record, rec_slots, first, sums)
    _lib.call("voom_spill_record", ctypes.cast(ptrs, ctypes.c_void_p), ctypes.addressof(sbytes),
              ctypes.addressof(counts), len(pools), _ptr(slots), slots.numel(), _ptr(record),
              rec_slots, int(first), int(bool(sums)), _stream(stream))


def reload_record(record: torch.Tensor, pools: list[torch.Tensor], slots: torch.Tensor, *,
                  rec_slots: int | None = None, first: int = 0, tag: int = 0,
                  status: torch.Tensor | None = None,
                  stream: torch.cuda.Stream | None = None) -> None:
    """Byte-plane merge of record slots first .. first + len(slots) - 1 back
    into pool slots ``slots``.  ``tag`` != 0 compares every merged slot with the
    record's checksum and counts mismatches into ``status`` (device int32 [2],
    as page_sums_verify)."""
    rec_slots = slots.numel() if rec_slots is None else int(rec_slots)
    ptrs, sbytes, counts = _record_call_args(pools, slots, record, rec_slots, first, bool(tag))
    if tag:
        _require(status is not None and status.is_cuda and status.dtype == torch.int32
                 and status.numel() >= 2, "a tag needs a device int32 status of 2 words")
    _lib.call("voom_reload_record", _ptr(record), rec_slots, int(first),
              ctypes.cast(ptrs, ctypes.c_void_p), ctypes.addressof(sbytes),
              ctypes.addressof(counts), len(pools), _ptr(slots), slots.numel(), int(tag),
              _ptr(status) if tag else None, _stream(stream))


def slot_codec_supported(pool: torch.Tensor) -> bool:
    """True when one pool slot is a whole number of 64-byte lines (slot kernels)."""
    slot_elems = 1
    for d in pool.shape[1:]:
        slot_elems *= int(d)
    return (slot_elems * 2) % 64 == 0


def mla_workspace_bytes(batch: int, num_heads: int, num_ranges: int = 0) -> int:
    return int(_lib.lib().voom_mla_workspace_bytes(batch, num_heads, num_ranges))


def mla_latent_decode(q_lat: torch.Tensor, lat_pool: torch.Tensor, block_table: torch.Tensor,
                      ctx_lens: torch.Tensor, *, scale: float, out: torch.Tensor | None = None,
                      return_lse: bool = False, num_ranges: int = 0,
                      ws: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None):
    """Latent contraction of absorbed MLA over a paged latent cache.

    q_lat [B, H, 576] bf16; lat_pool [slots, page_tokens, 576] bf16;
    block_table [B, max_pages] int32; ctx_lens [B] int32.  Returns
    weighted_c [B, H, 512] bf16 (runtime/glm.py:133-164, dense path).
    """
    dev = _require_device(q_lat, lat_pool, block_table, ctx_lens, out)
    _require(q_lat.dim() == 3 and lat_pool.dim() == 3, "q_lat [B,H,576], lat_pool [slots,PT,576]")
    B, H, LD = q_lat.shape
    slots, PT, LD2 = lat_pool.shape
    _require(LD == LD2 == 576, "latent width must be 576 (512 + 64)")
    _require(q_lat.dtype == lat_pool.dtype == torch.bfloat16, "q_lat and lat_pool must be bf16")
    _require(block_table.dtype == torch.int32 and ctx_lens.dtype == torch.int32,
             "block_table and ctx_lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == B and tuple(ctx_lens.shape) == (B,),
             "block_table [B, max_pages], ctx_lens [B]")
    if _BOUNDS_CHECKS:
        check_block_table(block_table, ctx_lens, slots, PT, stream=stream)
    need = mla_workspace_bytes(B, H, num_ranges)
    if ws is None:
        ws = workspace(dev, need, tag=2)
    _require(ws.numel() * ws.element_size() >= need, "workspace too small")
    if out is None:
        out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev) if return_lse else None
    _lib.call("voom_mla_absorbed_decode", _ptr(q_lat), _ptr(lat_pool), _ptr(block_table),
              _ptr(ctx_lens), _ptr(out), _ptr(lse), _ptr(ws), need, B, H, LD, 512, PT,
              block_table.shape[1], slots, float(scale), int(num_ranges), _stream(stream))
    return (out, lse) if return_lse else out


def mla_sparse_decode(q_lat: torch.Tensor, lat_pool: torch.Tensor, block_table: torch.Tensor,
                      sel: torch.Tensor, sel_lens: torch.Tensor, *, scale: float,
                      out: torch.Tensor | None = None, return_lse: bool = False,
                      num_ranges: int = 0, ws: torch.Tensor | None = None,
                      stream: torch.cuda.Stream | None = None):
    """Latent contraction over the DSA-selected positions of each sequence.

    sel [B, k] int32 ascending logical positions, sel_lens [B] int32 (how many
    of each row are used); the rows are read through block_table from the
    pool, the gather of runtime/glm.py:280-289 fused into the contraction.
    Returns weighted_c [B, H, 512] bf16 (and the fp32 LSE with return_lse).
    """
    dev = _require_device(q_lat, lat_pool, block_table, sel, sel_lens, out)
    _require(q_lat.dim() == 3 and lat_pool.dim() == 3, "q_lat [B,H,576], lat_pool [slots,PT,576]")
    B, H, LD = q_lat.shape
    slots, PT, LD2 = lat_pool.shape
    _require(LD == LD2 == 576, "latent width must be 576 (512 + 64)")
    _require(q_lat.dtype == lat_pool.dtype == torch.bfloat16, "q_lat and lat_pool must be bf16")
    _require(block_table.dtype == sel.dtype == sel_lens.dtype == torch.int32,
             "block_table, sel and sel_lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == B and sel.dim() == 2
             and sel.shape[0] == B and tuple(sel_lens.shape) == (B,),
             "block_table [B, max_pages], sel [B, k], sel_lens [B]")
    if _BOUNDS_CHECKS:
        check_selection(sel, sel_lens, block_table, slots, PT, stream=stream)
    need = int(_lib.lib().voom_mla_sparse_workspace_bytes(B, H, sel.shape[1], int(num_ranges)))
    if ws is None:
        ws = workspace(dev, need, tag=2)
    _require(ws.numel() * ws.element_size() >= need, "workspace too small")
    if out is None:
        out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev) if return_lse else None
    _lib.call("voom_mla_sparse_decode", _ptr(q_lat), _ptr(lat_pool), _ptr(block_table),
              _ptr(sel), _ptr(sel_lens), _ptr(out), _ptr(lse), _ptr(ws), need, B, H, LD, 512, PT,
              block_table.shape[1], slots, sel.shape[1], float(scale), int(num_ranges),
              _stream(stream))
    return (out, lse) if return_lse else out


def dsa_index_scores(q_idx: torch.Tensor, w_head: torch.Tensor, k_idx: torch.Tensor,
                     lens: torch.Tensor, *, scale: float, out: torch.Tensor | None = None,
                     stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Lightning-indexer scores of a decode step (runtime/glm_dsa.py:140-150).

    q_idx [B, NH, 128] bf16 (after the indexer RoPE), w_head [B, NH] fp32
    (weights_proj output times NH^-0.5), k_idx [B, cap, 128] bf16, lens [B]
    int32.  Returns scores [B, cap] fp32; entries at or past lens[b] are left
    as they were.
    """
    dev = _require_device(q_idx, w_head, k_idx, lens, out)
    _require(q_idx.dim() == 3 and k_idx.dim() == 3 and w_head.dim() == 2,
             "q_idx [B,NH,D], w_head [B,NH], k_idx [B,cap,D]")
    B, NH, D = q_idx.shape
    _require(k_idx.shape[0] == B and k_idx.shape[2] == D and tuple(w_head.shape) == (B, NH)
             and tuple(lens.shape) == (B,), "inconsistent DSA shapes")
    _require(q_idx.dtype == k_idx.dtype == torch.bfloat16 and w_head.dtype == torch.float32
             and lens.dtype == torch.int32, "q_idx/k_idx bf16, w_head fp32, lens int32")
    cap = k_idx.shape[1]
    if out is None:
        out = torch.empty((B, cap), dtype=torch.float32, device=dev)
    _require(tuple(out.shape) == (B, cap) and out.dtype == torch.float32, "scores [B, cap] fp32")
    _lib.call("voom_dsa_index_scores", _ptr(q_idx), _ptr(w_head), _ptr(k_idx), _ptr(lens),
              _ptr(out), B, NH, D, cap, float(scale), _stream(stream))
    return out


def dsa_topk(scores: torch.Tensor, lens: torch.Tensor, k: int, *,
             sel: torch.Tensor | None = None, sel_lens: torch.Tensor | None = None,
             stream: torch.cuda.Stream | None = None):
    """Top-k of each row's first lens[b] scores as ascending int32 indices
    (runtime/glm_dsa.py:151-160).  Returns (sel [B, k], sel_lens [B]);
    sel_lens[b] = min(lens[b], k), entries past it are unspecified.  sel and
    sel_lens may be given (int32, those shapes) to be written in place."""
    dev = _require_device(scores, lens, sel, sel_lens)
    _require(scores.dim() == 2 and scores.dtype == torch.float32, "scores [B, cap] fp32")
    _require(lens.dtype == torch.int32 and tuple(lens.shape) == (scores.shape[0],), "lens [B] int32")
    _require(int(k) > 0, "k must be positive")
    B, cap = scores.shape
    if sel is None:
        sel = torch.empty((B, int(k)), dtype=torch.int32, device=dev)
    if sel_lens is None:
        sel_lens = torch.empty((B,), dtype=torch.int32, device=dev)
    _require(sel.dtype == sel_lens.dtype == torch.int32 and tuple(sel.shape) == (B, int(k))
             and tuple(sel_lens.shape) == (B,), "sel [B, k] and sel_lens [B] int32")
    need = int(_lib.lib().voom_dsa_topk_workspace_bytes(B, cap))
    ws = workspace(dev, need, tag=4)
    _lib.call("voom_dsa_topk", _ptr(scores), _ptr(lens), _ptr(sel), _ptr(sel_lens), _ptr(ws),
              need, B, cap, int(k), _stream(stream))
    return sel, sel_lens


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                 delta: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Residual add (x += delta, in place, when delta is given) and RMSNorm of
    x [..., hidden] bf16 with HF Llama's cast order; returns the normed rows."""
    dev = _require_device(x, weight, delta, out)
    _require(x.dtype == weight.dtype == torch.bfloat16, "bf16 rows and weight")
    H = x.shape[-1]
    _require(tuple(weight.shape) == (H,), "weight [hidden]")
    _require(delta is None or (delta.shape == x.shape and delta.dtype == x.dtype), "delta like x")
    if out is None:
        out = torch.empty_like(x)
    _lib.call("voom_add_rms_norm", _ptr(x), _ptr(delta), _ptr(weight), _ptr(out),
              x.numel() // H, H, float(eps), _stream(stream))
    return out


def rope_split(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_q_heads: int,
               num_kv_heads: int, head_dim: int, stream: torch.cuda.Stream | None = None):
    """qkv [B, L, (nq + 2 nkv) * hd] -> (q [B, nq, L, hd], k [B, nkv, L, hd],
    v [B, nkv, L, hd]), q and k rotated with cos/sin [L, hd] fp32."""
    dev = _require_device(qkv, cos, sin)
    B, L, W = qkv.shape
    _require(W == (num_q_heads + 2 * num_kv_heads) * head_dim, "qkv width")
    _require(qkv.dtype == torch.bfloat16 and cos.dtype == sin.dtype == torch.float32
             and tuple(cos.shape) == (L, head_dim) == tuple(sin.shape), "bf16 qkv, fp32 [L, hd] tables")
    q = torch.empty((B, num_q_heads, L, head_dim), dtype=qkv.dtype, device=dev)
    k = torch.empty((B, num_kv_heads, L, head_dim), dtype=qkv.dtype, device=dev)
    v = torch.empty_like(k)
    _lib.call("voom_rope_split", _ptr(qkv), _ptr(cos), _ptr(sin), _ptr(q), _ptr(k), _ptr(v),
              B, L, num_q_heads, num_kv_heads, head_dim, _stream(stream))
    return q, k, v


def silu_mul(gate_up: torch.Tensor, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """gate_up [..., 2 I] (gate first) -> bf16(silu(gate)) * up [..., I]."""
    dev = _require_device(gate_up)
    _require(gate_up.dtype == torch.bfloat16 and gate_up.shape[-1] % 2 == 0, "bf16 [..., 2I]")
    inter = gate_up.shape[-1] // 2
    out = torch.empty((*gate_up.shape[:-1], inter), dtype=gate_up.dtype, device=dev)
    _lib.call("voom_silu_mul", _ptr(gate_up), _ptr(out), gate_up.numel() // (2 * inter), inter,
              _stream(stream))
    return out


GEMV_MAX_K = 2048


def _norm_prologue(x: torch.Tensor, ln_weight, delta, x_out):
    """Checks of the optional residual-add + RMSNorm prologue arguments."""
    if ln_weight is None:
        _require(delta is None and x_out is None, "delta and x_out need ln_weight")
        return
    _require(ln_weight.dtype == torch.bfloat16 and tuple(ln_weight.shape) == (x.shape[-1],),
             "ln_weight bf16 [K]")
    for t, name in ((delta, "delta"), (x_out, "x_out")):
        _require(t is None or (t.shape == x.shape and t.dtype == x.dtype and t.is_contiguous()),
                 f"{name} like x")
    _require(x_out is None or (x_out.data_ptr() != x.data_ptr() and
                               (delta is None or x_out.data_ptr() != delta.data_ptr())),
             "x_out must not alias x or delta")


def gemv(x: torch.Tensor, weight: torch.Tensor, *, swiglu: bool = False,
         ln_weight: torch.Tensor | None = None, eps: float = 1e-5,
         delta: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
         stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """One-token projection: x [..., K] holding one row, weight [N, K] bf16 ->
    y [..., N] = x . weight^T (fp32 sums, bf16 out).  swiglu: weight is the
    fused [gate; up] [2I, K] and y [..., I] = bf16(silu(gate)) * up.

    With ln_weight the projection's input is add_rms_norm's output instead:
    v = x + delta (x alone without delta) normed with ln_weight and eps, and
    v is written to x_out (when given; a buffer other than x and delta).
    Bit-identical to add_rms_norm followed by the projection."""
    dev = _require_device(x, weight, ln_weight, delta, x_out)
    _require(x.dtype == weight.dtype == torch.bfloat16, "bf16 x and weight")
    _norm_prologue(x, ln_weight, delta, x_out)
    _require(weight.dim() == 2 and x.shape[-1] == weight.shape[1], "weight [N, K] with K = x's")
    _require(x.numel() == x.shape[-1], "gemv takes one row of activations")
    K = weight.shape[1]
    _require(K % 8 == 0 and K <= GEMV_MAX_K, f"K must be a multiple of 8 up to {GEMV_MAX_K}")
    n = weight.shape[0] // 2 if swiglu else weight.shape[0]
    _require(not swiglu or weight.shape[0] % 2 == 0, "swiglu weight rows must be even")
    y = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=dev)
    _lib.call("voom_add_rms_norm_gemv", _ptr(x), _ptr(delta), _ptr(ln_weight), float(eps),
              _ptr(x_out), _ptr(weight), _ptr(y), n, K, int(swiglu), _stream(stream))
    return y


def lm_head_argmax(x: torch.Tensor, weight: torch.Tensor, token: torch.Tensor, *,
                   token_copy: torch.Tensor | None = None,
                   ln_weight: torch.Tensor | None = None, eps: float = 1e-5,
                   delta: torch.Tensor | None = None,
                   stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Greedy next token of one row: token[0] (int64, and token_copy[0] when
    given) = argmax of the bf16 logits x . weight^T, lowest index among ties,
    as ``gemv(x, weight).argmax()``; with ln_weight (and delta) the final
    residual add + RMSNorm of ``gemv`` comes first.  No logits are stored."""
    dev = _require_device(x, weight, token, token_copy, ln_weight, delta)
    _require(x.dtype == weight.dtype == torch.bfloat16, "bf16 x and weight")
    _require(weight.dim() == 2 and x.shape[-1] == weight.shape[1] and x.numel() == x.shape[-1],
             "one row x [K] and weight [N, K]")
    _norm_prologue(x, ln_weight, delta, None)
    N, K = weight.shape
    _require(K % 8 == 0 and K <= GEMV_MAX_K, f"K must be a multiple of 8 up to {GEMV_MAX_K}")
    for t in (token, token_copy):
        _require(t is None or (t.dtype == torch.int64 and t.numel() >= 1), "int64 token outputs")
    need = 8 * ((N + 15) // 16)
    ws = workspace(dev, need, tag=5)
    _lib.call("voom_lm_head_argmax", _ptr(x), _ptr(delta), _ptr(ln_weight), float(eps),
              _ptr(weight), N, K, _ptr(ws), ws.numel(), _ptr(token), _ptr(token_copy),
              _stream(stream))
    return token


def qkv_rope_append(x: torch.Tensor, w_qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
                    position: torch.Tensor, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    *, ln_weight: torch.Tensor | None = None, eps: float = 1e-5,
                    delta: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """One decode token of one sequence: q [1, nq, 1, hd] of the fused qkv
    projection of x (one row of K), rotated with the fp32 rows cos/sin [1, hd]
    of its position (or, given whole tables [rows, hd], their row position[0]); k, v rotated/written into the pools at position[0]
    (int32 device tensor) through block_table row 0.  Bit-identical to gemv,
    rope_split and append_kv in sequence.  ln_weight, eps, delta, x_out: the
    residual-add + RMSNorm prologue of ``gemv``."""
    dev = _require_device(x, w_qkv, cos, sin, k_pool, v_pool, block_table, position,
                          ln_weight, delta, x_out)
    _norm_prologue(x, ln_weight, delta, x_out)
    nq, nkv, hd = int(num_q_heads), int(num_kv_heads), int(head_dim)
    K = w_qkv.shape[1]
    _require(x.numel() == K == x.shape[-1], "x must be one row of the projection's K")
    _require(w_qkv.shape[0] == (nq + 2 * nkv) * hd, "w_qkv rows must be (nq + 2 nkv) * hd")
    _require(x.dtype == w_qkv.dtype == k_pool.dtype == v_pool.dtype == torch.bfloat16, "bf16")
    _require(cos.dtype == sin.dtype == torch.float32 and cos.shape[-1] == sin.shape[-1] == hd
             and cos.shape == sin.shape, "fp32 cos/sin rows of head_dim")
    # several rows: whole tables indexed by the device position in the kernel
    rope_rows = cos.numel() // hd if cos.numel() > hd else 0
    slots, NKVp, PT, Dp = k_pool.shape
    _require(NKVp == nkv and Dp == hd, "pool geometry does not match the heads")
    _check_v_pool(v_pool, slots, nkv, hd, PT)
    _require(block_table.dtype == position.dtype == torch.int32 and block_table.dim() == 2,
             "int32 block_table [B, max_pages] and position")
    q = torch.empty((1, nq, 1, hd), dtype=x.dtype, device=dev)
    _lib.call("voom_qkv_rope_append", _ptr(w_qkv), _ptr(x), _ptr(delta), _ptr(ln_weight),
              float(eps), _ptr(x_out), _ptr(cos), _ptr(sin), _ptr(q),
              _ptr(k_pool), _ptr(v_pool), _ptr(block_table), _ptr(position), nq, nkv, hd, K, PT,
              block_table.shape[1], slots, rope_rows, _stream(stream))
    return q


def split_kv_b(kv_b: torch.Tensor, num_heads: int, dn: int, dv: int):
    """kv_b_proj weight [H*(dn+dv), C] -> (W_UK [H, dn, C], W_UV^T [H, C, dv]), contiguous.

    The split of runtime/glm.py:124-125; W_UV is pre-transposed once so the
    output projection is a plain batched product.
    """
    C = kv_b.shape[-1]
    w = kv_b.reshape(num_heads, dn + dv, C)
    return w[:, :dn, :].contiguous(), w[:, dn:, :].transpose(1, 2).contiguous()


class HeadWeights:
    """Per-head weights w [H, K, N] packed once for ``head_gemv``
    (``voom_mla_pack_head_weights``): the operand order of its matrix
    instructions, so that every weight load is a contiguous 1 KiB."""

    __slots__ = ("packed", "heads", "k", "n")

    def __init__(self, w: torch.Tensor, *, stream: torch.cuda.Stream | None = None):
        dev = _require_device(w)
        _require(w.dtype == torch.bfloat16 and w.dim() == 3, "w must be bf16 [H, K, N]")
        side = _side_stream(stream)
        w = w.contiguous()
        self.heads, self.k, self.n = (int(v) for v in w.shape)
        nbytes = int(_lib.lib().voom_mla_head_weights_bytes(self.heads, self.k, self.n))
        self.packed = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev)
        if side is not None:
            side.wait_stream(torch.cuda.current_stream())  # w (and its copy) are ready
        _lib.call("voom_mla_pack_head_weights", _ptr(w), _ptr(self.packed), self.heads, self.k,
                  self.n, _stream(stream))
        _used_on(side, w, self.packed)

    @property
    def shape(self):
        return (self.heads, self.k, self.n)


def pack_head_weights(w, *, stream: torch.cuda.Stream | None = None) -> HeadWeights:
    """``w`` as HeadWeights (packed once; a HeadWeights is returned as is)."""
    return w if isinstance(w, HeadWeights) else HeadWeights(w, stream=stream)


def mla_absorb_query(q_nope: torch.Tensor, q_rope: torch.Tensor, w_uk):
    """q_lat = [q_nope . W_UK | q_rope] [B, H, 576] (runtime/glm.py:129-132).

    q_nope [B, H, dn], q_rope [B, H, 64] bf16, W_UK [H, dn, 512] (a tensor,
    packed on each call, or HeadWeights packed once); the per-head product
    runs as one weight stream (``head_gemv``).
    """
    q_nope = q_nope.contiguous()
    q_rope = q_rope.contiguous()
    dev = _require_device(q_nope, q_rope)
    _require(q_nope.dtype == q_rope.dtype == torch.bfloat16 and q_nope.dim() == q_rope.dim() == 3,
             "bf16 q_nope [B, H, dn] and q_rope [B, H, dr]")
    B, H, dn = q_nope.shape
    _require(tuple(q_rope.shape[:2]) == (B, H) and 1 <= B <= 16, "q_rope [B, H, dr], B <= 16")
    w_uk = pack_head_weights(w_uk)
    _require(w_uk.packed.device == dev and w_uk.heads == H and w_uk.k == dn,
             "W_UK must be [H, dn, C] for q_nope [B, H, dn]")
    C, dr = w_uk.n, q_rope.shape[-1]
    q_lat = torch.empty((B, H, C + dr), dtype=q_nope.dtype, device=dev)
    _lib.call("voom_mla_absorb_query", _ptr(q_nope), _ptr(q_rope), _ptr(w_uk.packed), _ptr(q_lat),
              B, H, dn, C, dr, _stream(None))
    return q_lat


def mla_project_out(wc: torch.Tensor, w_uv_t) -> torch.Tensor:
    """weighted_c [B, H, 512] . W_UV -> [B, H, dv] (runtime/glm.py:200-202)."""
    return head_gemv(wc, w_uv_t)


def head_gemv(x: torch.Tensor, w, *, out: torch.Tensor | None = None,
              stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """y [B, H, N] = x [B, H, K] . w [H, K, N] per head (fp32 sums, bf16 out)
    for decode-sized B (<= 16): the absorbed-MLA products as one weight
    stream on matrix instructions (``voom_mla_head_gemv``).  ``w`` is a
    HeadWeights (pack_head_weights, once) or a bf16 tensor [H, K, N], packed
    on the spot.  ``out`` may be wider than N in its last dimension (only the
    first N columns are written)."""
    x = x.contiguous()
    dev = _require_device(x)
    _require(x.dtype == torch.bfloat16 and x.dim() == 3, "bf16 x [B, H, K]")
    B, H, K = x.shape
    _require(1 <= B <= 16, "head_gemv: batch must be 1..16")
    if not isinstance(w, HeadWeights):
        _require(isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.dim() == 3,
                 "w must be HeadWeights or bf16 [H, K, N]")
        _require(w.shape[0] == H and w.shape[1] == K, "w must be [H, K, N] for x [B, H, K]")
        w = HeadWeights(w, stream=stream)
    _require(w.packed.device == dev, "w and x must be on the same device")
    _require(w.heads == H and w.k == K, "w must be [H, K, N] for x [B, H, K]")
    N = w.n
    if out is None:
        out = torch.empty((B, H, N), dtype=x.dtype, device=dev)
    _require(out.dtype == x.dtype and out.device == dev and out.dim() == 3 and
             tuple(out.shape[:2]) == (B, H) and out.shape[2] >= N and out.is_contiguous(),
             "out [B, H, >= N] contiguous bf16")
    side = _side_stream(stream)
    if side is not None:
        side.wait_stream(torch.cuda.current_stream())  # x's contiguous copy and out are ready
    _lib.call("voom_mla_head_gemv", _ptr(x), _ptr(w.packed), _ptr(out), B, H, K, N, K,
              out.shape[2], _stream(stream))
    _used_on(side, x, out)
    return out


def mla_latent_decode_project(q_lat: torch.Tensor, lat_pool: torch.Tensor,
                              block_table: torch.Tensor, ctx_lens: torch.Tensor, w_uv_t, *,
                              scale: float, num_ranges: int = 0, return_weighted_c: bool = False,
                              return_lse: bool = False, ws: torch.Tensor | None = None,
                              stream: torch.cuda.Stream | None = None):
    """Latent contraction and output projection: y [B, H, dv] = weighted_c .
    W_UV (runtime/glm.py:133-164, 200-202) with the merge of the range
    partials and the projection in one launch (``voom_mla_absorbed_decode_project``;
    H a multiple of 64, B <= 16, dv <= 128).  ``w_uv_t`` is W_UV^T [H, 512,
    dv] or its HeadWeights.  Returns y, then weighted_c [B, H, 512] and the
    log-sum-exp [B, H] when asked for."""
    dev = _require_device(q_lat, lat_pool, block_table, ctx_lens)
    _require(q_lat.dim() == 3 and lat_pool.dim() == 3, "q_lat [B,H,576], lat_pool [slots,PT,576]")
    B, H, LD = q_lat.shape
    slots, PT, LD2 = lat_pool.shape
    _require(LD == LD2 == 576, "latent width must be 576 (512 + 64)")
    _require(q_lat.dtype == lat_pool.dtype == torch.bfloat16, "q_lat and lat_pool must be bf16")
    _require(block_table.dtype == torch.int32 and ctx_lens.dtype == torch.int32,
             "block_table and ctx_lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == B and tuple(ctx_lens.shape) == (B,),
             "block_table [B, max_pages], ctx_lens [B]")
    w_uv = pack_head_weights(w_uv_t, stream=stream)
    _require(w_uv.packed.device == dev and w_uv.heads == H and w_uv.k == 512,
             "W_UV^T must be [H, 512, dv]")
    if _BOUNDS_CHECKS:
        check_block_table(block_table, ctx_lens, slots, PT, stream=stream)
    need = mla_workspace_bytes(B, H, num_ranges)
    if ws is None:
        ws = workspace(dev, need, tag=2)
    _require(ws.numel() * ws.element_size() >= need, "workspace too small")
    y = torch.empty((B, H, w_uv.n), dtype=torch.bfloat16, device=dev)
    wc = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev) if return_weighted_c else None
    lse = torch.empty((B, H), dtype=torch.float32, device=dev) if return_lse else None
    _lib.call("voom_mla_absorbed_decode_project", _ptr(q_lat), _ptr(lat_pool), _ptr(block_table),
              _ptr(ctx_lens), _ptr(w_uv.packed), w_uv.n, _ptr(y), _ptr(wc), _ptr(lse), _ptr(ws),
              need, B, H, LD, 512, PT, block_table.shape[1], slots, float(scale), int(num_ranges),
              _stream(stream))
    _used_on(_side_stream(stream), y, wc, lse, ws)
    res = (y,) + ((wc,) if return_weighted_c else ()) + ((lse,) if return_lse else ())
    return res if len(res) > 1 else y


def mla_absorbed_decode(q_nope: torch.Tensor, q_rope: torch.Tensor, lat_pool: torch.Tensor,
                        block_table: torch.Tensor, ctx_lens: torch.Tensor, w_uk, w_uv_t, *,
                        scale: float, num_ranges: int = 0, return_weighted_c: bool = False):
    """Absorbed MLA decode of one query token: runtime/glm.py:78-202.

    q_nope [B, H, dn], q_rope [B, H, 64] bf16; W_UK [H, dn, 512] and W_UV^T
    [H, 512, dv] from split_kv_b (tensors, or HeadWeights packed once).
    q_lat = [q_nope . W_UK | q_rope] comes from one launch
    (``voom_mla_absorb_query``); the latent contraction runs in the HIP latent
    kernel, and with 64-head groups (H a multiple of 64, B <= 16, dv <= 128)
    the merge of its partials and weighted_c . W_UV share one launch.
    Returns the per-head output [B, H, dv] bf16 (before o_proj).
    """
    q_lat = mla_absorb_query(q_nope, q_rope, w_uk)
    B, H = q_lat.shape[:2]
    dv = w_uv_t.shape[-1]
    if H % 64 == 0 and B <= 16 and dv <= 128:
        res = mla_latent_decode_project(q_lat, lat_pool, block_table, ctx_lens, w_uv_t,
                                        scale=scale, num_ranges=num_ranges,
                                        return_weighted_c=return_weighted_c)
        return res
    wc = mla_latent_decode(q_lat, lat_pool, block_table, ctx_lens, scale=scale,
                           num_ranges=num_ranges)
    out = mla_project_out(wc, w_uv_t)
    return (out, wc) if return_weighted_c else out


def append_rows(src: torch.Tensor, pool: torch.Tensor, block_table: torch.Tensor,
                positions: torch.Tensor, *, stream: torch.cuda.Stream | None = None) -> None:
    """Write token rows src [B, L, W] into a row pool [slots, PT, W] at positions[b] + t."""
    _require_device(src, pool, block_table, positions)
    B, L, W = src.shape
    slots, PT, W2 = pool.shape
    _require(W == W2 and src.dtype == pool.dtype and src.element_size() == 2,
             "src and pool must be 16-bit with the same row width")
    _require(block_table.dtype == torch.int32 and positions.dtype == torch.int32
             and block_table.shape[0] == B and tuple(positions.shape) == (B,),
             "block_table [B, max_pages] and positions [B] must be int32")
    _lib.call("voom_append_rows", _ptr(src), _ptr(pool), _ptr(block_table), _ptr(positions), B, L,
              W, PT, block_table.shape[1], slots, _stream(stream))


def gather_rows(pool: torch.Tensor, block_table: torch.Tensor, seq_len: int, *,
                stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Logical rows [B, seq_len, W] of a row pool [slots, PT, W]."""
    dev = _require_device(pool, block_table)
    slots, PT, W = pool.shape
    B = block_table.shape[0]
    _require(block_table.dtype == torch.int32, "block_table must be int32")
    out = torch.empty((B, seq_len, W), dtype=pool.dtype, device=dev)
    _lib.call("voom_gather_rows", _ptr(pool), _ptr(block_table), _ptr(out), B, seq_len, W, PT,
              block_table.shape[1], slots, _stream(stream))
    return out


def rope_cache(max_position: int, head_dim: int, theta: float, *,
               denominators: torch.Tensor | None = None, device=None):
    """fp32 NeoX RoPE tables (cos, sin) [max_position, head_dim / 2]:
    angle = position / theta^(i / half) (runtime/pic_attention.py:150-167)."""
    if max_position <= 0 or head_dim <= 0 or head_dim % 2:
        raise ValueError("RoPE cache dimensions must be positive and even")
    half = head_dim // 2
    dev = torch.device(device) if device is not None else torch.device("cuda")
    if denominators is None:
        denominators = theta ** (torch.arange(half, dtype=torch.float32, device=dev) / half)
    else:
        _require(tuple(denominators.shape) == (half,), "RoPE denominators do not match head_dim")
        denominators = denominators.to(device=dev, dtype=torch.float32)
    angles = torch.arange(max_position, dtype=torch.float32, device=dev)[:, None] / denominators
    return torch.cos(angles).contiguous(), torch.sin(angles).contiguous()


DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}  # VOOM_DTYPE_*


def position_free_workspace_bytes(batch: int, num_q_heads: int, num_queries: int,
                                  num_kv_heads: int, head_dim: int, num_keys: int,
                                  dtype: torch.dtype = torch.bfloat16,
                                  num_splits: int = 0) -> int:
    return int(_lib.lib().voom_position_free_workspace_bytes(
        batch, num_q_heads, num_queries, num_kv_heads, head_dim, num_keys, DTYPE_CODES[dtype],
        num_splits))


def _as_int32(t: torch.Tensor) -> torch.Tensor:
    """Integer index tensors go to the kernel as int32, as the reference casts
    them (runtime/pic_attention.py:223-224)."""
    if t.dtype == torch.int32:
        return t
    _require(not t.is_floating_point() and not t.is_complex(),
             "block table and positions must be integer tensors")
    return t.to(torch.int32)


def position_free_paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                                  block_table: torch.Tensor, key_positions: torch.Tensor,
                                  query_positions: torch.Tensor, cos: torch.Tensor,
                                  sin: torch.Tensor, *, scale: float, num_splits: int = 0,
                                  stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Attend rotated q [B, Nq, Tq, D] to unrotated K / V pages [P, Nkv, BLOCK, D]
    through block_table [ceil(Tk / BLOCK)], rotating each key at its logical
    position (runtime/pic_attention.py:184-232, same arguments and checks).
    Repeating a physical block id is legal and is the sharing primitive.  q and
    the pages share one dtype (bf16, fp16 or fp32); the RoPE tables are fp32
    or that dtype."""
    _require_device(q, k_pages, v_pages, block_table, key_positions, query_positions, cos, sin)
    if q.dim() != 4 or k_pages.dim() != 4 or tuple(v_pages.shape) != tuple(k_pages.shape):
        raise ValueError("invalid Q/K/V page ranks or shapes")
    B, NQ, TQ, D = q.shape
    P, NKV, BLOCK, Dp = k_pages.shape
    TK = key_positions.numel()
    if Dp != D or D % 32 or NQ % NKV or query_positions.numel() != TQ:
        raise ValueError("unsupported head or position geometry")
    if block_table.dim() != 1 or block_table.numel() != (TK + BLOCK - 1) // BLOCK:
        raise ValueError("block table does not cover logical key positions")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] * 2 != D:
        raise ValueError("RoPE cache does not match head dimension")
    if not (q.dtype == k_pages.dtype == v_pages.dtype):
        raise ValueError("Q/K/V page dtypes must match")
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"unsupported Q/K/V dtype {q.dtype}")
    if cos.dtype != sin.dtype or cos.dtype not in (torch.float32, q.dtype):
        raise ValueError("RoPE cache must be FP32 or match the Q/K/V dtype")
    if D > 256:
        raise ValueError(f"head_dim {D} unsupported (a multiple of 32 up to 256)")
    for t in (q, k_pages, v_pages, cos, sin):
        _require(t.is_contiguous(), "tensors must be contiguous")
    block_table = _as_int32(block_table)
    key_positions = _as_int32(key_positions)
    query_positions = _as_int32(query_positions)
    if bounds_checks_enabled():
        check_position_free_pages(block_table, key_positions, BLOCK, P, cos.shape[0],
                                  stream=stream)
    need = position_free_workspace_bytes(B, NQ, TQ, NKV, D, TK, q.dtype, num_splits)
    ws = workspace(q.device, need, tag=3)
    out = torch.empty_like(q)
    _lib.call("voom_position_free_attention", _ptr(q), _ptr(k_pages), _ptr(v_pages),
              _ptr(block_table), _ptr(key_positions), _ptr(query_positions), _ptr(cos),
              _ptr(sin), _ptr(out), _ptr(ws), need, B, NQ, TQ, NKV, D, BLOCK, P, TK,
              cos.shape[0], DTYPE_CODES[q.dtype], DTYPE_CODES[cos.dtype], float(scale),
              int(num_splits), _stream(stream))
    return out
