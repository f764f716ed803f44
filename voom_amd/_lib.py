"""ctypes binding of libvoom_hip.so (the C ABI declared in include/voom_hip.h).

There is no fallback: if the library is missing or does not load, every
operation raises.  Return codes map to exceptions the way the reference's
kernel wrapper does (runtime/pic_attention.py:195-213): validation failures
raise ``ValueError`` and device/runtime failures raise ``RuntimeError``.
"""

from __future__ import annotations

import atexit
import ctypes
import threading
from ctypes import c_float, c_int, c_size_t, c_void_p

from ._build import LIB_PATH

VOOM_EINVAL = -1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = c_void_p
# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "voom_last_error": (ctypes.c_char_p, []),
    "voom_abi_version": (c_int, []),
    "voom_paged_gqa_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "voom_paged_gqa_default_splits": (c_int, []),
    "voom_paged_gqa_decode": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_size_t,
                                      c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                      c_float, c_int, _P]),
    "voom_paged_gqa_noalloc_max_bytes": (c_size_t, []),
    "voom_paged_gqa_decode_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int,
                                              c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "voom_paged_gqa_partials": (c_int, [_P, _P, _P, _P, _P, _P, c_size_t, c_int, c_int, c_int,
                                        c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "voom_paged_gqa_combine": (c_int, [_P, _P, _P, _P, c_size_t, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_int, _P]),
    "voom_merge_attn_states": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, _P]),
    "voom_fold_attn_state": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P]),
    "voom_mla_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "voom_mla_absorbed_decode": (c_int, [_P, _P, _P, _P, _P, _P, _P, c_size_t, c_int, c_int,
                                         c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "voom_mla_absorbed_decode_project": (c_int, [_P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, c_size_t,
                                                 c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                                 c_float, c_int, _P]),
    "voom_mla_sparse_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "voom_mla_sparse_decode": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, c_size_t, c_int, c_int,
                                       c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                       _P]),
    "voom_dsa_index_scores": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float,
                                      _P]),
    "voom_dsa_topk_workspace_bytes": (c_size_t, [c_int, c_int]),
    "voom_dsa_topk": (c_int, [_P, _P, _P, _P, _P, c_size_t, c_int, c_int, c_int, _P]),
    "voom_add_rms_norm": (c_int, [_P, _P, _P, _P, c_int, c_int, c_float, _P]),
    "voom_rope_split": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_silu_mul": (c_int, [_P, _P, c_int, c_int, _P]),
    "voom_gemv_bf16": (c_int, [_P, _P, _P, c_int, c_int, c_int, _P]),
    "voom_qkv_rope_append": (c_int, [_P, _P, _P, _P, c_float, _P, _P, _P, _P, _P, _P, _P, _P,
                                     c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                     _P]),
    "voom_mla_head_gemv": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_mla_head_weights_bytes": (c_size_t, [c_int, c_int, c_int]),
    "voom_mla_pack_head_weights": (c_int, [_P, _P, c_int, c_int, c_int, _P]),
    "voom_mla_absorb_query": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_lm_head_argmax": (c_int, [_P, _P, _P, c_float, _P, c_int, c_int, _P, c_size_t, _P, _P,
                                    _P]),
    "voom_add_rms_norm_gemv": (c_int, [_P, _P, _P, c_float, _P, _P, _P, c_int, c_int, c_int,
                                       _P]),
    "voom_position_free_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int,
                                                      c_int, c_int]),
    "voom_position_free_attention": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_size_t,
                                             c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                             c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "voom_check_block_table": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "voom_check_selection": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_check_position_free_pages": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "voom_append_kv": (c_int, [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int,
                               c_int, c_int, _P]),
    "voom_gather_kv": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int,
                               c_int, _P]),
    "voom_append_rows": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_gather_rows": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "voom_byteplane_split": (c_int, [_P, _P, _P, c_size_t, _P]),
    "voom_byteplane_merge": (c_int, [_P, _P, _P, c_size_t, _P]),
    "voom_byteplane_split_slots": (c_int, [_P, _P, c_int, c_size_t, c_int, _P, _P, _P, _P]),
    "voom_byteplane_merge_slots": (c_int, [_P, _P, _P, _P, c_int, c_size_t, c_int, _P, _P]),
    "voom_page_sums_verify": (c_int, [_P, _P, c_int, c_int, _P, _P]),
    "voom_record_prepare": (c_int, []),
    "voom_spill_record": (c_int, [_P, _P, _P, c_int, _P, c_int, _P, c_int, c_int, c_int, _P]),
    "voom_reload_record": (c_int, [_P, c_int, c_int, _P, _P, _P, c_int, _P, c_int, c_int, _P,
                                   _P]),
    "voom_copy_rows": (c_int, [_P, c_size_t, _P, c_size_t, c_size_t, c_size_t, _P]),
}


class VoomLibraryError(RuntimeError):
    """libvoom_hip.so is missing or failed to load."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise VoomLibraryError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() first")
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:  # pragma: no cover - depends on the box
                raise VoomLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
            atexit.register(_teardown)
    return _lib


def _teardown() -> None:
    """At interpreter exit, before the HIP runtime's static finalisers: wait for
    the device, then drop the cached kernel workspaces and every pinned host
    arena, so that no device or pinned allocation of this package outlives the
    Python objects that own it (profiler tools that trace copies finalise
    their own state at exit too)."""
    try:
        import torch

        if not torch.cuda.is_initialized():
            return
        torch.cuda.synchronize()
        from . import host_arena, ops

        ops._WORKSPACES.clear()
        host_arena.close_all()
        import gc

        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        host_empty = getattr(torch._C, "_host_emptyCache", None)
        if host_empty is not None:
            host_empty()
    except Exception:  # pragma: no cover - best effort at exit
        pass


def last_error() -> str:
    msg = lib().voom_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Raise for a non-zero ABI return code."""
    if rc == 0:
        return
    msg = last_error()
    if rc < 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
