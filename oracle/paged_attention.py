"""Paged decode attention, restated on the CPU (test infrastructure only).

The reference decode step is two moves:
  1. PagedKVCache.update concatenates every page of the layer in logical order,
     followed by the open tail (runtime/kv_paged.py:164-181).  With pages in a
     pool addressed through a block table, logical page p of a sequence is
     pool[table[p]]; the token at logical position t is page t // BLOCK,
     offset t % BLOCK (runtime/pic_attention.py:60-65).
  2. mx.fast.scaled_dot_product_attention(q, K, V, scale=hd**-0.5) with one
     query token and no mask (runtime/layer_runner.py:170-180); query head h
     reads KV head h // (NQ // NKV) (the GQA broadcast inside SDPA, the same
     map as kv_head = query_head / GQA in runtime/pic_attention.py:33).

Pages here are always in the reference's token-major layout [P, NKV, BLOCK, D]
for both K and V; callers holding a transposed V pool transpose it first.
"""

from __future__ import annotations

import numpy as np


def gather_logical(pages: np.ndarray, table_row: np.ndarray, ctx: int) -> np.ndarray:
    """Concatenate pages in logical order: [NKV, ctx, D] (kv_paged.py:164-181)."""
    P, NKV, BLOCK, D = pages.shape
    n_pages = -(-ctx // BLOCK)
    ids = np.asarray(table_row[:n_pages], dtype=np.int64)
    # [n_pages, NKV, BLOCK, D] -> [NKV, n_pages*BLOCK, D]
    seq = pages[ids].transpose(1, 0, 2, 3).reshape(NKV, n_pages * BLOCK, D)
    return seq[:, :ctx, :]


def sdpa_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                dtype=np.float32) -> np.ndarray:
    """softmax(q.K^T*scale).V for one query token per head with GQA broadcast.

    q [NQ, D]; k, v [NKV, S, D].  Returns [NQ, D] in ``dtype``.  An empty key
    set returns zeros.
    """
    NQ, D = q.shape
    NKV, S, _ = k.shape
    G = NQ // NKV
    out = np.zeros((NQ, D), dtype=dtype)
    if S == 0:
        return out
    qd = q.astype(dtype)
    for h in range(NQ):
        kh = k[h // G].astype(dtype)
        vh = v[h // G].astype(dtype)
        s = (kh @ qd[h]) * dtype(scale)
        s = s - s.max()
        p = np.exp(s)
        out[h] = (p @ vh) / p.sum()
    return out


def paged_decode(q: np.ndarray, k_pages: np.ndarray, v_pages: np.ndarray,
                 block_table: np.ndarray, ctx_lens: np.ndarray, scale: float,
                 dtype=np.float32) -> np.ndarray:
    """Reference decode over a page pool: q [B, NQ, D] -> out [B, NQ, D].

    Inputs are fp32 arrays holding the (bf16-representable) values.
    """
    B = q.shape[0]
    out = np.zeros(q.shape, dtype=dtype)
    for b in range(B):
        ctx = int(ctx_lens[b])
        k = gather_logical(k_pages, block_table[b], ctx)
        v = gather_logical(v_pages, block_table[b], ctx)
        out[b] = sdpa_decode(q[b], k, v, scale, dtype=dtype)
    return out


def paged_decode_lse(q: np.ndarray, k_pages: np.ndarray, block_table: np.ndarray,
                     ctx_lens: np.ndarray, scale: float) -> np.ndarray:
    """Natural-log sum-exp of the scaled scores per (b, q-head), in fp64."""
    B, NQ, D = q.shape
    NKV = k_pages.shape[1]
    G = NQ // NKV
    lse = np.full((B, NQ), -np.inf)
    for b in range(B):
        ctx = int(ctx_lens[b])
        if ctx == 0:
            continue
        k = gather_logical(k_pages, block_table[b], ctx).astype(np.float64)
        for h in range(NQ):
            s = (k[h // G] @ q[b, h].astype(np.float64)) * scale
            m = s.max()
            lse[b, h] = m + np.log(np.exp(s - m).sum())
    return lse


def paged_decode_torch(q, k_pages, v_pages, block_table, ctx_lens, scale: float):
    """The same decode in torch on the CPU, for the timed CPU baseline.

    The reference's own CPU path: concatenate each sequence's pages in logical
    order (runtime/kv_paged.py:164-181), then one fp32 scaled-dot-product
    attention call per sequence with the GQA broadcast inside it
    (mx.fast.scaled_dot_product_attention, runtime/layer_runner.py:170-180;
    here torch.nn.functional.scaled_dot_product_attention with enable_gqa).
    q [B, NQ, D], k_pages / v_pages [P, NKV, BLOCK, D] CPU tensors of any float
    dtype (bf16 pages are widened to fp32 after the gather), block_table
    [B, max_pages] and ctx_lens [B] integer arrays.  Returns fp32 [B, NQ, D].
    """
    import torch

    B, NQ, D = q.shape
    BLOCK = k_pages.shape[2]
    NKV = k_pages.shape[1]
    out = torch.zeros((B, NQ, D), dtype=torch.float32)
    for b in range(B):
        ctx = int(ctx_lens[b])
        if ctx == 0:
            continue
        n_pages = -(-ctx // BLOCK)
        ids = torch.as_tensor(np.asarray(block_table[b][:n_pages], dtype=np.int64))
        k = k_pages.index_select(0, ids).transpose(0, 1).reshape(NKV, n_pages * BLOCK, D)
        v = v_pages.index_select(0, ids).transpose(0, 1).reshape(NKV, n_pages * BLOCK, D)
        out[b] = sdpa_decode_torch(q[b], k[:, :ctx], v[:, :ctx], scale)
    return out


def sdpa_decode_torch(q, k, v, scale: float):
    """One query token per head over logical K/V in torch on the CPU:
    q [NQ, D], k / v [NKV, S, D] -> fp32 [NQ, D] (the reference's SDPA call,
    runtime/layer_runner.py:179-180, with the GQA broadcast)."""
    import torch.nn.functional as F

    return F.scaled_dot_product_attention(q.float()[None, :, None, :], k.float()[None],
                                          v.float()[None], scale=scale,
                                          enable_gqa=True)[0, :, 0]
