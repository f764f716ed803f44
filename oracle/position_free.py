"""CPU restatement of position-free paged attention -- TEST INFRASTRUCTURE ONLY.

Follows runtime/pic_attention.py:
  rope_tables      :150-167  angles = position / theta^(i / half), fp32
  rotate           :68-90    NeoX rotate-half of the stored key at its
                             logical position, fp32, then rounded to the
                             page element type T (bf16, fp16 or fp32)
  attention        :44-128   q * scale in fp32, visible iff key position <=
                             query position, softmax, zeros when nothing is
                             visible; page row ((blk * NKV + kvh) * BLOCK + off)
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def rope_tables(max_position: int, head_dim: int, theta: float):
    half = head_dim // 2
    den = np.float32(theta) ** (np.arange(half, dtype=np.float32) / np.float32(half))
    ang = np.arange(max_position, dtype=np.float32)[:, None] / den[None, :].astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _store(x: np.ndarray, store: str) -> np.ndarray:
    """x after a round trip through the page element type T."""
    if store == "bf16":
        return round_bf16(x)
    if store == "f16":
        return x.astype(np.float16).astype(np.float32)
    if store == "f32":
        return x.astype(np.float32)
    raise ValueError(f"unknown element type {store}")


def rotate(k: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray, *,
           bf16: bool = True, store: str | None = None) -> np.ndarray:
    """Rotate rows k [..., N, D] at positions [N] (rotate-half) in fp32, then
    round to the element type T (``store``: "bf16", "f16" or "f32"; default
    "bf16" when ``bf16`` else "f32"), as pic_attention.py:81-90 does."""
    store = store or ("bf16" if bf16 else "f32")
    half = k.shape[-1] // 2
    c = np.asarray(cos, dtype=np.float32)[positions]
    s = np.asarray(sin, dtype=np.float32)[positions]
    a = k[..., :half].astype(np.float32)
    b = k[..., half:].astype(np.float32)
    out = np.concatenate([a * c - b * s, b * c + a * s], axis=-1).astype(np.float32)
    return _store(out, store)


def attention(q: np.ndarray, k_pages: np.ndarray, v_pages: np.ndarray, block_table: np.ndarray,
              key_positions: np.ndarray, query_positions: np.ndarray, cos: np.ndarray,
              sin: np.ndarray, scale: float, *, bf16: bool = True, store: str | None = None,
              acc=np.float32) -> np.ndarray:
    """Output [B, NQ, TQ, D] in fp32 (before the final store in T).

    ``store`` is the element type the rotated keys are rounded to (see
    rotate); ``acc`` the type the scores, softmax and P.V are computed in
    (np.float64 gives an fp64 reference for fp32 pages)."""
    store = store or ("bf16" if bf16 else "f32")
    B, NQ, TQ, D = q.shape
    _, NKV, BLOCK, _ = k_pages.shape
    G = NQ // NKV
    TK = key_positions.size
    keys = np.arange(TK)
    pages = block_table[keys // BLOCK] if TK else np.zeros(0, np.int64)
    offs = keys % BLOCK
    out = np.zeros((B, NQ, TQ, D), dtype=np.float32)
    for kvh in range(NKV):
        k_rows = k_pages[pages, kvh, offs].astype(np.float32)     # [TK, D]
        v_rows = v_pages[pages, kvh, offs].astype(acc)
        k_rot = rotate(k_rows, key_positions, cos, sin, store=store).astype(acc)
        for b in range(B):
            for j in range(G):
                h = kvh * G + j
                qv = q[b, h].astype(acc) * acc(scale)                 # [TQ, D]
                s = qv @ k_rot.T                                      # [TQ, TK]
                vis = key_positions[None, :] <= query_positions[:, None]
                s = np.where(vis, s, -np.inf)
                m = s.max(axis=1, initial=-np.inf)
                ok = np.isfinite(m)
                p = np.where(vis, np.exp(s - np.where(ok, m, 0)[:, None]), 0.0)
                l = p.sum(axis=1)
                o = p @ v_rows
                out[b, h] = np.where(ok[:, None], o / np.where(l > 0, l, 1)[:, None], 0.0)
    return out


def attention_torch(q, k_pages, v_pages, block_table, key_positions, query_positions, cos, sin,
                    scale: float):
    """The same attention in torch on the CPU (the timed CPU baseline): gather
    the logical keys through the table, rotate them in fp32 at their positions
    and round to the page dtype, then masked fp32 SDPA with the GQA broadcast.
    q [B, NQ, TQ, D], pages [P, NKV, BLOCK, D] (any float dtype) -> fp32."""
    import torch
    import torch.nn.functional as F

    B, NQ, TQ, D = q.shape
    _, NKV, BLOCK, _ = k_pages.shape
    half = D // 2
    TK = key_positions.numel()
    keys = torch.arange(TK)
    pages = block_table.long()[keys // BLOCK]
    offs = keys % BLOCK
    k = k_pages[pages, :, offs].float()                       # [TK, NKV, D]
    v = v_pages[pages, :, offs].float()
    c = cos.float()[key_positions.long()][:, None, :]
    s = sin.float()[key_positions.long()][:, None, :]
    a, b = k[..., :half], k[..., half:]
    k = torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(k_pages.dtype).float()
    mask = key_positions.long()[None, :] <= query_positions.long()[:, None]   # [TQ, TK]
    out = F.scaled_dot_product_attention(q.float(), k.permute(1, 0, 2)[None],
                                         v.permute(1, 0, 2)[None], attn_mask=mask,
                                         scale=scale, enable_gqa=True)
    return torch.where(mask.any(dim=1)[None, None, :, None], out, torch.zeros_like(out))
