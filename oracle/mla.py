"""Absorbed and expanded MLA attention on the CPU (test infrastructure only).

``absorbed`` restates _mla_absorbed_attention (runtime/glm.py:78-210):
  w_kvb = kv_b.reshape(H, dn+dv, C); W_UK = w_kvb[:, :dn], W_UV = w_kvb[:, dn:]
  q_lat = [q_nope . W_UK | q_rope]                                 (:124-132)
  scores = (q_lat . lat^T) as fp32 * (dn+dr)^-0.5 * mult, causal
  for L > 1                                                         (:133-153)
  dense: softmax(scores) cast to the input dtype, . c               (:157-164)
  tiled: running max/sum/c in fp32 over key tiles, then cast        (:165-196)
  out = weighted_c . W_UV^T                                         (:200-202)
``expanded`` is the non-absorbed form the reference tests against
(tests/test_mla_absorbed.py:160-186): K = [c.W_UK^T | k_rope], V = c.W_UV^T.

With ``bf16=True`` every MLX op output that the reference produces in the
input dtype is rounded to bf16 at the same point (einsum, matmul, the softmax
cast), which is what the reference computes on bf16 caches.
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def _rnd(x: np.ndarray, bf16: bool) -> np.ndarray:
    return round_bf16(x.astype(np.float32)) if bf16 else x


def split_kvb(kv_b: np.ndarray, H: int, dn: int, dv: int):
    C = kv_b.shape[-1]
    w = kv_b.reshape(H, dn + dv, C)
    return w[:, :dn, :], w[:, dn:, :]


def absorbed_weighted_c(q_lat: np.ndarray, lat: np.ndarray, dr: int, scale: float, *,
                        offset: int = 0, key_tile_size: int = 0, bf16: bool = False,
                        dtype=np.float32) -> np.ndarray:
    """The latent contraction: q_lat [B,H,L,C+dr], lat [B,S,C+dr] -> [B,H,L,C]."""
    B, H, L, _ = q_lat.shape
    S = lat.shape[1]
    c = lat[..., :-dr]

    def score_tile(start: int, end: int) -> np.ndarray:
        tile = lat[:, start:end, :].astype(dtype)
        s = np.einsum("bhlk,bsk->bhls", q_lat.astype(dtype), tile)
        s = _rnd(s, bf16).astype(np.float32 if dtype == np.float32 else dtype) * scale
        if L > 1:
            qpos = np.arange(offset, offset + L)[:, None]
            kpos = np.arange(start, end)[None, :]
            s = s + np.where(kpos <= qpos, 0.0, -np.inf)[None, None]
        return s

    if key_tile_size <= 0 or key_tile_size >= S:
        s = score_tile(0, S)
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        p = p / p.sum(axis=-1, keepdims=True)
        p = _rnd(p, bf16)
        wc = np.einsum("bhls,bsc->bhlc", p, c.astype(dtype))
        return _rnd(wc, bf16)
    run_max = np.full((B, H, L, 1), -np.inf, dtype=dtype)
    run_sum = np.zeros((B, H, L, 1), dtype=dtype)
    run_c = np.zeros((B, H, L, c.shape[-1]), dtype=dtype)
    for start in range(0, S, key_tile_size):
        end = min(start + key_tile_size, S)
        s = score_tile(start, end)
        nxt = np.maximum(run_max, s.max(axis=-1, keepdims=True))
        old = np.exp(run_max - nxt)
        w = np.exp(s - nxt)
        run_sum = run_sum * old + w.sum(axis=-1, keepdims=True)
        run_c = run_c * old + np.einsum("bhls,bsc->bhlc", w, c[:, start:end].astype(dtype))
        run_max = nxt
    return _rnd(run_c / run_sum, bf16)


def absorbed(q_nope: np.ndarray, q_rope: np.ndarray, lat: np.ndarray, kv_b: np.ndarray,
             dn: int, dv: int, *, offset: int = 0, softmax_scale_mult: float = 1.0,
             key_tile_size: int = 0, bf16: bool = False, dtype=np.float32):
    """Per-head output [B,H,L,dv] of absorbed MLA (before o_proj) and weighted_c."""
    B, H, L, _ = q_nope.shape
    dr = q_rope.shape[-1]
    w_uk, w_uv = split_kvb(kv_b, H, dn, dv)
    q_abs = _rnd(np.einsum("bhld,hdc->bhlc", q_nope.astype(dtype), w_uk.astype(dtype)), bf16)
    q_lat = np.concatenate([q_abs, q_rope.astype(dtype)], axis=-1)
    scale = (dn + dr) ** -0.5 * softmax_scale_mult
    wc = absorbed_weighted_c(q_lat, lat, dr, scale, offset=offset,
                             key_tile_size=key_tile_size, bf16=bf16, dtype=dtype)
    out = _rnd(np.einsum("bhlc,hdc->bhld", wc, w_uv.astype(dtype)), bf16)
    return out, wc


def expanded(q_nope: np.ndarray, q_rope: np.ndarray, c_all: np.ndarray, k_rope: np.ndarray,
             kv_b: np.ndarray, dn: int, dv: int, *, offset: int = 0,
             dtype=np.float64) -> np.ndarray:
    """Expand-then-attend MLA [B,H,L,dv] (tests/test_mla_absorbed.py:160-186)."""
    B, H, L, _ = q_nope.shape
    S = c_all.shape[1]
    dr = q_rope.shape[-1]
    kvb = (c_all.astype(dtype) @ kv_b.astype(dtype).T).reshape(B, S, H, dn + dv)
    kvb = kvb.transpose(0, 2, 1, 3)
    k_nope, values = kvb[..., :dn], kvb[..., dn:]
    keys = np.concatenate(
        [k_nope, np.broadcast_to(k_rope.astype(dtype)[:, None], (B, H, S, dr))], axis=-1)
    queries = np.concatenate([q_nope, q_rope], axis=-1).astype(dtype)
    s = np.einsum("bhld,bhsd->bhls", queries, keys) * (dn + dr) ** -0.5
    qpos = np.arange(offset, offset + L)[:, None]
    kpos = np.arange(S)[None, :]
    s = s + np.where(kpos <= qpos, 0.0, -np.inf)[None, None]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhls,bhsd->bhld", p, values)


def project(out_heads: np.ndarray, o_proj: np.ndarray) -> np.ndarray:
    """[B,H,L,dv] -> [B,L,hidden] through o_proj (runtime/glm.py:203-210)."""
    B, H, L, dv = out_heads.shape
    return out_heads.transpose(0, 2, 1, 3).reshape(B, L, H * dv) @ o_proj.T


def absorbed_weighted_c_torch(q_lat, lat, dr: int, scale: float):
    """The dense decode contraction of absorbed_weighted_c (L = 1, bf16 cache) in
    torch on the CPU, for the timed CPU baseline: fp32 scores of the bf16
    operands rounded to bf16 as MLX's einsum output (runtime/glm.py:133-141),
    softmax in fp32 cast to bf16 (:157-161), then P . c rounded to bf16
    (:162-164).  q_lat [B, H, C + dr] and lat [B, S, C + dr] bf16 CPU tensors;
    returns weighted_c [B, H, C] as fp32 values of bf16 numbers."""
    import torch

    c = lat[..., :-dr]
    s = torch.bmm(q_lat.float(), lat.float().transpose(1, 2))
    s = s.to(torch.bfloat16).float() * scale
    p = torch.softmax(s, dim=-1).to(torch.bfloat16).float()
    return torch.bmm(p, c.float()).to(torch.bfloat16).float()
