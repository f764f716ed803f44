"""DSA (DeepSeek Sparse Attention) indexer state for GLM-5-style decode.

Restates runtime/glm_dsa.py's DSAState with the same methods and meaning:
  * ``observe`` (:99-111) appends every call's index keys to the layer's
    cache: k = layer_norm(h . wk^T) with interleaved RoPE on the first
    qk_rope_head_dim dims at absolute positions (rope first, pass-through
    second, :51-73);
  * ``update_and_select`` (:113-166) returns None while the cache holds at
    most index_topk keys (every position is selected, the dense path is
    exact), else the ascending top-k key indices per query, shape
    (B, L, index_topk); 'shared' layers reuse the last 'full' selection;
  * ``trim`` (:75-87) rolls the caches back and drops the selection.

The projections are torch ops, in the weights' dtype, with RoPE and the
layer norm computed in fp32 and rounded back, as the reference's MLX ops do.
The scores and the top-k are the HIP kernels voom_dsa_index_scores and
voom_dsa_topk; the index keys live in one device buffer per 'full' layer,
[B, capacity, head_dim], grown geometrically.
"""

from __future__ import annotations

import torch

from . import ops


def rope_interleaved(x: torch.Tensor, offset: int, dims: int, theta: float) -> torch.Tensor:
    """Interleaved ("traditional") RoPE of x[..., :dims] at positions
    offset + arange(L) along dim -2; the rest passes through (rope first,
    runtime/glm_dsa.py:69-73).  Computed in fp32, returned in x's dtype."""
    L = x.shape[-2]
    pos = torch.arange(offset, offset + L, dtype=torch.float32, device=x.device)
    inv = theta ** (-torch.arange(0, dims, 2, dtype=torch.float32, device=x.device) / dims)
    ang = pos[:, None] * inv[None, :]                     # [L, dims/2]
    cos, sin = torch.cos(ang), torch.sin(ang)
    xf = x[..., :dims].float()
    x1, x2 = xf[..., 0::2], xf[..., 1::2]
    out = torch.empty_like(xf)
    out[..., 0::2] = x1 * cos - x2 * sin
    out[..., 1::2] = x1 * sin + x2 * cos
    return torch.cat([out.to(x.dtype), x[..., dims:]], dim=-1)


def _linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return x.to(weight.dtype) @ weight.t()


def index_keys(h: torch.Tensor, w: dict, prefix: str, offset: int, *, rope_dims: int,
               theta: float) -> torch.Tensor:
    """k = RoPE(layer_norm(h . wk^T)) [B, L, head_dim] (runtime/glm_dsa.py:103-109)."""
    k = _linear(h, w[f"{prefix}.self_attn.indexer.wk.weight"])
    kf = torch.nn.functional.layer_norm(
        k.float(), (k.shape[-1],), w[f"{prefix}.self_attn.indexer.k_norm.weight"].float(),
        w[f"{prefix}.self_attn.indexer.k_norm.bias"].float(), 1e-6)
    return rope_interleaved(kf.to(k.dtype), offset, rope_dims, theta)


def index_queries(q_a: torch.Tensor, h: torch.Tensor, w: dict, prefix: str, offset: int, *,
                  n_heads: int, head_dim: int, rope_dims: int, theta: float):
    """(q_idx [B, L, NH, head_dim], w_head [B, L, NH] fp32 times NH^-0.5)
    (runtime/glm_dsa.py:130-150)."""
    B, L, _ = q_a.shape
    q = _linear(q_a, w[f"{prefix}.self_attn.indexer.wq_b.weight"]).reshape(B, L, n_heads, head_dim)
    q = rope_interleaved(q.transpose(1, 2), offset, rope_dims, theta).transpose(1, 2)
    wp = w[f"{prefix}.self_attn.indexer.weights_proj.weight"]
    w_head = (h.to(wp.dtype) @ wp.t()).float() * (n_heads ** -0.5)
    return q, w_head


class _KeyCache:
    """Index keys of one 'full' layer: [B, capacity, head_dim], length used."""

    def __init__(self, k: torch.Tensor):
        B, L, D = k.shape
        cap = max(256, L)
        self.buf = torch.empty((B, cap, D), dtype=k.dtype, device=k.device)
        self.buf[:, :L] = k
        self.length = L

    def append(self, k: torch.Tensor) -> None:
        B, L, D = k.shape
        need = self.length + L
        if need > self.buf.shape[1]:
            cap = max(need, self.buf.shape[1] + self.buf.shape[1] // 4, 256)
            grown = torch.empty((B, cap, D), dtype=self.buf.dtype, device=self.buf.device)
            grown[:, :self.length] = self.buf[:, :self.length]
            self.buf = grown
        self.buf[:, self.length:need] = k
        self.length = need

    def view(self) -> torch.Tensor:
        return self.buf[:, :self.length]


class DSAState:
    """Per-generation indexer state: cached index keys per 'full' layer and the
    selection shared with subsequent 'shared' layers."""

    def __init__(self, cfg=None, *, index_topk: int | None = None, index_n_heads: int = 32,
                 index_head_dim: int = 128, qk_rope_head_dim: int | None = None,
                 rope_theta: float | None = None):
        get = (lambda name, default: getattr(cfg, name, default)) if cfg is not None else (
            lambda name, default: default)
        self.index_topk = int(index_topk if index_topk is not None else get("index_topk", 2048))
        self.n_heads = int(get("index_n_heads", index_n_heads) or index_n_heads)
        self.head_dim = int(get("index_head_dim", index_head_dim) or index_head_dim)
        self.rope_dims = int(qk_rope_head_dim if qk_rope_head_dim is not None
                             else get("qk_rope_head_dim", 64))
        self.theta = float(rope_theta if rope_theta is not None else get("rope_theta", 10000.0))
        self.k_idx: dict[int, _KeyCache] = {}
        self.selection: torch.Tensor | None = None
        self.sel_layer = -1
        self.stats = {"observations": 0, "sparse_selects": 0, "shared_reuses": 0}

    def keys(self, layer: int) -> torch.Tensor | None:
        c = self.k_idx.get(layer)
        return None if c is None else c.view()

    def trim(self, length: int) -> None:
        for c in self.k_idx.values():
            c.length = min(c.length, int(length))
        self.selection = None
        self.sel_layer = -1

    def observe(self, layer: int, indexer_type: str, h: torch.Tensor, w: dict, prefix: str,
                offset: int = 0) -> None:
        if indexer_type != "full":
            return
        k_new = index_keys(h, w, prefix, offset, rope_dims=self.rope_dims, theta=self.theta)
        c = self.k_idx.get(layer)
        if c is None:
            self.k_idx[layer] = _KeyCache(k_new)
        else:
            c.append(k_new)
        self.stats["observations"] += 1

    def update_and_select(self, layer: int, indexer_type: str, h: torch.Tensor,
                          q_a: torch.Tensor, w: dict, prefix: str, offset: int):
        """(B, L, index_topk) int32 ascending key indices, or None when every
        cached key is selected."""
        if indexer_type == "shared":
            self.stats["shared_reuses"] += 1
            return self.selection
        c = self.k_idx.get(layer)
        if c is None or c.length <= self.index_topk:
            self.selection = None
            return None
        q_idx, w_head = index_queries(q_a, h, w, prefix, offset, n_heads=self.n_heads,
                                      head_dim=self.head_dim, rope_dims=self.rope_dims,
                                      theta=self.theta)
        B, L = q_idx.shape[:2]
        k_all = c.buf
        rows = []
        for t in range(L):  # query t (position offset + t) sees keys s <= offset + t
            n = min(c.length, offset + t + 1)
            lens = torch.full((B,), n, dtype=torch.int32, device=k_all.device)
            scores = ops.dsa_index_scores(q_idx[:, t].to(torch.bfloat16).contiguous(),
                                          w_head[:, t].contiguous(), k_all, lens,
                                          scale=self.head_dim ** -0.5)
            sel, _ = ops.dsa_topk(scores, lens, self.index_topk)
            rows.append(sel)
        sel = torch.stack(rows, dim=1)
        self.selection = sel
        self.sel_layer = layer
        self.stats["sparse_selects"] += 1
        return sel
