"""Seeded synthetic inputs for the paged-KV workloads (bench, smoke and tests).

The shapes and seeds are those of the benchmark configurations:
  gqa_decode_inputs   config 2 -- B=16, 32 q / 8 kv heads, D=128, contexts
                      U[1024, 32768] (seed 2), K,V ~ N(0,1) (seed 3) with
                      RoPE(theta=5e5) applied to K at positions U[0, 131072)
                      (seed 4), 64-token pages at a seeded permutation of pool
                      slots (seed 5), scale D^-0.5.
Random tensors are generated on the target device with torch generators; the
context lengths, positions and slot permutation come from numpy PCG64 so the
host can rebuild them exactly.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .page_pool import v_pages_to_tokens, v_slot_shape, v_tokens_to_pages


@dataclass
class PagedGQAInputs:
    q: torch.Tensor            # [B, NQ, D] bf16
    k_pool: torch.Tensor       # [slots, NKV, PT, D] bf16
    v_pool: torch.Tensor       # [slots, NKV, PT/32, D, 32] bf16 (V^T blocks)
    block_table: torch.Tensor  # [B, max_pages] int32
    ctx_lens: torch.Tensor     # [B] int32
    ctx_host: np.ndarray
    table_host: np.ndarray
    scale: float
    page_tokens: int

    @property
    def kv_bytes(self) -> int:
        B, NQ, D = self.q.shape
        NKV = self.k_pool.shape[1]
        return int(self.ctx_host.sum()) * NKV * D * 2 * 2

    def algorithmic_bytes(self) -> int:
        """K/V of every live token + q + out + table entries + lengths."""
        B, NQ, D = self.q.shape
        pages = int(np.sum(-(-self.ctx_host // self.page_tokens)))
        return self.kv_bytes + 2 * B * NQ * D * 2 + pages * 4 + B * 4

    def flops(self) -> int:
        B, NQ, D = self.q.shape
        return 4 * NQ * D * int(self.ctx_host.sum())


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float):
    """fp32 cos/sin [n, D/2]: angle = pos / theta^(i/half) (pic_attention.py:150-167)."""
    half = head_dim // 2
    inv = theta ** (torch.arange(half, dtype=torch.float32, device=positions.device) / half)
    ang = positions.to(torch.float32)[:, None] / inv[None, :]
    return torch.cos(ang), torch.sin(ang)


def apply_rope_neox(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE in fp32, x [..., n, D] with tables [n, D/2] (pic_attention.py:170-181)."""
    half = x.shape[-1] // 2
    a, b = x[..., :half].float(), x[..., half:].float()
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


def gqa_decode_inputs(*, batch: int = 16, num_q_heads: int = 32, num_kv_heads: int = 8,
                      head_dim: int = 128, page_tokens: int = 64, ctx_min: int = 1024,
                      ctx_max: int = 32768, ctx_lens=None, rope_theta: float = 5e5,
                      slack_pages: int = 0, device="cuda", seed_base: int = 0,
                      data_seed: int | None = None) -> PagedGQAInputs:
    """Config-2 style inputs.  ``data_seed`` replaces the K/V/q and position
    seeds only (same lengths and page table), which gives a second input set of
    identical shape for Infinity-Cache rotation."""
    dev = torch.device(device)
    if ctx_lens is None:
        ctx = np.random.default_rng(2 + seed_base).integers(ctx_min, ctx_max + 1, size=batch)
    else:
        ctx = np.asarray(ctx_lens, dtype=np.int64)
        batch = len(ctx)
    ctx = ctx.astype(np.int64)
    pages_per = -(-ctx // page_tokens)
    total_pages = int(pages_per.sum())
    slots = max(1, total_pages + slack_pages)
    max_pages = max(1, int(pages_per.max()) if batch else 1)
    perm = np.random.default_rng(5 + seed_base).permutation(slots)
    table = np.zeros((batch, max_pages), dtype=np.int32)
    cursor = 0
    for b in range(batch):
        n = int(pages_per[b])
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n

    gen = torch.Generator(device=dev)
    gen.manual_seed(3 + seed_base if data_seed is None else data_seed)
    NKV, D, PT = num_kv_heads, head_dim, page_tokens
    k_pool = torch.empty((slots, NKV, PT, D), dtype=torch.bfloat16, device=dev)
    v_pool = torch.empty((slots,) + v_slot_shape(NKV, D, PT), dtype=torch.bfloat16, device=dev)
    pos_rng = np.random.default_rng(4 + seed_base if data_seed is None else data_seed + 1)
    # Fill page by page in slot order, rotating K at random positions.
    chunk = 256
    for s0 in range(0, slots, chunk):
        s1 = min(slots, s0 + chunk)
        n = s1 - s0
        kr = torch.randn((n, NKV, PT, D), generator=gen, device=dev, dtype=torch.float32)
        vr = torch.randn((n, NKV, PT, D), generator=gen, device=dev, dtype=torch.float32)
        pos = torch.from_numpy(pos_rng.integers(0, 131072, size=n * PT)).to(dev)
        cos, sin = rope_tables(pos, D, rope_theta)
        cos = cos.view(n, 1, PT, D // 2)
        sin = sin.view(n, 1, PT, D // 2)
        kr = apply_rope_neox(kr, cos, sin)
        k_pool[s0:s1] = kr.to(torch.bfloat16)
        v_pool[s0:s1] = v_tokens_to_pages(vr.to(torch.bfloat16))
    q = torch.randn((batch, num_q_heads, D), generator=gen, device=dev,
                    dtype=torch.float32).to(torch.bfloat16)
    return PagedGQAInputs(
        q=q, k_pool=k_pool, v_pool=v_pool,
        block_table=torch.from_numpy(table).to(dev),
        ctx_lens=torch.from_numpy(ctx.astype(np.int32)).to(dev),
        ctx_host=ctx, table_host=table, scale=D ** -0.5, page_tokens=PT)


def to_reference_layout(inp: PagedGQAInputs):
    """Host fp32 copies in the reference page layout [P, NKV, PT, D] for K and V."""
    k = inp.k_pool.float().cpu().numpy()
    v = v_pages_to_tokens(inp.v_pool).float().cpu().numpy()
    q = inp.q.float().cpu().numpy()
    return q, k, v


@dataclass
class MLAInputs:
    q_nope: torch.Tensor       # [B, H, dn] bf16
    q_rope: torch.Tensor       # [B, H, 64] bf16
    lat_pool: torch.Tensor     # [slots, PT, 576] bf16
    block_table: torch.Tensor  # [B, max_pages] int32
    ctx_lens: torch.Tensor     # [B] int32
    kv_b: torch.Tensor         # [H*(dn+dv), 512] bf16
    ctx_host: np.ndarray
    table_host: np.ndarray
    dn: int
    dv: int
    scale: float
    page_tokens: int

    def latent_bytes(self) -> int:
        return int(self.ctx_host.sum()) * 576 * 2

    def latent_flops(self) -> int:
        H = self.q_nope.shape[1]
        return int(self.ctx_host.sum()) * H * (2 * 576 + 2 * 512)


def mla_decode_inputs(*, batch: int = 8, heads: int = 128, ctx: int = 16384, ctx_lens=None,
                      page_tokens: int = 64, dn: int = 128, dv: int = 128, slack_pages: int = 0,
                      device="cuda", seed: int = 8) -> MLAInputs:
    """Config 5: GLM/DeepSeek absorbed-MLA decode, latent [c_kv 512 | k_rope 64]
    ~ N(0,1) bf16 in 64-token pages at seeded-random slots; q_nope, q_rope
    ~ N(0,1); kv_b ~ N(0, 0.02) (dn = dv = 128 as in DeepSeek-V3); scale
    (dn + 64)^-0.5."""
    dev = torch.device(device)
    ctx_arr = np.full(batch, ctx, dtype=np.int64) if ctx_lens is None else \
        np.asarray(ctx_lens, dtype=np.int64)
    batch = len(ctx_arr)
    pages_per = -(-ctx_arr // page_tokens)
    slots = max(1, int(pages_per.sum()) + slack_pages)
    max_pages = max(1, int(pages_per.max()) if batch else 1)
    perm = np.random.default_rng(seed + 1).permutation(slots)
    table = np.zeros((batch, max_pages), dtype=np.int32)
    cur = 0
    for b in range(batch):
        n = int(pages_per[b])
        table[b, :n] = perm[cur:cur + n]
        cur += n
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    lat = torch.empty((slots, page_tokens, 576), dtype=torch.bfloat16, device=dev)
    for s0 in range(0, slots, 512):
        s1 = min(slots, s0 + 512)
        lat[s0:s1] = torch.randn((s1 - s0, page_tokens, 576), generator=gen, device=dev)
    q_nope = torch.randn((batch, heads, dn), generator=gen, device=dev).to(torch.bfloat16)
    q_rope = torch.randn((batch, heads, 64), generator=gen, device=dev).to(torch.bfloat16)
    kv_b = (torch.randn((heads * (dn + dv), 512), generator=gen, device=dev) * 0.02).to(
        torch.bfloat16)
    return MLAInputs(q_nope=q_nope, q_rope=q_rope, lat_pool=lat,
                     block_table=torch.from_numpy(table).to(dev),
                     ctx_lens=torch.from_numpy(ctx_arr.astype(np.int32)).to(dev), kv_b=kv_b,
                     ctx_host=ctx_arr, table_host=table, dn=dn, dv=dv,
                     scale=(dn + 64) ** -0.5, page_tokens=page_tokens)


def mla_logical_latent(inp: MLAInputs, b: int) -> np.ndarray:
    """Host fp32 latent rows [ctx_b, 576] of sequence b in logical order."""
    n = -(-int(inp.ctx_host[b]) // inp.page_tokens)
    ids = torch.from_numpy(inp.table_host[b, :n].astype(np.int64)).to(inp.lat_pool.device)
    rows = inp.lat_pool[ids].reshape(-1, 576)[: int(inp.ctx_host[b])]
    return rows.float().cpu().numpy()
