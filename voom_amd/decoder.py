"""Decode harness for the paged-KV path: a Llama-family decoder (SmolLM2-135M
shape by default) whose attention runs entirely through PagedKVCache.

It restates, for one dense architecture, the three reference pieces that
drive the cache:
  * ``_attention``  (runtime/layer_runner.py:48-182): q/k/v projections,
    NeoX RoPE at the cache offset, ``kv.append`` and then attention over the
    cache -- ``kv.attend`` for one query token, causal ``kv.attend_prefill``
    for a prompt (the reference's explicit causal mask at :166-177);
  * ``run_block``  (runtime/layer_runner.py:320-344): RMSNorm, attention,
    residual, RMSNorm, SwiGLU, residual;
  * the greedy decode loop of StreamingEngine.generate
    (runtime/engine.py:8459-8503): embed the pending token, sweep the
    layers at ``kv.offset``, final norm + tied lm_head, argmax.

GEMMs, norms and RoPE are plain PyTorch-ROCm ops (hipBLASLt GEMMs); every
attention call is the paged HIP kernel.  Weights use the Hugging Face Llama
parameter names so that an in-code ``LlamaForCausalLM`` can load them.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .kv_paged import PagedKVCache


@dataclass(frozen=True)
class DecoderConfig:
    """Model geometry; the defaults are SmolLM2-135M's."""

    num_hidden_layers: int = 30
    hidden_size: int = 576
    num_attention_heads: int = 9
    num_key_value_heads: int = 3
    head_dim: int = 64
    intermediate_size: int = 1536
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    vocab_size: int = 49152

    @property
    def param_count(self) -> int:
        h, i = self.hidden_size, self.intermediate_size
        qkv = h * (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim
        o = self.num_attention_heads * self.head_dim * h
        per_layer = qkv + o + 3 * h * i + 2 * h
        return self.vocab_size * h + self.num_hidden_layers * per_layer + h


def random_weights(cfg: DecoderConfig, seed: int = 0, device=None,
                   dtype=torch.bfloat16, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights under Hugging Face Llama names: matrices ~ N(0, std)
    drawn on the CPU from ``torch.Generator(seed)`` (the same values on every
    device), RMSNorm weights 1, lm_head tied to the embedding."""
    g = torch.Generator().manual_seed(seed)
    h, i = cfg.hidden_size, cfg.intermediate_size
    nq, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

    def mat(rows, cols):
        return (torch.randn((rows, cols), generator=g) * std).to(dtype)

    w = {"model.embed_tokens.weight": mat(cfg.vocab_size, h)}
    for layer in range(cfg.num_hidden_layers):
        p = f"model.layers.{layer}"
        w[f"{p}.self_attn.q_proj.weight"] = mat(nq * hd, h)
        w[f"{p}.self_attn.k_proj.weight"] = mat(nkv * hd, h)
        w[f"{p}.self_attn.v_proj.weight"] = mat(nkv * hd, h)
        w[f"{p}.self_attn.o_proj.weight"] = mat(h, nq * hd)
        w[f"{p}.mlp.gate_proj.weight"] = mat(i, h)
        w[f"{p}.mlp.up_proj.weight"] = mat(i, h)
        w[f"{p}.mlp.down_proj.weight"] = mat(h, i)
        w[f"{p}.input_layernorm.weight"] = torch.ones(h, dtype=dtype)
        w[f"{p}.post_attention_layernorm.weight"] = torch.ones(h, dtype=dtype)
    w["model.norm.weight"] = torch.ones(h, dtype=dtype)
    if device is not None:
        w = {k: v.to(device) for k, v in w.items()}
    return w


class PagedDecoder:
    """Greedy decoder over a PagedKVCache (one GEMM per fused projection)."""

    def __init__(self, cfg: DecoderConfig, weights: dict[str, torch.Tensor], device=None):
        self.cfg = cfg
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        dev = self.device
        w = {k: v.to(dev).contiguous() for k, v in weights.items()}
        self.embed = w["model.embed_tokens.weight"]
        self.final_norm = w["model.norm.weight"]
        self.layers = []
        for layer in range(cfg.num_hidden_layers):
            p = f"model.layers.{layer}"
            self.layers.append({
                "qkv": torch.cat([w[f"{p}.self_attn.q_proj.weight"],
                                  w[f"{p}.self_attn.k_proj.weight"],
                                  w[f"{p}.self_attn.v_proj.weight"]], 0).contiguous(),
                "o": w[f"{p}.self_attn.o_proj.weight"],
                "gate_up": torch.cat([w[f"{p}.mlp.gate_proj.weight"],
                                      w[f"{p}.mlp.up_proj.weight"]], 0).contiguous(),
                "down": w[f"{p}.mlp.down_proj.weight"],
                "ln1": w[f"{p}.input_layernorm.weight"],
                "ln2": w[f"{p}.post_attention_layernorm.weight"],
            })
        half = cfg.head_dim // 2
        self.inv_freq = 1.0 / (cfg.rope_theta ** (
            torch.arange(half, dtype=torch.float32, device=dev) / half))

    # ---- pieces -------------------------------------------------------------

    def _rms_norm(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """fp32 statistics, result cast back before the weight (HF LlamaRMSNorm)."""
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.cfg.rms_norm_eps)
        return weight * xf.to(x.dtype)

    @staticmethod
    def _linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        return F.linear(x.reshape(-1, shape[-1]), weight).reshape(*shape[:-1], weight.shape[0])

    def _rope(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """NeoX (rotate-half) RoPE on x [B, H, L, D] at integer positions [L]."""
        ang = positions.to(torch.float32)[:, None] * self.inv_freq[None, :]
        cos = torch.cat([ang.cos(), ang.cos()], -1)
        sin = torch.cat([ang.sin(), ang.sin()], -1)
        xf = x.float()
        half = x.shape[-1] // 2
        rot = torch.cat([-xf[..., half:], xf[..., :half]], -1)
        return (xf * cos + rot * sin).to(x.dtype)

    def _attention(self, h: torch.Tensor, layer: int, kv: PagedKVCache,
                   offset: int) -> torch.Tensor:
        cfg = self.cfg
        B, L, _ = h.shape
        nq, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        qkv = self._linear(h, self.layers[layer]["qkv"])
        q, k, v = qkv.split([nq * hd, nkv * hd, nkv * hd], dim=-1)
        q = q.reshape(B, L, nq, hd).transpose(1, 2)
        k = k.reshape(B, L, nkv, hd).transpose(1, 2)
        v = v.reshape(B, L, nkv, hd).transpose(1, 2).contiguous()
        pos = torch.arange(offset, offset + L, device=h.device)
        q = self._rope(q, pos).contiguous()
        k = self._rope(k, pos).contiguous()
        kv.append(layer, k, v)
        if L == 1:
            attn = kv.attend(layer, q, scale=hd ** -0.5)
        else:
            attn = kv.attend_prefill(layer, q, scale=hd ** -0.5)
        attn = attn.transpose(1, 2).reshape(B, L, nq * hd)
        return self._linear(attn, self.layers[layer]["o"])

    def run_block(self, x: torch.Tensor, layer: int, kv: PagedKVCache, offset: int):
        lw = self.layers[layer]
        x = x + self._attention(self._rms_norm(x, lw["ln1"]), layer, kv, offset)
        h = self._rms_norm(x, lw["ln2"])
        gate, up = self._linear(h, lw["gate_up"]).chunk(2, dim=-1)
        return x + self._linear(F.silu(gate) * up, lw["down"])

    # ---- model --------------------------------------------------------------

    def new_cache(self, max_bytes: int = 1 << 62, page_positions: int = 64,
                  **kw) -> PagedKVCache:
        return PagedKVCache(self.cfg.num_hidden_layers, max_bytes,
                            page_positions=page_positions, device=self.device, **kw)

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, kv: PagedKVCache,
                last_only: bool = False) -> torch.Tensor:
        """Logits [B, L, vocab] (fp32) for tokens [B, L] appended at kv.offset."""
        offset = kv.offset
        x = self.embed[tokens]
        for layer in range(self.cfg.num_hidden_layers):
            x = self.run_block(x, layer, kv, offset)
        if last_only:
            x = x[:, -1:]
        x = self._rms_norm(x, self.final_norm)
        return self._linear(x, self.embed).float()

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_tokens: int, kv: PagedKVCache):
        """Greedy decode: prefill ``prompt`` [1, L], then ``max_tokens`` tokens.

        Returns (generated token ids, prefill seconds, per-token seconds), each
        time measured to the token's argmax on the host, as the reference's
        loop does.
        """
        t0 = time.perf_counter()
        logits = self.forward(prompt.to(self.device), kv, last_only=True)
        nxt = int(logits[0, -1].argmax())
        prefill_s = time.perf_counter() - t0
        out = [nxt]
        times = []
        pending = torch.empty((1, 1), dtype=torch.long, device=self.device)
        while len(out) < max_tokens:
            t1 = time.perf_counter()
            pending.fill_(nxt)
            logits = self.forward(pending, kv)
            nxt = int(logits[0, -1].argmax())
            times.append(time.perf_counter() - t1)
            out.append(nxt)
        return out, prefill_s, times
