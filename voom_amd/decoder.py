"""Decode harness for the paged-KV path: a Llama-family decoder (SmolLM2-135M
shape by default) whose attention runs entirely through PagedKVCache.

It restates, for one dense architecture, the three reference pieces that
drive the cache:
  * ``_block``, the attention part (runtime/layer_runner.py:48-182): q/k/v
    projections, NeoX RoPE at the cache offset, ``kv.append`` and then
    attention over the cache -- ``kv.attend`` for one query token, causal
    ``kv.attend_prefill`` for a prompt (the reference's explicit causal mask
    at :166-177);
  * ``_block``, the rest of the layer (runtime/layer_runner.py:320-344):
    RMSNorm, attention, residual, RMSNorm, SwiGLU, residual;
  * the greedy decode loop of StreamingEngine.generate
    (runtime/engine.py:8459-8503): embed the pending token, sweep the
    layers at ``kv.offset``, final norm + tied lm_head, argmax.

GEMMs are PyTorch-ROCm (hipBLASLt); the residual add + RMSNorm, RoPE with
the q/k/v split, and SwiGLU are fused HIP kernels (voom_add_rms_norm,
voom_rope_split, voom_silu_mul), and every attention call is the paged HIP
kernel.  ``generate_graph`` replays each decode step from one captured HIP
graph.  Weights use the Hugging Face Llama parameter names so that an
in-code ``LlamaForCausalLM`` can load them.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
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

    def _norm(self, x: torch.Tensor, weight: torch.Tensor,
              delta: torch.Tensor | None = None) -> torch.Tensor:
        """x += delta (in place, when given), then RMSNorm: fp32 statistics,
        result cast to bf16 before the weight (HF LlamaRMSNorm)."""
        return ops.add_rms_norm(x, weight, self.cfg.rms_norm_eps, delta=delta)

    @staticmethod
    def _linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """x . weight^T: one row of activations (a decode step) through the
        one-token GEMV kernel, more rows (prefill, batches) through the library
        GEMM."""
        shape = x.shape
        if x.numel() == shape[-1] and shape[-1] <= ops.GEMV_MAX_K:
            return ops.gemv(x.contiguous(), weight)
        return F.linear(x.reshape(-1, shape[-1]), weight).reshape(*shape[:-1], weight.shape[0])

    def _mlp(self, h: torch.Tensor, lw: dict) -> torch.Tensor:
        """down(bf16(silu(gate(h))) * up(h)); one row fuses gate/up and SwiGLU."""
        if h.numel() == h.shape[-1] and h.shape[-1] <= ops.GEMV_MAX_K:
            act = ops.gemv(h.contiguous(), lw["gate_up"], swiglu=True)
        else:
            act = ops.silu_mul(self._linear(h, lw["gate_up"]))
        return self._linear(act, lw["down"])

    def _rope_tables(self, positions: torch.Tensor):
        """fp32 cos/sin [L, head_dim] at integer positions [L] (NeoX layout)."""
        ang = positions.to(torch.float32)[:, None] * self.inv_freq[None, :]
        return (torch.cat([ang.cos(), ang.cos()], -1).contiguous(),
                torch.cat([ang.sin(), ang.sin()], -1).contiguous())

    def _block_token(self, x: torch.Tensor, spare: torch.Tensor, delta: torch.Tensor | None,
                     layer: int, kv: PagedKVCache, cos: torch.Tensor, sin: torch.Tensor):
        """``_block`` for one token of one sequence in a captured step, with
        each residual add and RMSNorm folded into the projection that consumes
        it.  The residual stream moves between two buffers instead of being
        updated in place: x holds it before the layer (before adding
        ``delta``), a fused launch reads one buffer and writes the sum to the
        other.  Returns (the MLP output = the next layer's delta, the buffer
        holding the stream, the spare buffer)."""
        cfg = self.cfg
        lw = self.layers[layer]
        nq, hd, eps = cfg.num_attention_heads, cfg.head_dim, cfg.rms_norm_eps
        if delta is None:
            q = kv.project_append_at(layer, x, lw["qkv"], cos, sin, nq, ln_weight=lw["ln1"],
                                     eps=eps)
        else:
            q = kv.project_append_at(layer, x, lw["qkv"], cos, sin, nq, ln_weight=lw["ln1"],
                                     eps=eps, delta=delta, x_out=spare)
            x, spare = spare, x
        attn = kv.attend_at(layer, q, hd ** -0.5)
        o = ops.gemv(attn.reshape(1, 1, nq * hd), lw["o"])
        act = ops.gemv(x, lw["gate_up"], swiglu=True, ln_weight=lw["ln2"], eps=eps, delta=o,
                       x_out=spare)
        return ops.gemv(act, lw["down"]), spare, x

    def _block(self, x: torch.Tensor, delta: torch.Tensor | None, layer: int,
               kv: PagedKVCache, cos: torch.Tensor, sin: torch.Tensor,
               graph: bool = False) -> torch.Tensor:
        """One layer on the residual stream x [B, L, H] (updated in place with
        the previous layer's MLP output ``delta``); returns this layer's MLP
        output, the next layer's delta."""
        cfg = self.cfg
        lw = self.layers[layer]
        B, L, _ = x.shape
        nq, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        h = self._norm(x, lw["ln1"], delta)
        if graph:
            q, k, v = ops.rope_split(self._linear(h, lw["qkv"]), cos, sin, nq, nkv, hd)
            kv.append_at(layer, k, v)
            attn = kv.attend_at(layer, q, hd ** -0.5)
        else:
            q, k, v = ops.rope_split(self._linear(h, lw["qkv"]), cos, sin, nq, nkv, hd)
            kv.append(layer, k, v)
            attn = (kv.attend(layer, q, scale=hd ** -0.5) if L == 1
                    else kv.attend_prefill(layer, q, scale=hd ** -0.5))
        o = self._linear(attn.transpose(1, 2).reshape(B, L, nq * hd), lw["o"])
        h = self._norm(x, lw["ln2"], o)
        return self._mlp(h, lw)

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
        L = tokens.shape[1]
        cos, sin = self._rope_tables(torch.arange(offset, offset + L, device=self.device))
        x = self.embed[tokens]
        delta = None
        for layer in range(self.cfg.num_hidden_layers):
            delta = self._block(x, delta, layer, kv, cos, sin)
        x = self._norm(x, self.final_norm, delta)
        if last_only:
            x = x[:, -1:]
        return self._linear(x, self.embed).float()

    # ---- one decode step in a HIP graph ------------------------------------------

    def _graph_step(self, tok: torch.Tensor, nxt: torch.Tensor, kv: PagedKVCache,
                    logits: torch.Tensor | None = None) -> None:
        """One token per sequence from device state only: tok [B, 1] in, the
        greedy next token written to nxt [B] and back into tok, K/V written at
        the cache's device position counter, counters advanced.  Every op is a
        device op with fixed shapes and addresses, so the step can be captured
        and replayed; it computes what ``forward`` computes for one token.
        ``logits`` [B, vocab] fp32, when given, also receives the step's logits."""
        B = tok.shape[0]
        x = self.embed[tok]
        delta = None
        cfg = self.cfg
        if B == 1 and max(cfg.hidden_size, cfg.intermediate_size,
                          cfg.num_attention_heads * cfg.head_dim) <= ops.GEMV_MAX_K:
            # whole RoPE tables (capture_decode's, one row per reserved
            # position, the same elementwise torch ops as _rope_tables): the
            # qkv kernel reads the row of the device position
            cos, sin = self._rope_rows
            spare = torch.empty_like(x)
            for layer in range(cfg.num_hidden_layers):
                delta, x, spare = self._block_token(x, spare, delta, layer, kv, cos, sin)
            if logits is not None:
                logits.copy_(ops.gemv(x, self.embed, ln_weight=self.final_norm,
                                      eps=cfg.rms_norm_eps, delta=delta).reshape(logits.shape))
            # final norm, lm_head and argmax in two launches, no logits stored
            ops.lm_head_argmax(x, self.embed, nxt, token_copy=tok, ln_weight=self.final_norm,
                               eps=cfg.rms_norm_eps, delta=delta)
            kv.step_counters()
            return
        cos, sin = self._rope_tables(kv._pos_dev[:1])
        for layer in range(self.cfg.num_hidden_layers):
            delta = self._block(x, delta, layer, kv, cos, sin, graph=True)
        x = self._norm(x, self.final_norm, delta)
        step_logits = self._linear(x, self.embed).float()
        if logits is not None:
            logits.copy_(step_logits[:, -1])
        nxt.copy_(step_logits[:, -1].argmax(-1))
        tok.copy_(nxt.view(B, 1))
        kv.step_counters()

    @torch.no_grad()
    def capture_decode(self, kv: PagedKVCache, max_len: int,
                       logits: torch.Tensor | None = None):
        """Reserve the cache up to ``max_len`` tokens and capture one decode
        step; returns (graph, tok [B, 1], nxt [B]).  Before each replay put the
        step's input token in ``tok`` (a replay leaves its output there);
        after it call ``kv.advance(1)``.  ``logits`` [B, vocab] fp32, when
        given, receives each replayed step's logits (teacher-forced checks)."""
        kv.reserve(max_len)
        self._rope_rows = self._rope_tables(torch.arange(max(int(max_len), 1),
                                                         device=self.device))
        B = kv._batch
        tok = torch.zeros((B, 1), dtype=torch.long, device=self.device)
        nxt = torch.zeros((B,), dtype=torch.long, device=self.device)
        # one eager run on a side stream sets up the libraries' handles and the
        # workspaces; its K/V write lands at the next position and is
        # overwritten by the first replay, and its counter step is undone
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._graph_step(tok, nxt, kv, logits)
        torch.cuda.current_stream().wait_stream(side)
        kv._counters_dev.sub_(1)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._graph_step(tok, nxt, kv, logits)
        torch.cuda.synchronize()
        # the replays read these tables: they live as long as the graph does,
        # also after a later capture replaces self._rope_rows
        graph.voom_rope_rows = self._rope_rows
        # and the library workspaces the captured launches point into: a later
        # call that grows one replaces it in the cache, and the old buffer
        # must outlive the graph
        graph.voom_workspaces = list(ops._WORKSPACES.values())
        return graph, tok, nxt

    @torch.no_grad()
    def generate_graph(self, prompt: torch.Tensor, max_tokens: int, kv: PagedKVCache):
        """``generate`` with every decode step replayed from one captured HIP
        graph.  Same returns; each per-token time still ends at the token's
        argmax on the host."""
        t0 = time.perf_counter()
        logits = self.forward(prompt.to(self.device), kv, last_only=True)
        first = int(logits[0, -1].argmax())
        prefill_s = time.perf_counter() - t0
        graph, tok, nxt = self.capture_decode(kv, kv.offset + max_tokens)
        out = [first]
        times = []
        tok.fill_(first)
        while len(out) < max_tokens:
            t1 = time.perf_counter()
            graph.replay()
            kv.advance(1)
            out.append(int(nxt[0]))
            times.append(time.perf_counter() - t1)
        return out, prefill_s, times

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
