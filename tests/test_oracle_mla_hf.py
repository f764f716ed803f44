"""Pins oracle/mla.py's absorbed MLA against Hugging Face's GlmMoeDsaAttention,
an implementation independent of the reference, as the reference's own test
does for its runtime (tests/test_f33_mla_attention.py:85-118, max abs diff
below 1e-4).

HF runs the whole attention block in fp32 with an indexer top-k at least the
sequence length, so its selection mask is a no-op and the block is plain
causal MLA.  The test takes the block's projections, norms and interleaved
RoPE from HF's own submodules (they sit outside the paged path), builds the
latent rows [kv_a_layernorm(c_kv) | rope(k_rot)] and the query halves from
them, and compares the oracle's absorbed attention + o_proj, in fp64, with
HF's output.  A planted mistake (the softmax scale over dn instead of
dn + dr) must fail the same bar."""
import numpy as np
import pytest
import torch

from oracle import mla as omla

transformers = pytest.importorskip("transformers")
hf_mod = pytest.importorskip("transformers.models.glm_moe_dsa.modeling_glm_moe_dsa")


def build_hf_attention(hidden, heads, dn, dr, dv, kv_rank, q_rank, topk, seed, std=None):
    """GlmMoeDsaAttention with random weights: N(0, std) for every parameter
    (the reference test's 0.3), or, with std=None, N(0, 1.5 / sqrt(fan_in))
    for the projections and 1 + N(0, 0.1) for the norm weights."""
    torch.manual_seed(seed)
    cfg = transformers.GlmMoeDsaConfig(
        vocab_size=64, hidden_size=hidden, intermediate_size=64, moe_intermediate_size=16,
        num_hidden_layers=1, first_k_dense_replace=0, num_attention_heads=heads,
        num_key_value_heads=heads, n_shared_experts=1, n_routed_experts=8,
        num_experts_per_tok=2, kv_lora_rank=kv_rank, q_lora_rank=q_rank,
        qk_rope_head_dim=dr, qk_nope_head_dim=dn, v_head_dim=dv, index_topk=topk,
        indexer_types=["full"], attn_implementation="eager", rope_theta=10000.0)
    attn = hf_mod.GlmMoeDsaAttention(cfg, layer_idx=0).eval()
    with torch.no_grad():
        for p in attn.parameters():
            if std is not None:
                p.normal_(mean=0.0, std=std)
            elif p.dim() == 2:
                p.normal_(mean=0.0, std=1.5 / p.shape[1] ** 0.5)
            else:
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
    return attn, hf_mod.GlmMoeDsaRotaryEmbedding(cfg)


def hf_forward_and_latents(attn, rope, h):
    """HF's output [1, S, hidden] and, from the same submodules, q_nope
    [1, H, S, dn], the roped q_rope [1, H, S, dr] and the latent rows
    [1, S, kv_rank + dr]."""
    S = h.shape[1]
    pos = torch.arange(S)[None, :]
    cos, sin = rope(h, pos)
    with torch.no_grad():
        out, _, _ = attn(h, (cos, sin), None, past_key_values=None, position_ids=pos)
        H, dn, dr = attn.num_heads, attn.qk_nope_head_dim, attn.qk_rope_head_dim
        q = attn.q_b_proj(attn.q_a_layernorm(attn.q_a_proj(h)))
        q = q.view(1, S, H, dn + dr).transpose(1, 2)
        q_nope, q_rot = q[..., :dn], q[..., dn:]
        ckv = attn.kv_a_proj_with_mqa(h)
        c = attn.kv_a_layernorm(ckv[..., :attn.kv_lora_rank])
        k_rot = ckv[..., attn.kv_lora_rank:].view(1, 1, S, dr)
        q_rot, k_rot = hf_mod.apply_rotary_pos_emb_interleave(q_rot, k_rot, cos, sin)
        lat = torch.cat([c, k_rot[:, 0]], dim=-1)
    return out, q_nope.contiguous(), q_rot.contiguous(), lat


def oracle_output(attn, q_nope, q_rope, lat, *, scale_mult=1.0):
    kv_b = attn.kv_b_proj.weight.detach().double().numpy()
    o_proj = attn.o_proj.weight.detach().double().numpy()
    heads, _ = omla.absorbed(q_nope.double().numpy(), q_rope.double().numpy(),
                             lat.double().numpy(), kv_b, attn.qk_nope_head_dim,
                             attn.v_head_dim, softmax_scale_mult=scale_mult,
                             dtype=np.float64)
    return omla.project(heads, o_proj)


# (hidden, heads, dn, dr, dv, kv_rank, q_rank, S, std): the reference test's
# geometry and init, then the latent width the HIP kernels take (512 + 64)
CASES = [
    (48, 4, 8, 8, 16, 16, 32, 5, 0.3),
    (48, 4, 8, 8, 16, 16, 32, 23, 0.3),
    (128, 8, 32, 64, 48, 512, 64, 40, None),
]


@pytest.mark.parametrize("hidden,heads,dn,dr,dv,kv_rank,q_rank,S,std", CASES)
def test_absorbed_oracle_matches_hf(hidden, heads, dn, dr, dv, kv_rank, q_rank, S, std):
    attn, rope = build_hf_attention(hidden, heads, dn, dr, dv, kv_rank, q_rank, topk=S + 3,
                                    seed=0, std=std)
    torch.manual_seed(1)
    h = torch.randn(1, S, hidden)
    hf_out, q_nope, q_rope, lat = hf_forward_and_latents(attn, rope, h)
    ref = hf_out.double().numpy()
    got = oracle_output(attn, q_nope, q_rope, lat)
    assert got.shape == ref.shape
    scale = max(1.0, float(np.abs(ref).max()))
    assert np.max(np.abs(got - ref)) < 1e-4 * scale
    # the bar is tight enough to see a scale over dn alone
    wrong = oracle_output(attn, q_nope, q_rope, lat, scale_mult=((dn + dr) / dn) ** 0.5)
    assert np.max(np.abs(wrong - ref)) > 1e-3 * scale
