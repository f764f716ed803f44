"""The HIP absorbed-MLA decode (voom_mla_absorb_query + the latent kernel + the
fused merge and W_UV projection) against Hugging Face's GlmMoeDsaAttention in
fp32, the independent implementation the reference checks its MLA against
(tests/test_f33_mla_attention.py:85-118).

HF computes causal MLA over S = 100 tokens.  The latent rows and query
halves come from HF's own projections, norms and RoPE (outside the paged
path), are rounded to bf16 and go through the kernels: each tested query row
t is a batch entry whose context is the first t + 1 latent rows of a
two-page table (64-token pages).  o_proj runs in fp32 on the host.  Bar:
relative L2 error per output row <= 2e-2 (bf16 inputs and bf16 kernel
outputs; a CPU emulation of the same rounding lands at 0.2-1.0 %)."""
import numpy as np
import pytest
import torch

from test_oracle_mla_hf import build_hf_attention, hf_forward_and_latents

pytestmark = pytest.mark.gpu

H, DN, DR, DV, S, HIDDEN, KV_RANK, Q_RANK, PT = 64, 128, 64, 128, 100, 256, 512, 128, 64
ROWS = [0, 1, 31, 63, 64, 99]


@pytest.mark.parametrize("seed", [3, 9])
def test_absorbed_decode_matches_hf(seed):
    from voom_amd import ops

    attn, rope = build_hf_attention(HIDDEN, H, DN, DR, DV, KV_RANK, Q_RANK, topk=S + 3, seed=seed)
    with torch.no_grad():  # the kernels read bf16 weights: give HF the same values
        for p in (attn.kv_b_proj.weight, attn.o_proj.weight):
            p.copy_(p.to(torch.bfloat16).float())
    torch.manual_seed(seed + 1)
    h = torch.randn(1, S, HIDDEN)
    hf_out, q_nope, q_rope, lat = hf_forward_and_latents(attn, rope, h)

    dev = torch.device("cuda", 0)
    B = len(ROWS)
    pages = (S + PT - 1) // PT
    pool = torch.zeros(pages, PT, KV_RANK + DR, dtype=torch.bfloat16)
    pool.view(-1, KV_RANK + DR)[:S] = lat[0].to(torch.bfloat16)
    table = torch.arange(pages, dtype=torch.int32).repeat(B, 1)
    ctx = torch.tensor([t + 1 for t in ROWS], dtype=torch.int32)
    qn = torch.stack([q_nope[0, :, t] for t in ROWS]).to(torch.bfloat16)  # [B, H, dn]
    qr = torch.stack([q_rope[0, :, t] for t in ROWS]).to(torch.bfloat16)  # [B, H, dr]
    w_uk, w_uv_t = ops.split_kv_b(attn.kv_b_proj.weight.detach().to(torch.bfloat16).to(dev),
                                  H, DN, DV)
    out = ops.mla_absorbed_decode(qn.to(dev), qr.to(dev), pool.to(dev), table.to(dev),
                                  ctx.to(dev), w_uk, w_uv_t, scale=(DN + DR) ** -0.5)
    torch.cuda.synchronize()
    assert out.shape == (B, H, DV)
    y = out.float().cpu().reshape(B, H * DV).double() @ attn.o_proj.weight.detach().double().T
    for i, t in enumerate(ROWS):
        ref = hf_out[0, t].double()
        rel = float(torch.linalg.vector_norm(y[i] - ref) / torch.linalg.vector_norm(ref))
        assert rel <= 2e-2, f"row {t}: relative L2 error {rel:.4f} against HF"
