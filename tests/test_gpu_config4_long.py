"""Config 4 at its stated size: one sequence of 131072 tokens at the 32B-class
GQA shape (64 q heads, 8 KV heads, head_dim 128) in 64-token pages, the oldest
40 % of the pages spilled to pinned host memory; three decode steps of
append + attend, each reloading the spilled pages on the side stream while
the resident pages are attended (the reference reloads every spilled page on
every call, runtime/kv_paged.py:164-171), against the CPU oracle's
concatenate-then-SDPA restatement at 2e-2 abs / 1e-2 rel."""
import numpy as np
import pytest
import torch

from oracle import paged_attention as opa
from voom_amd import synthetic
from voom_amd.kv_paged import PagedKVCache

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def test_config4_full_size_attend_with_40pct_spilled():
    NQ, NKV, D, PT, S = 64, 8, 128, 64, 131072
    print("[config4] building a 131072-token sequence", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(9)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 62, page_positions=PT, resident_pages=1,
                      initial_slots=S // PT + 8)
    pos = torch.arange(S, device="cuda")
    ks, vs = [], []
    chunk = 16384
    for c0 in range(0, S, chunk):
        kr = torch.randn((1, NKV, chunk, D), generator=gen, device="cuda")
        cos, sin = synthetic.rope_tables(pos[c0:c0 + chunk], D, 5e5)
        k = synthetic.apply_rope_neox(kr, cos, sin).to(torch.bfloat16)
        v = torch.randn((1, NKV, chunk, D), generator=gen, device="cuda").to(torch.bfloat16)
        kv.append(0, k, v)
        ks.append(k)
        vs.append(v)
    n_spill = int(0.4 * (S // PT))
    assert n_spill == 819
    kv.arena.reserve(n_spill * kv.page_nbytes + (16 << 20))
    assert kv.spill([(0, i) for i in range(n_spill)]) == n_spill
    assert sum(not p.resident for p in kv._pages[0]) == n_spill
    k_all = torch.cat(ks, 2)[0].cpu()
    v_all = torch.cat(vs, 2)[0].cpu()
    del ks, vs
    for step in range(3):
        q = torch.randn((1, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
        nk = torch.randn((1, NKV, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
        nv = torch.randn((1, NKV, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
        kv.append(0, nk, nv)
        out = kv.attend(0, q)
        torch.cuda.synchronize()
        print(f"[config4] step {step}: {kv.offset} tokens, {n_spill} pages reloaded", flush=True)
        k_all = torch.cat([k_all, nk[0].cpu()], 1)
        v_all = torch.cat([v_all, nv[0].cpu()], 1)
        ref = opa.sdpa_decode_torch(q[0, :, 0].cpu(), k_all, v_all, D ** -0.5).numpy()
        np.testing.assert_allclose(out[0, :, 0].float().cpu().numpy(), ref, atol=ATOL,
                                   rtol=RTOL)
    assert all(not kv._pages[0][i].resident for i in range(n_spill))
    assert kv.stats.reloads == 3 * n_spill
    kv.release()
    torch.cuda.empty_cache()
