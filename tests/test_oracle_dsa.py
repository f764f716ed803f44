"""Pins oracle/dsa.py (runtime/glm_dsa.py:113-166 restated) and the host-side
indexer projections of voom_amd/dsa.py:
  * against Hugging Face's GlmMoeDsaIndexer -- an independent implementation,
    the one the reference's own test compares with (tests/test_f33_dsa_
    indexer.py) -- on seeded small configurations: the oracle's selection
    computed from voom_amd.dsa's projections equals HF's;
  * the top-k against a full sort (distinct scores), the tie rule and the
    n <= k case;
  * a single head with unit weight ranks keys by relu(q . k)."""
import numpy as np
import pytest
import torch

from oracle import dsa as odsa
from voom_amd import dsa as vdsa

transformers = pytest.importorskip("transformers")
hf_mod = pytest.importorskip("transformers.models.glm_moe_dsa.modeling_glm_moe_dsa")

HIDDEN, Q_LORA, DR, NH, HD = 48, 32, 8, 32, 128


def _hf_indexer(seed: int, topk: int):
    torch.manual_seed(seed)
    cfg = transformers.GlmMoeDsaConfig(
        vocab_size=64, hidden_size=HIDDEN, intermediate_size=64, moe_intermediate_size=16,
        num_hidden_layers=1, first_k_dense_replace=0, num_attention_heads=4,
        num_key_value_heads=4, n_shared_experts=1, n_routed_experts=8, num_experts_per_tok=2,
        kv_lora_rank=16, q_lora_rank=Q_LORA, qk_rope_head_dim=DR, qk_nope_head_dim=8,
        v_head_dim=16, index_topk=topk, index_n_heads=NH, index_head_dim=HD,
        indexer_types=["full"], attn_implementation="eager", rope_theta=10000.0)
    ind = hf_mod.GlmMoeDsaIndexer(cfg, layer_idx=0).eval()
    with torch.no_grad():
        for p in ind.parameters():
            p.normal_(mean=0.0, std=0.3)
    rope = hf_mod.GlmMoeDsaRotaryEmbedding(cfg)
    q_a = torch.nn.Linear(HIDDEN, Q_LORA, bias=False)
    q_norm = hf_mod.GlmMoeDsaRMSNorm(Q_LORA)
    with torch.no_grad():
        q_a.weight.normal_(mean=0.0, std=0.3)
    return ind, rope, q_a, q_norm


@pytest.mark.parametrize("seed,S,topk", [(2, 7, 4), (5, 7, 4), (11, 40, 8), (17, 96, 16)])
def test_selection_matches_hf_indexer(seed, S, topk):
    ind, rope, q_a, q_norm = _hf_indexer(seed, topk)
    torch.manual_seed(1000 + seed)
    h = torch.randn(1, S, HIDDEN)
    pos = torch.arange(S)[None, :]
    cos, sin = rope(h, pos)
    with torch.no_grad():
        q_resid = q_norm(q_a(h))
        hf = ind(h, q_resid, (cos, sin), None, pos, past_key_values=None)
    hf_last = sorted(int(i) for i in hf[0, -1].tolist())

    sd = ind.state_dict()
    w = {f"l.self_attn.indexer.{k}": v for k, v in sd.items()}
    with torch.no_grad():
        k_all = vdsa.index_keys(h, w, "l", 0, rope_dims=DR, theta=10000.0)       # [1, S, HD]
        q_idx, w_head = vdsa.index_queries(q_resid[:, -1:], h[:, -1:], w, "l", S - 1,
                                           n_heads=NH, head_dim=HD, rope_dims=DR,
                                           theta=10000.0)
    sel = odsa.select(q_idx[0, 0].numpy(), w_head[0, 0].numpy(), k_all[0].numpy(), S, topk,
                      HD ** -0.5)
    assert sel.tolist() == hf_last


def test_topk_equals_full_sort_for_distinct_scores():
    rng = np.random.default_rng(0)
    s = rng.permutation(5000).astype(np.float32) * np.float32(0.37) - 900
    for n, k in [(5000, 2048), (3000, 1), (4097, 4096)]:
        want = np.sort(np.argsort(-s[:n], kind="stable")[:k])
        assert odsa.topk(s, n, k).tolist() == want.tolist()


def test_topk_ties_keep_lowest_indices_and_short_rows_keep_all():
    s = np.array([1, 5, 5, 2, 5, 5, 0], dtype=np.float32)
    assert odsa.topk(s, 7, 3).tolist() == [1, 2, 4]
    assert odsa.topk(s, 7, 1).tolist() == [1]
    assert odsa.topk(s, 4, 8).tolist() == [0, 1, 2, 3]
    assert odsa.topk(s, 7, 7).tolist() == list(range(7))


def test_single_head_ranks_by_relu_dot():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 16)).astype(np.float32)
    k = rng.standard_normal((200, 16)).astype(np.float32)
    sc = odsa.index_scores(q, np.ones(1, np.float32), k, 1.0)
    dots = (k @ q[0]).astype(np.float32)
    np.testing.assert_allclose(sc, np.maximum(dots, 0), rtol=1e-6, atol=1e-6)
    pos = np.flatnonzero(dots > 0)
    want = np.sort(pos[np.argsort(-dots[pos])][:10])
    assert odsa.topk(sc, 200, 10).tolist() == want.tolist()


def test_torch_cpu_selection_matches_numpy_for_distinct_scores():
    """The torch-CPU selection (the timed CPU baseline) equals the pinned numpy
    selection when no two scores tie."""
    import torch

    from oracle import dsa as odsa

    rng = np.random.default_rng(9)
    q = rng.standard_normal((8, 64)).astype(np.float32)
    w = rng.standard_normal(8).astype(np.float32)
    k = rng.standard_normal((3000, 64)).astype(np.float32)
    ref = odsa.select(q, w, k, 3000, 256, 0.125)
    got = odsa.select_torch(torch.from_numpy(q), torch.from_numpy(w), torch.from_numpy(k), 256,
                            0.125)
    assert np.array_equal(got.numpy(), ref)
