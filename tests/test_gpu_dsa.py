"""GPU parity of the DSA selection kernels and the sparse absorbed-MLA
contraction against oracle/dsa.py and oracle/mla.py (runtime/glm_dsa.py:
113-166 and runtime/glm.py:280-289 restated).

* index scores: fp32, within 1e-5 relative + 1e-5 absolute of the oracle
  (the bf16 products are exact in fp32; only the summation order differs);
* top-k: bit-exact against the oracle's top-k of the same scores (index
  sets, ascending order, lowest indices among ties);
* end to end: the GPU selection differs from the oracle's only by keys whose
  scores lie within the score tolerance of the k-th score;
* sparse MLA: 2e-2 abs / 1e-2 rel in bf16, as the dense MLA tests; over all
  positions it equals the dense kernel bit for bit."""
import numpy as np
import pytest
import torch

from oracle import dsa as odsa
from oracle import mla as omla
from voom_amd import _lib, ops, synthetic

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _index_inputs(B, NH, cap, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, NH, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    w = (torch.randn((B, NH), generator=g) * NH ** -0.5).float()
    return q, k, w


@pytest.mark.parametrize("B,NH,cap,lens", [(1, 32, 7000, [7000]), (3, 16, 1200, [1, 517, 1200]),
                                           (2, 64, 3000, [2048, 2049]), (1, 48, 70000, [69999])])
def test_index_scores_match_oracle(B, NH, cap, lens):
    print(f"[dsa] scores B={B} NH={NH} cap={cap}", flush=True)
    q, k, w = _index_inputs(B, NH, cap, seed=NH + cap)
    ln = torch.tensor(lens, dtype=torch.int32)
    out = torch.full((B, cap), -7.0, dtype=torch.float32, device="cuda")
    ops.dsa_index_scores(q.cuda(), w.cuda(), k.cuda(), ln.cuda(), scale=128 ** -0.5, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(B):
        n = lens[b]
        ref = odsa.index_scores(q[b].float().numpy(), w[b].numpy(), k[b, :n].float().numpy(),
                                128 ** -0.5)
        np.testing.assert_allclose(got[b, :n], ref, rtol=1e-5, atol=1e-5)
        assert np.all(got[b, n:] == -7.0)          # past lens untouched


def _check_topk(scores_np, lens, k):
    sc = torch.from_numpy(scores_np).cuda()
    ln = torch.tensor(lens, dtype=torch.int32, device="cuda")
    sel, sl = ops.dsa_topk(sc, ln, k)
    torch.cuda.synchronize()
    sel, sl = sel.cpu().numpy(), sl.cpu().numpy()
    for b, n in enumerate(lens):
        want = odsa.topk(scores_np[b], n, k)
        assert sl[b] == len(want)
        assert sel[b, :sl[b]].tolist() == want.tolist(), f"row {b} n={n} k={k}"


@pytest.mark.parametrize("n,k", [(131072, 2048), (4097, 2048), (5000, 1), (3000, 2999),
                                 (2048, 2048), (100, 2048), (65536, 64)])
def test_topk_exact(n, k):
    print(f"[dsa] topk n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k)
    s = rng.standard_normal((2, n)).astype(np.float32) * 3
    _check_topk(s, [n, max(1, n // 2)], k)


@pytest.mark.parametrize("n", [40000, 131072, 200000, 500000, 600000])
def test_topk_chunk_layouts_and_concentrated_candidates(n):
    # Rows of 10, 32, 49, 123 and 147 chunks of 4096 keys (candidates in
    # 256-slot segments per wavefront up to 128 chunks, one segment per chunk
    # above).  Row 0: random scores, candidates spread over every segment;
    # row 1: ascending scores, so that every candidate sits in the last
    # chunks and every other segment is empty.
    print(f"[dsa] topk chunk layouts n={n}", flush=True)
    rng = np.random.default_rng(n)
    s = np.stack([rng.standard_normal(n), np.sort(rng.standard_normal(n))]).astype(np.float32)
    _check_topk(s, [n, n], 2048)


def test_topk_sample_misplaced_threshold_falls_back_to_memory():
    # The threshold comes from runs of 4 keys every n / 1024 positions.  Row 0
    # puts the row's highest keys exactly there, so the threshold leaves
    # fewer than k keys above it; row 1 ties 20,000 keys at the maximum, so
    # more than 16,384 candidates pass it.  Both take the exact select over
    # the row in memory and must still match the oracle bit for bit.
    print("[dsa] topk memory fallback", flush=True)
    n, k = 131072, 2048
    rng = np.random.default_rng(11)
    row0 = rng.standard_normal(n).astype(np.float32)
    runs = (np.arange(1024, dtype=np.int64) * n // 1024) & ~3
    for d in range(4):
        row0[runs + d] = 100.0 + rng.random(1024).astype(np.float32)
    row1 = rng.standard_normal(n).astype(np.float32)
    row1[rng.choice(n, 20000, replace=False)] = 50.0
    _check_topk(np.stack([row0, row1]), [n, n], k)


def test_topk_seeded_sweep_across_the_segment_layouts():
    """40 seeded batches: rows up to 700,000 keys (either side of the
    128-chunk bound between per-wavefront segments and per-chunk packing),
    k from 1 to 8,192, batches of 1-4 rows of mixed lengths, and score
    distributions with wide and narrow ranges, ties, sorted runs, infinities
    and signed zeros; every row bit-exact against the oracle."""
    rng = np.random.default_rng(4242)
    for case in range(40):
        B = int(rng.integers(1, 5))
        cap = int(rng.choice([3000, 20000, 131072, 262144, 530000, 700000]))
        k = int(rng.choice([1, 64, 1000, 2048, 4096, 8192]))
        lens = [int(x) for x in rng.integers(1, cap + 1, size=B)]
        lens[int(rng.integers(0, B))] = cap
        rows = []
        for _ in range(B):
            kind = int(rng.integers(0, 6))
            if kind == 0:
                r = rng.standard_normal(cap) * 10.0 ** rng.uniform(-3, 3)
            elif kind == 1:
                r = np.round(rng.standard_normal(cap) * 3)
            elif kind == 2:
                r = rng.exponential(1.0, cap) + 1e4
            elif kind == 3:
                r = np.sort(rng.standard_normal(cap))[::(1 if rng.random() < 0.5 else -1)].copy()
            elif kind == 4:
                r = rng.standard_normal(cap)
                r[rng.integers(0, cap, 50)] = np.inf
                r[rng.integers(0, cap, 50)] = -np.inf
            else:
                r = (np.where(rng.random(cap) < 0.5, 0.0, -0.0) +
                     (rng.random(cap) < 0.001) * rng.standard_normal(cap))
            rows.append(r.astype(np.float32))
        print(f"[dsa] sweep case {case}: B={B} cap={cap} k={k}", flush=True)
        _check_topk(np.stack(rows), lens, k)


def test_topk_ties_negative_and_special_values():
    print("[dsa] topk ties", flush=True)
    rng = np.random.default_rng(7)
    n = 20000
    rows = [
        np.round(rng.standard_normal(n) * 2).astype(np.float32),      # heavy ties
        np.full(n, 1.5, np.float32),                                   # all equal
        -np.abs(rng.standard_normal(n)).astype(np.float32),            # all negative
        np.where(rng.random(n) < 0.5, 0.0, -0.0).astype(np.float32),  # signed zeros
    ]
    rows[0][123] = np.inf
    rows[2][5] = -np.inf
    _check_topk(np.stack(rows), [n, n, n, n], 2048)


def test_selection_end_to_end_against_oracle():
    print("[dsa] select end to end", flush=True)
    q, k, w = _index_inputs(1, 32, 40000, seed=99)
    n, K = 40000, 2048
    ln = torch.tensor([n], dtype=torch.int32, device="cuda")
    sc = ops.dsa_index_scores(q.cuda(), w.cuda(), k.cuda(), ln, scale=128 ** -0.5)
    sel, _ = ops.dsa_topk(sc, ln, K)
    torch.cuda.synchronize()
    ref_sc = odsa.index_scores(q[0].float().numpy(), w[0].numpy(), k[0].float().numpy(),
                               128 ** -0.5)
    ref = set(odsa.topk(ref_sc, n, K).tolist())
    got = set(sel[0].cpu().numpy().tolist())
    kth = np.sort(ref_sc)[::-1][K - 1]
    for i in got ^ ref:
        assert abs(ref_sc[i] - kth) <= 1e-5 * abs(kth) + 1e-5, (i, ref_sc[i], kth)
    assert len(got) == K


def _q_lat(inp):
    w_uk, _ = ops.split_kv_b(inp.kv_b, inp.q_nope.shape[1], inp.dn, inp.dv)
    q_abs = torch.bmm(inp.q_nope.transpose(0, 1).contiguous(), w_uk).transpose(0, 1)
    return torch.cat([q_abs, inp.q_rope], -1).contiguous()


@pytest.mark.parametrize("nr", [10, 16, 40])
@pytest.mark.parametrize("scaled", [False, True])
def test_sparse_over_all_positions_equals_dense(nr, scaled):
    """Same range split (so the same rounding), same rows: bit for bit.
    scaled: latent quarters times 2^20, 1, 2^24, 2^-2 (q times the inverse),
    so that the fp16 range partials of some quarters carry exponents."""
    print(f"[dsa] sparse == dense nr={nr} scaled={scaled}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=64, ctx_lens=[1000, 2500], slack_pages=2)
    q = _q_lat(inp)
    if scaled:
        for qi, sh in enumerate((20, 0, 24, -2)):
            inp.lat_pool[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** sh
            q[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** -sh
    dense, lse_d = ops.mla_latent_decode(q, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                         scale=inp.scale, return_lse=True, num_ranges=nr)
    sel = torch.arange(2500, dtype=torch.int32, device="cuda").repeat(2, 1).contiguous()
    sparse, lse_s = ops.mla_sparse_decode(q, inp.lat_pool, inp.block_table, sel, inp.ctx_lens,
                                          scale=inp.scale, return_lse=True, num_ranges=nr)
    torch.cuda.synchronize()
    assert torch.equal(dense, sparse)
    assert torch.equal(lse_d, lse_s)


@pytest.mark.parametrize("heads,pt,k", [(128, 64, 2048), (32, 128, 300), (64, 256, 1)])
def test_sparse_selection_matches_oracle(heads, pt, k):
    print(f"[dsa] sparse heads={heads} pt={pt} k={k}", flush=True)
    ctx = [5000, 3001]
    inp = synthetic.mla_decode_inputs(batch=2, heads=heads, ctx_lens=ctx, page_tokens=pt,
                                      slack_pages=3)
    q = _q_lat(inp)
    rng = np.random.default_rng(k + pt)
    sel_np = np.zeros((2, k), dtype=np.int32)
    lens = []
    for b, c in enumerate(ctx):
        m = min(k, c) if b == 0 else max(1, min(k, c) // 2)   # second row: a short selection
        sel_np[b, :m] = np.sort(rng.choice(c, size=m, replace=False))
        lens.append(m)
    sel = torch.from_numpy(sel_np).cuda()
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    wc = ops.mla_sparse_decode(q, inp.lat_pool, inp.block_table, sel, sl, scale=inp.scale)
    torch.cuda.synchronize()
    got = wc.float().cpu().numpy()
    ql = q.float().cpu().numpy()
    for b in range(2):
        lat = odsa.gather(synthetic.mla_logical_latent(inp, b), sel_np[b, :lens[b]])
        ref = omla.absorbed_weighted_c(ql[b:b + 1, :, None, :], lat[None], 64, inp.scale,
                                       bf16=True)[0, :, 0]
        np.testing.assert_allclose(got[b], ref, atol=ATOL, rtol=RTOL)


def test_sparse_validation():
    inp = synthetic.mla_decode_inputs(batch=1, heads=32, ctx_lens=[100])
    q = _q_lat(inp)
    sel = torch.zeros((1, 8), dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError):
        ops.mla_sparse_decode(q, inp.lat_pool, inp.block_table, sel, inp.ctx_lens, scale=1.0)
    with pytest.raises(ValueError):
        ops.dsa_topk(torch.zeros((1, 8), device="cuda"), torch.ones(1, dtype=torch.int32,
                                                                     device="cuda"), 0)
    # a range may hold at most four 64-row tiles: 600 positions need 3 ranges
    sel = torch.zeros((1, 600), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="ranges"):
        ops.mla_sparse_decode(q, inp.lat_pool, inp.block_table, sel, inp.ctx_lens, scale=1.0,
                              num_ranges=2)


def test_dsa_state_selects_like_the_oracle():
    """DSAState over a growing index-key cache (observe on prefill and decode,
    update_and_select past index_topk, shared-layer reuse, trim)."""
    from voom_amd.dsa import DSAState, index_keys, index_queries
    print("[dsa] DSAState end to end", flush=True)
    g = torch.Generator().manual_seed(12)
    HID, QL, NH, HD, DR, TOPK = 256, 64, 32, 128, 64, 256

    def rnd(*shape, std=0.05):
        return (torch.randn(shape, generator=g) * std).to(torch.bfloat16).cuda()

    w = {"l.self_attn.indexer.wq_b.weight": rnd(NH * HD, QL),
         "l.self_attn.indexer.wk.weight": rnd(HD, HID),
         "l.self_attn.indexer.k_norm.weight": (1 + rnd(HD).float()).to(torch.bfloat16),
         "l.self_attn.indexer.k_norm.bias": rnd(HD),
         "l.self_attn.indexer.weights_proj.weight": rnd(NH, HID)}
    st = DSAState(index_topk=TOPK, index_n_heads=NH, index_head_dim=HD, qk_rope_head_dim=DR,
                  rope_theta=10000.0)
    S = 1500
    h = rnd(1, S, HID, std=1.0)
    st.observe(0, "full", h[:, :200], w, "l", offset=0)
    st.observe(0, "full", h[:, 200:], w, "l", offset=200)
    q_a = rnd(1, 1, QL, std=1.0)
    h1 = rnd(1, 1, HID, std=1.0)
    st.observe(0, "full", h1, w, "l", offset=S)
    sel = st.update_and_select(0, "full", h1, q_a, w, "l", offset=S)
    torch.cuda.synchronize()
    assert sel.shape == (1, 1, TOPK) and st.stats["sparse_selects"] >= 1
    assert st.update_and_select(1, "shared", h1, q_a, w, "l", offset=S) is sel

    k_all = index_keys(torch.cat([h, h1], 1), w, "l", 0, rope_dims=DR, theta=10000.0)
    assert torch.equal(st.keys(0), k_all)           # chunked observe == one pass
    q_idx, w_head = index_queries(q_a, h1, w, "l", S, n_heads=NH, head_dim=HD, rope_dims=DR,
                                  theta=10000.0)
    ref_sc = odsa.index_scores(q_idx[0, 0].float().cpu().numpy(), w_head[0, 0].cpu().numpy(),
                               k_all[0].float().cpu().numpy(), HD ** -0.5)
    ref = set(odsa.topk(ref_sc, S + 1, TOPK).tolist())
    got = set(sel[0, 0].cpu().numpy().tolist())
    kth = np.sort(ref_sc)[::-1][TOPK - 1]
    for i in got ^ ref:
        assert abs(ref_sc[i] - kth) <= 1e-5 * abs(kth) + 1e-5
    st.trim(1000)
    assert st.keys(0).shape[1] == 1000 and st.selection is None


@pytest.mark.parametrize("budget_pages", [None, 3])
def test_attend_mla_with_selection_matches_oracle(budget_pages):
    """PagedKVCache.attend_mla(selection=...) -- the DSA gather feeding absorbed
    MLA -- over resident and spilled latent pages."""
    from voom_amd.kv_paged import PagedKVCache
    print(f"[dsa] attend_mla selection budget_pages={budget_pages}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(21)
    B, H, dn, dv, C, dr, PT, S, K = 1, 32, 128, 128, 512, 64, 64, 3000, 700
    kv_b = (torch.randn((H * (dn + dv), C), generator=gen, device="cuda") * C ** -0.5
            ).to(torch.bfloat16)
    w_uk, w_uv_t = ops.split_kv_b(kv_b, H, dn, dv)
    page_bytes = B * (C + dr) * 2 * PT
    max_bytes = 1 << 40 if budget_pages is None else budget_pages * page_bytes
    kv = PagedKVCache(num_layers=1, max_bytes=max_bytes, page_positions=PT, resident_pages=1)
    lat = torch.randn((B, S, C + dr), generator=gen, device="cuda").to(torch.bfloat16)
    kv.append_latent(0, lat)
    if budget_pages is not None:
        assert any(not p.resident for p in kv._pages[0])
    rng = np.random.default_rng(4)
    sel_np = np.sort(rng.choice(S, size=K, replace=False)).astype(np.int32)
    sel = torch.from_numpy(sel_np)[None, None].cuda()            # (B, L=1, k), as DSAState
    q_nope = torch.randn((B, H, dn), generator=gen, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn((B, H, dr), generator=gen, device="cuda").to(torch.bfloat16)
    out, wc = kv.attend_mla(0, q_nope, q_rope, w_uk, w_uv_t, (dn + dr) ** -0.5,
                            return_weighted_c=True, selection=sel)
    torch.cuda.synchronize()
    ref_out, ref_wc = omla.absorbed(
        q_nope.float().cpu().numpy()[:, :, None], q_rope.float().cpu().numpy()[:, :, None],
        lat.float().cpu().numpy()[:, sel_np], kv_b.float().cpu().numpy(), dn, dv, bf16=True)
    np.testing.assert_allclose(wc.float().cpu().numpy(), ref_wc[:, :, 0], atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_out[:, :, 0], atol=ATOL, rtol=RTOL)
    kv.release()


def test_topk_random_rows_lengths_and_distributions():
    """Seeded sweep over the three selection paths (every key a candidate,
    the sampled threshold, the in-memory fallback): row lengths from 1 to
    140,000 within one batch, k from 1 to 4,096, and score distributions with
    wide and narrow ranges, heavy ties, infinities and signed zeros; every row
    bit-exact against the oracle."""
    rng = np.random.default_rng(2027)
    for case in range(6):
        k = int(rng.choice([1, 7, 64, 2048, 3000, 4096]))
        cap = int(rng.choice([5000, 20000, 140000]))
        lens = [int(x) for x in rng.integers(1, cap + 1, size=4)]
        lens[0] = cap
        rows = []
        for b in range(4):
            kind = int(rng.integers(0, 5))
            if kind == 0:
                r = rng.standard_normal(cap) * 10.0 ** rng.uniform(-3, 3)
            elif kind == 1:
                r = np.round(rng.standard_normal(cap) * 4)               # heavy ties
            elif kind == 2:
                r = rng.exponential(1.0, cap) + 1e4                     # narrow relative range
            elif kind == 3:
                r = np.where(rng.random(cap) < 0.3, 0.0, -0.0) + (rng.random(cap) < 0.01)
            else:
                r = rng.standard_normal(cap)
                r[rng.integers(0, cap, 5)] = np.inf
                r[rng.integers(0, cap, 5)] = -np.inf
            rows.append(r.astype(np.float32))
        print(f"[dsa] random case {case}: k={k} cap={cap} lens={lens}", flush=True)
        _check_topk(np.stack(rows), lens, k)


def test_topk_workspace_counters_return_to_zero():
    """The top-k is one launch: the chunk workgroups of a row count their
    arrival in the workspace and the last one selects.  The counters must be
    zero again after every call (the next call relies on it), whatever the
    rows: many rows per call, rows on each of the three paths (every key
    selected, every key a candidate, the sampled threshold), and calls of
    different batch sizes back to back on the same workspace."""
    print("[dsa] topk counters", flush=True)
    rng = np.random.default_rng(404)
    cap, k = 70000, 512
    need = _lib.lib().voom_dsa_topk_workspace_bytes(16, cap)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    for B in (16, 3, 16, 1):
        lens = [int(x) for x in rng.integers(1, cap + 1, size=B)]
        lens[0] = cap
        if B > 2:
            lens[1], lens[2] = 300, 9000          # every key selected; every key a candidate
        scores = (rng.standard_normal((B, cap)) * 2).astype(np.float32)
        sc = torch.from_numpy(scores).cuda()
        ln = torch.tensor(lens, dtype=torch.int32, device="cuda")
        sel = torch.empty((B, k), dtype=torch.int32, device="cuda")
        sl = torch.empty((B,), dtype=torch.int32, device="cuda")
        for _ in range(2):
            _lib.call("voom_dsa_topk", sc.data_ptr(), ln.data_ptr(), sel.data_ptr(),
                          sl.data_ptr(), ws.data_ptr(), need, B, cap, k,
                          torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            assert int(ws[:4 * 16].view(torch.int32).abs().sum()) == 0, "counters left non-zero"
        got, got_l = sel.cpu().numpy(), sl.cpu().numpy()
        for b in range(B):
            want = odsa.topk(scores[b], lens[b], k)
            assert got_l[b] == len(want)
            assert got[b, :got_l[b]].tolist() == want.tolist(), (B, b, lens[b])
