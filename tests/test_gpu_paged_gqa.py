"""GPU parity of voom_paged_gqa_decode against the CPU oracle.

Tolerance: 2e-2 abs / 1e-2 rel on bf16 outputs (fp32 accumulation), the
north-star bar and the reference's own bf16 tolerance for its paged kernel
(tests/test_pic_attention.py:48).
"""
import numpy as np
import pytest
import torch

from oracle import paged_attention as opa
from voom_amd import ops, synthetic
from voom_amd.page_pool import v_pages_to_tokens, v_tokens_to_pages

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def run_case(name, **kw):
    print(f"[gqa] case {name} {kw}", flush=True)
    splits = kw.pop("num_splits", None)
    inp = synthetic.gqa_decode_inputs(device="cuda", **kw)
    out, lse = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table,
                                    inp.ctx_lens, scale=inp.scale, return_lse=True,
                                    num_splits=splits)
    torch.cuda.synchronize()
    q, k, v = synthetic.to_reference_layout(inp)
    ref = opa.paged_decode(q, k, v, inp.table_host, inp.ctx_host, inp.scale)
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
    ref_lse = opa.paged_decode_lse(q, k, inp.table_host, inp.ctx_host, inp.scale)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)
    return inp, out


@pytest.mark.parametrize("D,NQ,NKV", [(128, 8, 2), (128, 32, 8), (128, 64, 8), (64, 9, 3),
                                      (128, 16, 1), (64, 4, 4)])
def test_small_ragged_matches_oracle(D, NQ, NKV):
    run_case(f"ragged D={D} NQ={NQ} NKV={NKV}", batch=4, ctx_lens=[1, 19, 64, 300],
             num_q_heads=NQ, num_kv_heads=NKV, head_dim=D, page_tokens=64, slack_pages=5)


@pytest.mark.parametrize("PT", [32, 64, 128, 256])
def test_page_sizes(PT):
    run_case(f"page_tokens={PT}", batch=3, ctx_lens=[PT - 1, PT, 5 * PT + 7],
             num_q_heads=32, num_kv_heads=8, head_dim=128, page_tokens=PT, slack_pages=2)


@pytest.mark.parametrize("splits", [1, 2, 7, 64, 1000])
def test_split_counts_agree(splits):
    run_case(f"splits={splits}", batch=5, ctx_lens=[33, 1000, 2049, 70, 4000],
             num_q_heads=32, num_kv_heads=8, head_dim=128, page_tokens=64, num_splits=splits)


@pytest.mark.parametrize("D,splits", [(128, 96), (64, 5)])
def test_partials_then_combine_is_the_decode_bitwise(D, splits):
    # with an explicit split count the decode is exactly the two halves
    print(f"[gqa] case partials+combine D={D} splits={splits}", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=3, ctx_lens=[0, 700, 2500], num_q_heads=16,
                                      num_kv_heads=4, head_dim=D, device="cuda")
    whole, lse = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table,
                                      inp.ctx_lens, scale=inp.scale, return_lse=True,
                                      num_splits=splits)
    n = splits
    ws = torch.empty(ops.gqa_workspace_bytes(3, 16, 4, D, n), dtype=torch.uint8, device="cuda")
    ops.paged_gqa_partials(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens,
                           scale=inp.scale, num_splits=n, ws=ws)
    out = torch.empty_like(inp.q)
    lse2 = torch.empty_like(lse)
    ops.paged_gqa_combine(inp.ctx_lens, out, ws, num_kv_heads=4, page_tokens=64,
                          max_pages=inp.block_table.shape[1], num_splits=n, lse=lse2)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), whole.view(torch.int16))
    assert torch.equal(lse2, lse)


@pytest.mark.parametrize("D,G", [(128, 4), (64, 3), (128, 16)])
def test_short_tables_take_the_segment_kernel_and_match(D, G):
    # a block table of <= 1024 tokens with the default split count runs one
    # workgroup per (sequence, kv head); it must agree with the oracle and with
    # split-K (same math, another merge order), LSE included, empty rows zero
    print(f"[gqa] case segment kernel D={D} G={G}", flush=True)
    NKV = 2 if G == 16 else 4
    inp = synthetic.gqa_decode_inputs(batch=4, ctx_lens=[0, 1, 700, 1000], num_q_heads=NKV * G,
                                      num_kv_heads=NKV, head_dim=D, device="cuda")
    assert inp.block_table.shape[1] * 64 <= 1024
    seg, lse_s = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table,
                                      inp.ctx_lens, scale=inp.scale, return_lse=True)
    spl, lse_k = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table,
                                      inp.ctx_lens, scale=inp.scale, return_lse=True,
                                      num_splits=64)
    torch.cuda.synchronize()
    q, k, v = synthetic.to_reference_layout(inp)
    ref = opa.paged_decode(q, k, v, inp.table_host, inp.ctx_host, inp.scale)
    np.testing.assert_allclose(seg.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(seg.float().cpu().numpy(), spl.float().cpu().numpy(),
                               atol=ATOL, rtol=RTOL)
    assert torch.equal(seg[0], torch.zeros_like(seg[0]))
    assert bool(torch.isneginf(lse_s[0]).all())
    # fp32 normalisers summed in another order: a few 1e-5 relative apart
    torch.testing.assert_close(lse_s[1:], lse_k[1:], rtol=1e-4, atol=1e-4)


def test_empty_sequence_gives_zeros():
    print("[gqa] case empty sequence", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=3, ctx_lens=[0, 40, 0], num_q_heads=8,
                                      num_kv_heads=2, head_dim=128, device="cuda")
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    torch.cuda.synchronize()
    assert torch.all(out[0] == 0) and torch.all(out[2] == 0)
    q, k, v = synthetic.to_reference_layout(inp)
    ref = opa.paged_decode(q, k, v, inp.table_host, inp.ctx_host, inp.scale)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_single_token_context_returns_value_row_exactly():
    print("[gqa] case ctx=1 exact", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=2, ctx_lens=[1, 1], num_q_heads=8, num_kv_heads=2,
                                      head_dim=128, device="cuda")
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    torch.cuda.synchronize()
    for b in range(2):
        slot = int(inp.table_host[b, 0])
        for h in range(8):
            assert torch.equal(out[b, h], v_pages_to_tokens(inp.v_pool[slot:slot + 1])[0, h // 4, 0])


def test_nan_garbage_past_context_is_ignored():
    print("[gqa] case NaN past context", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=2, ctx_lens=[70, 100], num_q_heads=8,
                                      num_kv_heads=2, head_dim=128, device="cuda")
    ref = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens).clone()
    for b, ctx in enumerate(inp.ctx_host):
        last = int(inp.table_host[b, (ctx - 1) // 64])
        off = int(ctx % 64)
        inp.k_pool[last, :, off:, :] = float("nan")
        vt = v_pages_to_tokens(inp.v_pool[last:last + 1]).clone()
        vt[:, :, off:] = float("nan")
        inp.v_pool[last:last + 1] = v_tokens_to_pages(vt)
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_paging_invariance_is_bitwise():
    print("[gqa] case paging invariance", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=4, ctx_lens=[500, 64, 1300, 77], num_q_heads=32,
                                      num_kv_heads=8, head_dim=128, slack_pages=9, device="cuda")
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    slots = inp.k_pool.shape[0]
    perm = torch.from_numpy(np.random.default_rng(11).permutation(slots)).cuda()
    inv = torch.argsort(perm)
    k2 = inp.k_pool[perm].contiguous()
    v2 = inp.v_pool[perm].contiguous()
    table2 = inv[inp.block_table.long()].to(torch.int32).contiguous()
    out2 = ops.paged_gqa_decode(inp.q, k2, v2, table2, inp.ctx_lens)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_repeated_physical_pages():
    print("[gqa] case repeated page ids", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=1, ctx_lens=[192], num_q_heads=8, num_kv_heads=2,
                                      head_dim=128, device="cuda")
    table = torch.tensor([[1, 2, 1]], dtype=torch.int32, device="cuda")
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, table, inp.ctx_lens)
    torch.cuda.synchronize()
    q, k, v = synthetic.to_reference_layout(inp)
    ref = opa.paged_decode(q, k, v, table.cpu().numpy(), inp.ctx_host, inp.scale)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_outlier_keys_stay_stable():
    print("[gqa] case outlier keys", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=2, ctx_lens=[900, 2000], num_q_heads=32,
                                      num_kv_heads=8, head_dim=128, device="cuda")
    inp.k_pool[..., :4] *= 20
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    torch.cuda.synchronize()
    q, k, v = synthetic.to_reference_layout(inp)
    ref = opa.paged_decode(q, k, v, inp.table_host, inp.ctx_host, inp.scale)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_merge_states_equals_full_attention():
    print("[gqa] case LSE merge", flush=True)
    inp = synthetic.gqa_decode_inputs(batch=2, ctx_lens=[640, 1280], num_q_heads=32,
                                      num_kv_heads=8, head_dim=128, device="cuda")
    full = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens)
    # split each sequence's pages into first half / second half
    half = [int(c) // 128 for c in inp.ctx_host]
    tab = inp.table_host
    t1 = np.zeros_like(tab)
    t2 = np.zeros_like(tab)
    c1, c2 = [], []
    for b in range(2):
        n = -(-int(inp.ctx_host[b]) // 64)
        t1[b, :half[b]] = tab[b, :half[b]]
        t2[b, :n - half[b]] = tab[b, half[b]:n]
        c1.append(half[b] * 64)
        c2.append(int(inp.ctx_host[b]) - half[b] * 64)
    T1, T2 = torch.from_numpy(t1).cuda(), torch.from_numpy(t2).cuda()
    C1 = torch.tensor(c1, dtype=torch.int32, device="cuda")
    C2 = torch.tensor(c2, dtype=torch.int32, device="cuda")
    o1, l1 = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, T1, C1, return_lse=True)
    o2, l2 = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, T2, C2, return_lse=True)
    merged, _ = ops.merge_attn_states(o1, l1, o2, l2)
    torch.cuda.synchronize()
    np.testing.assert_allclose(merged.float().cpu().numpy(), full.float().cpu().numpy(),
                               atol=ATOL, rtol=RTOL)


def test_config2_full_size_matches_oracle_on_every_sequence():
    print("[gqa] case config-2 full size", flush=True)
    inp = synthetic.gqa_decode_inputs(device="cuda")
    out = ops.paged_gqa_decode(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens,
                               scale=inp.scale)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for b in range(inp.q.shape[0]):
        slots = inp.table_host[b, : -(-int(inp.ctx_host[b]) // 64)]
        idx = torch.from_numpy(slots.astype(np.int64)).cuda()
        k = inp.k_pool[idx].float().cpu().numpy()
        v = v_pages_to_tokens(inp.v_pool[idx]).float().cpu().numpy()
        table = np.arange(len(slots))[None]
        q = inp.q[b:b + 1].float().cpu().numpy()
        ref = opa.paged_decode(q, k, v, table, inp.ctx_host[b:b + 1], inp.scale)
        np.testing.assert_allclose(got[b:b + 1], ref, atol=ATOL, rtol=RTOL)
