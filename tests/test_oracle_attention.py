"""Pins the paged decode-attention oracle with closed forms and invariants.

Each case is chosen so that a plausible slip in the restatement fails it:
a wrong scale, a wrong GQA head map, a wrong page order or offset, a dropped
max-subtraction (overflow), or a mis-sliced context.
"""
import numpy as np
import pytest

from oracle import paged_attention as opa


def make_pages(rng, P, NKV, BLOCK, D, scale=1.0):
    k = rng.standard_normal((P, NKV, BLOCK, D)).astype(np.float32) * scale
    v = rng.standard_normal((P, NKV, BLOCK, D)).astype(np.float32)
    return k, v


def test_single_key_returns_its_value_row():
    rng = np.random.default_rng(1)
    k, v = make_pages(rng, 3, 2, 4, 8)
    table = np.array([[2, 0, 1]])
    q = rng.standard_normal((1, 4, 8)).astype(np.float32)
    out = opa.paged_decode(q, k, v, table, np.array([1]), 8 ** -0.5)
    # logical token 0 lives in physical page 2, offset 0
    for h in range(4):
        np.testing.assert_allclose(out[0, h], v[2, h // 2, 0], rtol=0, atol=0)


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(2)
    P, NKV, BLOCK, D = 4, 1, 4, 8
    k = np.broadcast_to(rng.standard_normal(D).astype(np.float32), (P, NKV, BLOCK, D)).copy()
    v = rng.standard_normal((P, NKV, BLOCK, D)).astype(np.float32)
    table = np.array([[3, 1, 0, 2]])
    q = rng.standard_normal((1, 2, D)).astype(np.float32)
    ctx = 11
    out = opa.paged_decode(q, k, v, table, np.array([ctx]), 0.3)
    logical = np.concatenate([v[p, 0] for p in table[0]], axis=0)[:ctx]
    np.testing.assert_allclose(out[0, 0], logical.mean(axis=0), rtol=1e-5, atol=1e-6)


def test_two_keys_logistic_weight_uses_the_scale():
    D = 4
    k = np.zeros((1, 1, 2, D), dtype=np.float32)
    k[0, 0, 0, 0] = 3.0
    k[0, 0, 1, 0] = -1.0
    v = np.zeros((1, 1, 2, D), dtype=np.float32)
    v[0, 0, 0, 1] = 1.0
    v[0, 0, 1, 2] = 1.0
    q = np.zeros((1, 1, D), dtype=np.float32)
    q[0, 0, 0] = 0.5
    scale = 0.7
    out = opa.paged_decode(q, k, v, np.array([[0]]), np.array([2]), scale)
    w = 1.0 / (1.0 + np.exp(-(3.0 * 0.5 - (-1.0) * 0.5) * scale))
    np.testing.assert_allclose(out[0, 0], [0.0, w, 1 - w, 0.0], rtol=1e-6, atol=1e-7)


def test_gqa_head_map_is_h_div_group():
    P, NKV, BLOCK, D, NQ = 2, 4, 4, 8, 12
    k = np.zeros((P, NKV, BLOCK, D), dtype=np.float32)
    v = np.zeros((P, NKV, BLOCK, D), dtype=np.float32)
    for j in range(NKV):
        v[:, j] = j
    q = np.ones((1, NQ, D), dtype=np.float32)
    out = opa.paged_decode(q, k, v, np.array([[1, 0]]), np.array([7]), 1.0)
    for h in range(NQ):
        np.testing.assert_allclose(out[0, h], h // (NQ // NKV))


def test_page_placement_is_invisible():
    rng = np.random.default_rng(3)
    P, NKV, BLOCK, D = 6, 2, 4, 8
    k, v = make_pages(rng, P, NKV, BLOCK, D)
    q = rng.standard_normal((1, 4, D)).astype(np.float32)
    table = np.array([[4, 1, 5, 0]])
    out = opa.paged_decode(q, k, v, table, np.array([14]), 0.35)
    perm = rng.permutation(P)
    inv = np.argsort(perm)
    k2, v2 = k[perm], v[perm]          # physical page perm[i] now sits at slot i
    table2 = inv[table]
    out2 = opa.paged_decode(q, k2, v2, table2, np.array([14]), 0.35)
    np.testing.assert_array_equal(out, out2)


def test_repeated_physical_page_reads_the_same_page_twice():
    # The reference allows a block table like [0, 1, 0] (tests/test_pic_attention.py:52-81).
    rng = np.random.default_rng(4)
    k, v = make_pages(rng, 2, 1, 4, 8)
    q = rng.standard_normal((1, 1, 8)).astype(np.float32)
    out = opa.paged_decode(q, k, v, np.array([[0, 1, 0]]), np.array([12]), 0.35)
    kk = np.concatenate([k[0, 0], k[1, 0], k[0, 0]])
    vv = np.concatenate([v[0, 0], v[1, 0], v[0, 0]])
    s = kk @ q[0, 0] * 0.35
    p = np.exp(s - s.max())
    np.testing.assert_allclose(out[0, 0], p @ vv / p.sum(), rtol=1e-5, atol=1e-6)


def test_large_scores_do_not_overflow():
    rng = np.random.default_rng(5)
    k, v = make_pages(rng, 2, 1, 4, 8, scale=400.0)
    q = rng.standard_normal((1, 1, 8)).astype(np.float32)
    out = opa.paged_decode(q, k, v, np.array([[0, 1]]), np.array([8]), 1.0)
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("ctx", [1, 5, 19, 32, 33])
def test_matches_fp64_brute_force(ctx):
    rng = np.random.default_rng(100 + ctx)
    P, NKV, BLOCK, D, NQ = 12, 2, 4, 16, 6
    k, v = make_pages(rng, P, NKV, BLOCK, D)
    q = rng.standard_normal((1, NQ, D)).astype(np.float32)
    table = rng.permutation(P)[None, :]
    out = opa.paged_decode(q, k, v, table, np.array([ctx]), D ** -0.5)
    # brute force: per head, token by token, in float64
    for h in range(NQ):
        j = h // (NQ // NKV)
        num = np.zeros(D)
        den = 0.0
        scores = []
        for t in range(ctx):
            page, off = table[0, t // BLOCK], t % BLOCK
            scores.append(float(np.dot(k[page, j, off].astype(np.float64), q[0, h])) * D ** -0.5)
        m = max(scores)
        for t in range(ctx):
            page, off = table[0, t // BLOCK], t % BLOCK
            w = np.exp(scores[t] - m)
            num += w * v[page, j, off]
            den += w
        np.testing.assert_allclose(out[0, h], num / den, rtol=1e-5, atol=1e-6)


def test_lse_matches_closed_form_for_equal_scores():
    # all scores equal s0 -> lse = s0 + ln(ctx)
    D = 8
    k = np.zeros((2, 1, 4, D), dtype=np.float32)
    k[..., 0] = 2.0
    v = np.zeros_like(k)
    q = np.zeros((1, 1, D), dtype=np.float32)
    q[0, 0, 0] = 1.5
    lse = opa.paged_decode_lse(q, k, np.array([[1, 0]]), np.array([6]), 0.5)
    np.testing.assert_allclose(lse[0, 0], 2.0 * 1.5 * 0.5 + np.log(6.0), rtol=1e-12)


def test_empty_context_gives_zeros():
    k = np.ones((1, 1, 4, 8), dtype=np.float32)
    out = opa.paged_decode(np.ones((1, 2, 8), np.float32), k, k, np.array([[0]]), np.array([0]), 1.0)
    assert np.all(out == 0)


@pytest.mark.parametrize("ctx", [[1, 5, 19], [32, 33, 0]])
def test_torch_cpu_restatement_matches_fp64_numpy(ctx):
    """The torch-CPU SDPA restatement (the timed CPU baseline) agrees with the
    numpy restatement evaluated in fp64, itself pinned by the brute force
    above: a wrong GQA map or page order in either fails here."""
    import torch

    rng = np.random.default_rng(7 + sum(ctx))
    P, NKV, BLOCK, D, NQ = 16, 2, 4, 16, 8
    k, v = make_pages(rng, P, NKV, BLOCK, D)
    q = rng.standard_normal((3, NQ, D)).astype(np.float32)
    table = np.stack([rng.permutation(P)[:9] for _ in range(3)])
    lens = np.array(ctx)
    ref = opa.paged_decode(q, k, v, table, lens, D ** -0.5, dtype=np.float64)
    got = opa.paged_decode_torch(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                 table, lens, D ** -0.5)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-6)
