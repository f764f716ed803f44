"""GPU parity of the absorbed-MLA paged decode against the CPU oracle
(oracle/mla.py, a restatement of runtime/glm.py:78-210).

Tolerance 2e-2 abs / 1e-2 rel on bf16 outputs (fp32 accumulation)."""
import numpy as np
import pytest
import torch

from oracle import mla as omla
from voom_amd import ops, synthetic

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def q_lat_of(inp):
    w_uk, w_uv_t = ops.split_kv_b(inp.kv_b, inp.q_nope.shape[1], inp.dn, inp.dv)
    q_abs = torch.bmm(inp.q_nope.transpose(0, 1).contiguous(), w_uk).transpose(0, 1)
    return torch.cat([q_abs, inp.q_rope], -1).contiguous(), w_uk, w_uv_t


def check_latent(inp, num_ranges=0, batches=None):
    q_lat, _, _ = q_lat_of(inp)
    wc, lse = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                    scale=inp.scale, return_lse=True, num_ranges=num_ranges)
    torch.cuda.synchronize()
    got = wc.float().cpu().numpy()
    ql = q_lat.float().cpu().numpy()
    for b in (batches if batches is not None else range(q_lat.shape[0])):
        lat = synthetic.mla_logical_latent(inp, b)
        ref = omla.absorbed_weighted_c(ql[b:b + 1, :, None, :], lat[None], 64, inp.scale,
                                       bf16=True)[0, :, 0]
        np.testing.assert_allclose(got[b], ref, atol=ATOL, rtol=RTOL)
        s = (ql[b].astype(np.float64) @ lat.T.astype(np.float64)) * inp.scale
        m = s.max(axis=1)
        ref_lse = m + np.log(np.exp(s - m[:, None]).sum(axis=1))
        np.testing.assert_allclose(lse[b].cpu().numpy(), ref_lse, atol=1e-2, rtol=1e-3)
    return wc


@pytest.mark.parametrize("ctx", [[1, 64], [63, 65, 200], [300, 1000]])
def test_latent_contraction_small(ctx):
    print(f"[mla] latent ctx={ctx}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=len(ctx), heads=32, ctx_lens=ctx, slack_pages=3)
    check_latent(inp)


@pytest.mark.parametrize("ctx", [[1, 64], [63, 65, 200], [300, 1000, 4097]])
def test_latent_contraction_small_128_heads(ctx):
    print(f"[mla] latent 128 heads ctx={ctx}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=len(ctx), heads=128, ctx_lens=ctx, slack_pages=2)
    check_latent(inp)


@pytest.mark.parametrize("nr", [1, 3, 8, 40])
def test_range_splits_agree_128_heads(nr):
    print(f"[mla] 128 heads ranges={nr}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=128, ctx_lens=[777, 2048])
    check_latent(inp, num_ranges=nr)


@pytest.mark.parametrize("heads", [64, 128])
@pytest.mark.parametrize("jump", [[(0, 40), (1, 250)], [(0, 700 - 3), (1, 130)]])
def test_restart_after_a_late_jump(heads, jump):
    # Latent rows scaled so that the scores of a few tokens sit far more than
    # 2^64 (log2 units) above the first tile's: the kernel keeps the first
    # tile's maximum as the softmax reference and starts a range over when a
    # later score exceeds it by that much.  Token 40 lies in the first tile
    # of sequence 0, 697 in its last tile, 250 and 130 in later tiles of
    # sequence 1.
    print(f"[mla] restart heads={heads} jump={jump}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=heads, ctx_lens=[700, 300])
    lat = inp.lat_pool
    lat.mul_(0.05)
    for b, tok in jump:
        slot = int(inp.table_host[b, tok // 64])
        lat[slot, tok % 64] *= 2000.0
    q_lat, _, _ = q_lat_of(inp)
    ql = q_lat.float().cpu().numpy()
    for nr in (1, 3):
        wc, lse = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                        scale=inp.scale, return_lse=True, num_ranges=nr)
        torch.cuda.synchronize()
        got = wc.float().cpu().numpy()
        for b in range(2):
            lat_b = synthetic.mla_logical_latent(inp, b)
            ref = omla.absorbed_weighted_c(ql[b:b + 1, :, None, :], lat_b[None], 64, inp.scale,
                                           bf16=True)[0, :, 0]
            # the jump rows put outputs in the hundreds: the bar is taken
            # relative to each sequence's largest output
            top = float(np.abs(ref).max())
            np.testing.assert_allclose(got[b] / top, ref / top, atol=ATOL, rtol=0)
            s_ = (ql[b].astype(np.float64) @ lat_b.T.astype(np.float64)) * inp.scale
            m = s_.max(axis=1)
            ref_lse = m + np.log(np.exp(s_ - m[:, None]).sum(axis=1))
            np.testing.assert_allclose(lse[b].cpu().numpy(), ref_lse, atol=1e-2, rtol=1e-3)


@pytest.mark.parametrize("shifts", [(20, 0, 24, -2), (-24, 0, -30, 6)])
@pytest.mark.parametrize("heads", [64, 128])
def test_quarters_of_very_different_magnitude(heads, shifts):
    # The fp16 range partials of 64-head groups scale each 128-dim quarter of
    # a row by its own power of two (largest magnitude in [2^14, 2^15)).
    # Latent quarters scaled by powers of two, with q scaled by the inverse (a
    # power-of-two scale of a bf16 value is exact, so the scores do not
    # change), put the outputs of some quarters far past the fp16 range
    # (2^20, 2^24) or far below its normal range (2^-24, 2^-30, where fp16
    # holds at most a few bits); each quarter is checked relative to its own
    # scale.
    print(f"[mla] quarter magnitudes heads={heads} shifts={shifts}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=heads, ctx_lens=[333, 1500])
    q_lat, _, _ = q_lat_of(inp)
    for qi, sh in enumerate(shifts):
        inp.lat_pool[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** sh
        q_lat[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** -sh
    ql = q_lat.float().cpu().numpy()
    refs = []
    for b in range(2):
        lat_b = synthetic.mla_logical_latent(inp, b)
        refs.append(omla.absorbed_weighted_c(ql[b:b + 1, :, None, :], lat_b[None], 64,
                                             inp.scale, bf16=True)[0, :, 0])
    for qi, sh in enumerate(shifts):
        top = float(np.abs(refs[1][:, 128 * qi:128 * (qi + 1)]).max())
        if sh >= 20:
            assert top > 2.0 ** 16  # past the fp16 range
        if sh <= -24:
            assert top < 2.0 ** -14  # below fp16's smallest normal
    for nr in (1, 3, 16):
        wc = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                   scale=inp.scale, num_ranges=nr)
        torch.cuda.synchronize()
        got = wc.float().cpu().numpy()
        for b in range(2):
            for qi, sh in enumerate(shifts):
                sl = slice(128 * qi, 128 * (qi + 1))
                np.testing.assert_allclose(got[b][:, sl] * 2.0 ** -sh, refs[b][:, sl] * 2.0 ** -sh,
                                           atol=ATOL, rtol=RTOL)


def test_seeded_sweep_of_shapes_and_quarter_magnitudes():
    """25 seeded cases: 1-3 sequences of 1-3,000 tokens, 64 or 128 heads,
    pages of 64-256 tokens, 0 (default), 1, 3, 16 or 40 ranges, and each
    latent quarter scaled by its own power of two in 2^-30 .. 2^24 (q by the
    inverse); every quarter checked against the oracle at its own scale."""
    rng = np.random.default_rng(777)
    for case in range(25):
        B = int(rng.integers(1, 4))
        H = int(rng.choice([64, 128]))
        pt = int(rng.choice([64, 128, 256]))
        ctx = [int(x) for x in rng.integers(1, 3000, size=B)]
        nr = int(rng.choice([0, 1, 3, 16, 40]))
        print(f"[mla] sweep case {case}: B={B} H={H} pt={pt} nr={nr}", flush=True)
        inp = synthetic.mla_decode_inputs(batch=B, heads=H, ctx_lens=ctx, page_tokens=pt,
                                          slack_pages=1, seed=int(rng.integers(0, 1 << 30)))
        q_lat, _, _ = q_lat_of(inp)
        shifts = [int(x) for x in rng.integers(-30, 25, size=4)]
        for qi, sh in enumerate(shifts):
            inp.lat_pool[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** sh
            q_lat[..., 128 * qi:128 * (qi + 1)] *= 2.0 ** -sh
        wc = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                   scale=inp.scale, num_ranges=nr)
        torch.cuda.synchronize()
        got = wc.float().cpu().numpy()
        ql = q_lat.float().cpu().numpy()
        for b in range(B):
            lat = synthetic.mla_logical_latent(inp, b)
            ref = omla.absorbed_weighted_c(ql[b:b + 1, :, None, :], lat[None], 64, inp.scale,
                                           bf16=True)[0, :, 0]
            for qi, sh in enumerate(shifts):
                sl = slice(128 * qi, 128 * (qi + 1))
                np.testing.assert_allclose(got[b][:, sl] * 2.0 ** -sh, ref[:, sl] * 2.0 ** -sh,
                                           atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("nr", [1, 3, 8])
def test_range_splits_agree(nr):
    print(f"[mla] ranges={nr}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=64, ctx_lens=[777, 2048])
    check_latent(inp, num_ranges=nr)


@pytest.mark.parametrize("pt", [64, 128, 256])
def test_page_sizes(pt):
    print(f"[mla] page_tokens={pt}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=32, ctx_lens=[pt + 5, 3 * pt],
                                      page_tokens=pt)
    check_latent(inp)


def test_full_pipeline_matches_absorbed_and_expanded_oracles():
    print("[mla] full absorbed pipeline", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=32, ctx_lens=[500, 130])
    w_uk, w_uv_t = ops.split_kv_b(inp.kv_b, 32, inp.dn, inp.dv)
    out = ops.mla_absorbed_decode(inp.q_nope, inp.q_rope, inp.lat_pool, inp.block_table,
                                  inp.ctx_lens, w_uk, w_uv_t, scale=inp.scale)
    torch.cuda.synchronize()
    kv_b = inp.kv_b.float().cpu().numpy()
    for b in range(2):
        lat = synthetic.mla_logical_latent(inp, b)
        qn = inp.q_nope[b:b + 1, :, None].float().cpu().numpy()
        qr = inp.q_rope[b:b + 1, :, None].float().cpu().numpy()
        S = lat.shape[0]
        ref_bf, _ = omla.absorbed(qn, qr, lat[None], kv_b, inp.dn, inp.dv, offset=S - 1,
                                  bf16=True)
        ref_exp = omla.expanded(qn, qr, lat[None, :, :512], lat[None, :, 512:], kv_b, inp.dn,
                                inp.dv, offset=S - 1)
        got = out[b].float().cpu().numpy()
        np.testing.assert_allclose(got, ref_bf[0, :, 0], atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(got, ref_exp[0, :, 0], atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("heads,ctx", [(64, [500, 130, 64]), (128, [1000, 1])])
def test_fused_merge_and_projection(heads, ctx):
    """64-head groups: the merge of the range partials and weighted_c . W_UV in
    one launch give the bits of the two-launch path and match the oracles."""
    print(f"[mla] fused merge + projection H={heads} ctx={ctx}", flush=True)
    inp = synthetic.mla_decode_inputs(batch=len(ctx), heads=heads, ctx_lens=ctx)
    w_uk, w_uv_t = ops.split_kv_b(inp.kv_b, heads, inp.dn, inp.dv)
    q_lat = ops.mla_absorb_query(inp.q_nope, inp.q_rope, ops.pack_head_weights(w_uk))
    y, wc, lse = ops.mla_latent_decode_project(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                               w_uv_t, scale=inp.scale, return_weighted_c=True,
                                               return_lse=True)
    wc2, lse2 = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                      scale=inp.scale, return_lse=True)
    y2 = ops.mla_project_out(wc2, w_uv_t)
    out = ops.mla_absorbed_decode(inp.q_nope, inp.q_rope, inp.lat_pool, inp.block_table,
                                  inp.ctx_lens, w_uk, w_uv_t, scale=inp.scale)
    torch.cuda.synchronize()
    assert torch.equal(wc.view(torch.int16), wc2.view(torch.int16))
    assert torch.equal(lse, lse2)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(out.view(torch.int16), y.view(torch.int16))
    kv_b = inp.kv_b.float().cpu().numpy()
    for b in range(len(ctx)):
        lat = synthetic.mla_logical_latent(inp, b)
        qn = inp.q_nope[b:b + 1, :, None].float().cpu().numpy()
        qr = inp.q_rope[b:b + 1, :, None].float().cpu().numpy()
        S = lat.shape[0]
        ref_bf, _ = omla.absorbed(qn, qr, lat[None], kv_b, inp.dn, inp.dv, offset=S - 1,
                                  bf16=True)
        np.testing.assert_allclose(y[b].float().cpu().numpy(), ref_bf[0, :, 0], atol=ATOL,
                                   rtol=RTOL)


@pytest.mark.parametrize("heads", [32, 64, 128])
def test_empty_sequences_give_zeros(heads):
    """A sequence with no cached tokens gets a zero row and a log-sum-exp of
    -inf, as in the GQA kernels; the other rows of the batch match the oracle.
    Dense (default and 3 ranges), merge + projection in one launch (64-head
    groups) and the sparse contraction with a selection of length 0 alike."""
    print(f"[mla] empty sequences H={heads}", flush=True)
    ctx = [0, 300, 0, 65]
    inp = synthetic.mla_decode_inputs(batch=4, heads=heads, ctx_lens=ctx, slack_pages=2)
    q_lat, _, w_uv_t = q_lat_of(inp)
    ql = q_lat.float().cpu().numpy()
    refs = {b: omla.absorbed_weighted_c(ql[b:b + 1, :, None, :],
                                        synthetic.mla_logical_latent(inp, b)[None], 64, inp.scale,
                                        bf16=True)[0, :, 0] for b in (1, 3)}
    sel = torch.arange(max(ctx), dtype=torch.int32, device="cuda").repeat(4, 1).contiguous()
    for nr in (0, 3):
        wc, lse = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                                        scale=inp.scale, return_lse=True, num_ranges=nr)
        sp, lse_s = ops.mla_sparse_decode(q_lat, inp.lat_pool, inp.block_table, sel,
                                          inp.ctx_lens, scale=inp.scale, return_lse=True,
                                          num_ranges=nr)
        torch.cuda.synchronize()
        for out, l in ((wc, lse), (sp, lse_s)):
            for b in (0, 2):
                assert bool((out[b] == 0).all()), f"row {b} not zero (nr={nr})"
                assert bool(torch.isneginf(l[b]).all()), f"lse {b} not -inf (nr={nr})"
            got = out.float().cpu().numpy()
            for b in (1, 3):
                np.testing.assert_allclose(got[b], refs[b], atol=ATOL, rtol=RTOL)
        if heads % 64 == 0:
            y, wc2 = ops.mla_latent_decode_project(q_lat, inp.lat_pool, inp.block_table,
                                                   inp.ctx_lens, w_uv_t, scale=inp.scale,
                                                   num_ranges=nr, return_weighted_c=True)
            y2 = ops.mla_project_out(wc, w_uv_t)
            torch.cuda.synchronize()
            assert torch.equal(wc2.view(torch.int16), wc.view(torch.int16))
            assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
            assert bool((y[0] == 0).all()) and bool((y[2] == 0).all())


def test_paging_invariance_is_bitwise():
    print("[mla] paging invariance", flush=True)
    inp = synthetic.mla_decode_inputs(batch=2, heads=32, ctx_lens=[700, 333], slack_pages=7)
    q_lat, _, _ = q_lat_of(inp)
    a = ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                              scale=inp.scale)
    slots = inp.lat_pool.shape[0]
    perm = torch.from_numpy(np.random.default_rng(5).permutation(slots)).cuda()
    inv = torch.argsort(perm)
    pool2 = inp.lat_pool[perm].contiguous()
    table2 = inv[inp.block_table.long()].to(torch.int32).contiguous()
    b2 = ops.mla_latent_decode(q_lat, pool2, table2, inp.ctx_lens, scale=inp.scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b2)


def test_config5_full_size_every_sequence():
    print("[mla] config 5 full size", flush=True)
    inp = synthetic.mla_decode_inputs()
    check_latent(inp)


@pytest.mark.parametrize("B,H,K,N", [(8, 128, 128, 512), (8, 128, 512, 128), (3, 5, 40, 64),
                                     (16, 4, 512, 512), (1, 2, 1, 8), (9, 3, 100, 256),
                                     (2, 3, 64, 24), (5, 7, 1000, 40)])
def test_head_gemv_is_the_fp32_per_head_product_rounded(B, H, K, N):
    print(f"[mla] head_gemv B={B} H={H} K={K} N={N}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(B * 1000 + H + K + N)
    x = torch.randn((B, H, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((H, K, N), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    got = ops.head_gemv(x, w)
    # fp32 reference on the CPU (exact products, float64 sums)
    exact = torch.bmm(x.double().cpu().transpose(0, 1), w.double().cpu()).transpose(0, 1)
    scale = torch.bmm(x.double().cpu().abs().transpose(0, 1),
                      w.double().cpu().abs()).transpose(0, 1)
    torch.cuda.synchronize()
    err = (got.double().cpu() - exact).abs()
    assert got.shape == (B, H, N)
    assert bool((err <= exact.abs() * 2.0 ** -8 + scale * 1e-6).all())


def test_head_gemv_writes_into_a_wider_row_and_rejects_bad_shapes():
    x = torch.randn((2, 3, 64), device="cuda").to(torch.bfloat16)
    w = torch.randn((3, 64, 32), device="cuda").to(torch.bfloat16)
    out = torch.full((2, 3, 48), 7.0, dtype=torch.bfloat16, device="cuda")
    ops.head_gemv(x, w, out=out)
    ref = ops.head_gemv(x, w)
    torch.cuda.synchronize()
    assert torch.equal(out[..., :32].view(torch.int16), ref.view(torch.int16))
    assert bool((out[..., 32:] == 7.0).all())
    # weights packed once give the same bits as weights packed per call
    packed = ops.pack_head_weights(w)
    again = ops.head_gemv(x, packed)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(ValueError):
        ops.head_gemv(torch.zeros((17, 3, 64), dtype=torch.bfloat16, device="cuda"), w)
    with pytest.raises(ValueError):
        ops.head_gemv(x, torch.zeros((3, 48, 32), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        ops.head_gemv(x[:, :2], packed)
