"""GPU numerics of the decoder-block HIP kernels against plain PyTorch fp32
references of the same ops (Hugging Face Llama's formulas and cast order):
RoPE + split bit-exact (each product and sum rounded as torch rounds them);
RMSNorm and SwiGLU within one bf16 ulp (the fp32 reduction order and exp
implementation may differ)."""
import pytest
import torch
import torch.nn.functional as F

from voom_amd import ops

pytestmark = pytest.mark.gpu


def ulp_close(a: torch.Tensor, b: torch.Tensor, ulps: int = 1) -> None:
    ai = a.view(torch.int16).int()
    bi = b.view(torch.int16).int()
    # bf16 bit patterns of the same sign differ by the ulp count
    same_sign = (ai < 0) == (bi < 0)
    diff = (ai - bi).abs()
    bad = ~(same_sign & (diff <= ulps)) & (a.float() != b.float())
    assert not bool(bad.any()), f"{int(bad.sum())} values beyond {ulps} ulp"


@pytest.mark.parametrize("rows,H,with_delta", [(1, 576, True), (37, 576, False), (5, 4096, True)])
def test_add_rms_norm(rows, H, with_delta):
    print(f"[decoder-ops] rms rows={rows} H={H}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + H)
    x = torch.randn((rows, H), generator=g, device="cuda").to(torch.bfloat16)
    d = torch.randn((rows, H), generator=g, device="cuda").to(torch.bfloat16) if with_delta else None
    w = (1 + 0.1 * torch.randn((H,), generator=g, device="cuda")).to(torch.bfloat16)
    x_ref = x + d if with_delta else x.clone()
    xf = x_ref.float()
    ref = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16)
    got = ops.add_rms_norm(x, w, 1e-5, delta=d)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), x_ref.view(torch.int16))   # residual exact
    ulp_close(got, ref)


@pytest.mark.parametrize("B,L,nq,nkv,hd", [(1, 1, 9, 3, 64), (2, 33, 9, 3, 64), (1, 5, 32, 8, 128)])
def test_rope_split_is_the_torch_rotation(B, L, nq, nkv, hd):
    print(f"[decoder-ops] rope B={B} L={L}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(B * L + hd)
    qkv = torch.randn((B, L, (nq + 2 * nkv) * hd), generator=g, device="cuda").to(torch.bfloat16)
    pos = torch.arange(100, 100 + L, device="cuda")
    inv = 1.0 / (10000.0 ** (torch.arange(hd // 2, device="cuda", dtype=torch.float32) / (hd // 2)))
    ang = pos.float()[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1).contiguous()
    sin = torch.cat([ang.sin(), ang.sin()], -1).contiguous()
    q, k, v = ops.rope_split(qkv, cos, sin, nq, nkv, hd)
    torch.cuda.synchronize()

    def rope(x):  # x [B, H, L, hd]
        xf = x.float()
        rot = torch.cat([-xf[..., hd // 2:], xf[..., :hd // 2]], -1)
        return (xf * cos + rot * sin).to(x.dtype)

    qr, kr, vr = qkv.split([nq * hd, nkv * hd, nkv * hd], -1)
    assert torch.equal(q, rope(qr.reshape(B, L, nq, hd).transpose(1, 2)))
    assert torch.equal(k, rope(kr.reshape(B, L, nkv, hd).transpose(1, 2)))
    assert torch.equal(v, vr.reshape(B, L, nkv, hd).transpose(1, 2))


@pytest.mark.parametrize("rows,inter", [(1, 1536), (40, 1536), (3, 14336)])
def test_silu_mul(rows, inter):
    print(f"[decoder-ops] silu rows={rows}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + inter)
    gu = (torch.randn((rows, 2 * inter), generator=g, device="cuda") * 3).to(torch.bfloat16)
    gate, up = gu.chunk(2, dim=-1)
    ref = F.silu(gate) * up
    got = ops.silu_mul(gu)
    torch.cuda.synchronize()
    ulp_close(got, ref)


@pytest.mark.parametrize("n,k", [(1, 8), (5, 576), (960, 576), (576, 1536), (3072, 576),
                                 (7, 2048), (130, 520), (49152, 576)])
def test_gemv_is_the_fp32_product_rounded(n, k):
    # fp32 sums in a different order than the reference: within bf16 rounding of
    # the exact product, plus a term for cancellation near zero
    print(f"[decoder-ops] gemv n={n} k={k}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n * 7 + k)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    x = torch.randn((1, 1, k), generator=g, device="cuda").to(torch.bfloat16)
    got = ops.gemv(x, w)
    torch.cuda.synchronize()
    assert got.shape == (1, 1, n) and got.dtype == torch.bfloat16
    exact = (w.double() @ x.reshape(k).double())
    scale = (w.double().abs() @ x.reshape(k).double().abs())
    err = (got.reshape(n).double() - exact).abs()
    assert bool((err <= exact.abs() * 2.0 ** -8 + scale * 1e-6).all())


@pytest.mark.parametrize("inter,k", [(1, 8), (3, 576), (1536, 576), (7, 1544)])
def test_gemv_swiglu_is_projection_then_silu_mul(inter, k):
    print(f"[decoder-ops] gemv swiglu I={inter} k={k}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(inter * 3 + k)
    w = (torch.randn((2 * inter, k), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((k,), generator=g, device="cuda").to(torch.bfloat16)
    got = ops.gemv(x, w, swiglu=True)
    # the unfused path: projection rounded to bf16, then silu_mul's math
    gu = (w.float() @ x.float()).to(torch.bfloat16)
    ref = F.silu(gu[:inter]) * gu[inter:]
    torch.cuda.synchronize()
    assert got.shape == (inter,)
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=2e-3)


def test_gemv_rejects_unsupported_shapes():
    w = torch.zeros((4, 576), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.gemv(torch.zeros((2, 576), dtype=torch.bfloat16, device="cuda"), w)  # two rows
    with pytest.raises(ValueError):
        ops.gemv(torch.zeros((4096,), dtype=torch.bfloat16, device="cuda"),
                 torch.zeros((4, 4096), dtype=torch.bfloat16, device="cuda"))  # K too large
    with pytest.raises(ValueError):
        ops.gemv(torch.zeros((12,), dtype=torch.bfloat16, device="cuda"),
                 torch.zeros((4, 12), dtype=torch.bfloat16, device="cuda"))  # K % 8


@pytest.mark.parametrize("nq,nkv,hd,K,PT,pos", [(9, 3, 64, 576, 64, 100), (32, 8, 128, 2048, 32, 63),
                                                (4, 4, 64, 520, 64, 0), (6, 2, 64, 576, 16, 47)])
def test_qkv_rope_append_is_the_three_ops_bitwise(nq, nkv, hd, K, PT, pos):
    # the fused decode-token path against gemv -> rope_split -> append_kv
    from voom_amd.page_pool import v_slot_shape
    print(f"[decoder-ops] qkv_rope_append nq={nq} nkv={nkv} hd={hd} K={K} PT={PT} pos={pos}",
          flush=True)
    g = torch.Generator(device="cuda").manual_seed(nq + hd + K + pos)
    N = (nq + 2 * nkv) * hd
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((1, 1, K), generator=g, device="cuda").to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(hd // 2, device="cuda", dtype=torch.float32) / (hd // 2)))
    ang = pos * inv
    cos = torch.cat([ang.cos(), ang.cos()]).reshape(1, hd).contiguous()
    sin = torch.cat([ang.sin(), ang.sin()]).reshape(1, hd).contiguous()
    slots = 4
    table = torch.tensor([[2, 0, 3, 1]], dtype=torch.int32, device="cuda")
    position = torch.tensor([pos], dtype=torch.int32, device="cuda")
    kp = [torch.zeros((slots, nkv, PT, hd), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    vp = [torch.zeros((slots,) + v_slot_shape(nkv, hd, PT), dtype=torch.bfloat16, device="cuda")
          for _ in range(2)]
    q1 = ops.qkv_rope_append(x, w, cos, sin, kp[0], vp[0], table, position, nq, nkv, hd)
    q2, k2, v2 = ops.rope_split(ops.gemv(x, w), cos, sin, nq, nkv, hd)
    ops.append_kv(k2, v2, kp[1], vp[1], table, position)
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kp[0].view(torch.int16), kp[1].view(torch.int16))
    assert torch.equal(vp[0].view(torch.int16), vp[1].view(torch.int16))
    assert bool(kp[0].abs().sum() > 0) and bool(vp[0].abs().sum() > 0)


@pytest.mark.parametrize("n,k,swiglu,with_delta", [(960, 576, False, True), (1536, 576, True, True),
                                                   (7, 2048, False, False), (3, 1544, True, True),
                                                   (130, 8, False, True), (49152, 576, False, True)])
def test_norm_prologue_gemv_is_add_rms_norm_then_gemv_bitwise(n, k, swiglu, with_delta):
    # the residual-add + RMSNorm folded into the projection against the two ops
    print(f"[decoder-ops] norm gemv n={n} k={k} swiglu={swiglu} delta={with_delta}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n + 3 * k + int(swiglu))
    rows = 2 * n if swiglu else n
    w = (torch.randn((rows, k), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((1, 1, k), generator=g, device="cuda").to(torch.bfloat16)
    d = torch.randn((1, 1, k), generator=g, device="cuda").to(torch.bfloat16) if with_delta else None
    ln = (1 + 0.1 * torch.randn((k,), generator=g, device="cuda")).to(torch.bfloat16)
    x_before = x.clone()
    x_out = torch.full_like(x, 7.0) if with_delta else None
    got = ops.gemv(x, w, swiglu=swiglu, ln_weight=ln, eps=1e-5, delta=d, x_out=x_out)
    resid = x.clone()
    h = ops.add_rms_norm(resid, ln, 1e-5, delta=d)
    ref = ops.gemv(h, w, swiglu=swiglu)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(x.view(torch.int16), x_before.view(torch.int16))   # input untouched
    if with_delta:
        assert torch.equal(x_out.view(torch.int16), resid.view(torch.int16))


@pytest.mark.parametrize("nq,nkv,hd,K,PT,pos", [(9, 3, 64, 576, 64, 100), (32, 8, 128, 2048, 32, 63)])
def test_qkv_rope_append_norm_prologue_is_add_rms_norm_first_bitwise(nq, nkv, hd, K, PT, pos):
    from voom_amd.page_pool import v_slot_shape
    print(f"[decoder-ops] norm qkv_rope_append nq={nq} hd={hd} K={K}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(nq * hd + K)
    N = (nq + 2 * nkv) * hd
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((1, 1, K), generator=g, device="cuda").to(torch.bfloat16)
    d = torch.randn((1, 1, K), generator=g, device="cuda").to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn((K,), generator=g, device="cuda")).to(torch.bfloat16)
    ang = pos / (10000.0 ** (torch.arange(hd // 2, device="cuda", dtype=torch.float32) / (hd // 2)))
    cos = torch.cat([ang.cos(), ang.cos()]).reshape(1, hd).contiguous()
    sin = torch.cat([ang.sin(), ang.sin()]).reshape(1, hd).contiguous()
    table = torch.tensor([[2, 0, 3, 1]], dtype=torch.int32, device="cuda")
    position = torch.tensor([pos], dtype=torch.int32, device="cuda")
    kp = [torch.zeros((4, nkv, PT, hd), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    vp = [torch.zeros((4,) + v_slot_shape(nkv, hd, PT), dtype=torch.bfloat16, device="cuda")
          for _ in range(2)]
    x_out = torch.empty_like(x)
    q1 = ops.qkv_rope_append(x, w, cos, sin, kp[0], vp[0], table, position, nq, nkv, hd,
                             ln_weight=ln, eps=1e-5, delta=d, x_out=x_out)
    resid = x.clone()
    h = ops.add_rms_norm(resid, ln, 1e-5, delta=d)
    q2 = ops.qkv_rope_append(h, w, cos, sin, kp[1], vp[1], table, position, nq, nkv, hd)
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kp[0].view(torch.int16), kp[1].view(torch.int16))
    assert torch.equal(vp[0].view(torch.int16), vp[1].view(torch.int16))
    assert torch.equal(x_out.view(torch.int16), resid.view(torch.int16))


def test_norm_prologue_rejects_aliased_residual_output():
    x = torch.zeros((1, 1, 576), dtype=torch.bfloat16, device="cuda")
    d = torch.zeros_like(x)
    w = torch.zeros((4, 576), dtype=torch.bfloat16, device="cuda")
    ln = torch.ones((576,), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.gemv(x, w, ln_weight=ln, delta=d, x_out=x)
    with pytest.raises(ValueError):
        ops.gemv(x, w, delta=d)   # delta without ln_weight


@pytest.mark.parametrize("n,k,with_norm", [(49152, 576, True), (1003, 8, False), (5, 2048, True)])
def test_lm_head_argmax_is_torch_argmax_of_the_gemv_logits(n, k, with_norm):
    print(f"[decoder-ops] lm_head_argmax n={n} k={k} norm={with_norm}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((1, 1, k), generator=g, device="cuda").to(torch.bfloat16)
    d = torch.randn((1, 1, k), generator=g, device="cuda").to(torch.bfloat16) if with_norm else None
    ln = (1 + 0.1 * torch.randn((k,), generator=g, device="cuda")).to(torch.bfloat16) if with_norm else None
    tok = torch.full((1,), -1, dtype=torch.int64, device="cuda")
    tok2 = torch.full((1, 1), -1, dtype=torch.int64, device="cuda")
    ops.lm_head_argmax(x, w, tok, token_copy=tok2, ln_weight=ln, eps=1e-5, delta=d)
    h = ops.add_rms_norm(x.clone(), ln, 1e-5, delta=d) if with_norm else x
    ref = ops.gemv(h, w).float().reshape(n).argmax()
    torch.cuda.synchronize()
    assert int(tok[0]) == int(ref) == int(tok2[0, 0])


def test_lm_head_argmax_takes_the_lowest_index_among_ties():
    n, k = 4096, 64
    w = torch.zeros((n, k), dtype=torch.bfloat16, device="cuda")
    x = torch.ones((k,), dtype=torch.bfloat16, device="cuda")
    for r in (3001, 77, 2500):          # equal, largest logits
        w[r] = 0.5
    w[10] = -4.0
    tok = torch.zeros((1,), dtype=torch.int64, device="cuda")
    ops.lm_head_argmax(x, w, tok)
    torch.cuda.synchronize()
    assert int(tok[0]) == 77
    w[77] = 0.25                        # now 2500 and 3001 tie
    ops.lm_head_argmax(x, w, tok)
    torch.cuda.synchronize()
    assert int(tok[0]) == 2500
    w.fill_(0.0)
    w[:5] = -1.0                        # all logits <= 0: first zero logit wins
    ops.lm_head_argmax(x, w, tok)
    torch.cuda.synchronize()
    assert int(tok[0]) == 5 == int(ops.gemv(x, w).float().argmax())


def test_qkv_rope_append_reads_the_table_row_of_the_device_position():
    from voom_amd.page_pool import v_slot_shape
    nq, nkv, hd, K, PT, pos = 9, 3, 64, 576, 64, 100
    g = torch.Generator(device="cuda").manual_seed(11)
    w = (torch.randn(((nq + 2 * nkv) * hd, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = torch.randn((1, 1, K), generator=g, device="cuda").to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(hd // 2, device="cuda", dtype=torch.float32) / (hd // 2)))
    ang = torch.arange(300, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1).contiguous()
    sin = torch.cat([ang.sin(), ang.sin()], -1).contiguous()
    table = torch.tensor([[2, 0, 3, 1]], dtype=torch.int32, device="cuda")
    position = torch.tensor([pos], dtype=torch.int32, device="cuda")
    kp = [torch.zeros((4, nkv, PT, hd), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    vp = [torch.zeros((4,) + v_slot_shape(nkv, hd, PT), dtype=torch.bfloat16, device="cuda")
          for _ in range(2)]
    q1 = ops.qkv_rope_append(x, w, cos, sin, kp[0], vp[0], table, position, nq, nkv, hd)
    q2 = ops.qkv_rope_append(x, w, cos[pos:pos + 1].contiguous(), sin[pos:pos + 1].contiguous(),
                             kp[1], vp[1], table, position, nq, nkv, hd)
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kp[0].view(torch.int16), kp[1].view(torch.int16))
    assert torch.equal(vp[0].view(torch.int16), vp[1].view(torch.int16))
