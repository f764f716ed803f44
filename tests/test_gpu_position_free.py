"""GPU parity of voom_position_free_attention against oracle/position_free.py
(runtime/pic_attention.py restated), 2e-2 abs / 1e-2 rel in bf16 -- the
reference's own test tolerance for this kernel (tests/test_pic_attention.py:48)."""
import numpy as np
import pytest
import torch

from oracle import position_free as opf
from voom_amd import ops

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


STORE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def run(B, NQ, NKV, TQ, D, BLOCK, TK, P, *, seed, kpos=None, qpos=None, table=None,
        num_splits=0, max_pos=None, dtype=torch.bfloat16, table_dtype=torch.float32,
        scale_in=1.0, atol=ATOL, rtol=RTOL):
    print(f"[pf] B={B} NQ={NQ} NKV={NKV} TQ={TQ} D={D} BLOCK={BLOCK} TK={TK} P={P} "
          f"splits={num_splits} dtype={dtype} tables={table_dtype}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((B, NQ, TQ, D), generator=g) * scale_in).to(dtype)
    kp = (torch.randn((P, NKV, BLOCK, D), generator=g) * scale_in).to(dtype)
    vp = (torch.randn((P, NKV, BLOCK, D), generator=g) * scale_in).to(dtype)
    nblk = (TK + BLOCK - 1) // BLOCK
    if table is None:
        table = torch.randint(0, P, (nblk,), generator=g, dtype=torch.int32)
    if kpos is None:
        kpos = torch.arange(TK, dtype=torch.int32)
    if qpos is None:
        qpos = torch.arange(TK - TQ, TK, dtype=torch.int32).clamp(min=0)
    max_pos = max_pos or max(int(kpos.max()) + 1 if TK else 1, int(qpos.max()) + 1)
    cos, sin = ops.rope_cache(max_pos, D, 10000.0, device="cuda")
    cos, sin = cos.to(table_dtype), sin.to(table_dtype)
    out = ops.position_free_paged_attention(
        q.cuda(), kp.cuda(), vp.cuda(), table.cuda(), kpos.cuda(), qpos.cuda(), cos, sin,
        scale=D ** -0.5, num_splits=num_splits)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    f64 = dtype == torch.float32
    ref = opf.attention(q.float().numpy(), kp.float().numpy(), vp.float().numpy(),
                        table.numpy().astype(np.int64), kpos.numpy().astype(np.int64),
                        qpos.numpy().astype(np.int64), cos.float().cpu().numpy(),
                        sin.float().cpu().numpy(), D ** -0.5, store=STORE[dtype],
                        acc=np.float64 if f64 else np.float32)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=atol, rtol=rtol)
    return out


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("BLOCK", [1, 4, 64])
def test_block_sizes_and_head_dims(D, BLOCK):
    run(1, 8, 2, 1, D, BLOCK, 300, max(8, 600 // BLOCK), seed=1)


@pytest.mark.parametrize("NQ,NKV,TQ", [(9, 3, 4), (4, 4, 2), (16, 1, 1), (32, 8, 4)])
def test_head_groups_and_queries(NQ, NKV, TQ):
    run(2, NQ, NKV, TQ, 64, 16, 517, 80, seed=2)


def test_repeated_pages_and_unordered_positions():
    g = torch.Generator().manual_seed(3)
    TK, BLOCK = 200, 1
    table = torch.randint(0, 7, (TK,), generator=g, dtype=torch.int32)  # heavy sharing
    kpos = torch.randperm(400, generator=g)[:TK].to(torch.int32)
    qpos = torch.tensor([150, 399], dtype=torch.int32)  # first query sees only part
    run(1, 8, 2, 2, 128, BLOCK, TK, 7, seed=3, kpos=kpos, qpos=qpos, table=table)


@pytest.mark.parametrize("splits", [1, 3, 40])
def test_split_counts(splits):
    run(1, 4, 1, 1, 128, 64, 3000, 60, seed=4, num_splits=splits)


def test_nothing_visible_and_empty_key_set():
    out = run(1, 4, 2, 2, 64, 4, 40, 12, seed=5,
              qpos=torch.tensor([0, 1], dtype=torch.int32),
              kpos=torch.arange(10, 50, dtype=torch.int32))
    assert torch.all(out == 0)
    out = run(1, 4, 2, 1, 64, 4, 0, 3, seed=6, qpos=torch.tensor([5], dtype=torch.int32))
    assert torch.all(out == 0)


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.bfloat16, 64),
                                     (torch.bfloat16, 128), (torch.float16, 64)])
def test_reference_geometry_across_element_types(dtype, D):
    """tests/test_pic_attention.py:11-49: B=1, 4q/2kv, 3 queries at positions
    16..18, 19 keys in 4-key pages, RoPE tables of 32 positions in the element
    type (fp32 for fp32), inputs N(0, 0.1).  Bar: 2e-5 for fp32 (here against
    the fp64 oracle), 2e-2 for bf16 (the reference's), 2e-3 for fp16."""
    tol = {torch.float32: 2e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dtype]
    run(1, 4, 2, 3, D, 4, 19, 5, seed=713, table=torch.arange(5, dtype=torch.int32),
        qpos=torch.tensor([16, 17, 18], dtype=torch.int32), max_pos=32, dtype=dtype,
        table_dtype=dtype, scale_in=0.1, atol=tol, rtol=tol)


def test_reference_shared_page_at_two_positions_fp32():
    """tests/test_pic_attention.py:52-81: pages A, B, A (table [0, 1, 0]) of 4
    keys, 2 q / 2 kv heads, D = 64, one query at position 11, fp32 pages and
    tables; 2e-5 against the fp64 oracle."""
    run(1, 2, 2, 1, 64, 4, 12, 2, seed=19, table=torch.tensor([0, 1, 0], dtype=torch.int32),
        qpos=torch.tensor([11], dtype=torch.int32), max_pos=16, dtype=torch.float32,
        scale_in=0.1, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("NQ,NKV,TQ", [(28, 4, 3), (28, 4, 4), (64, 8, 4), (16, 1, 4),
                                       (48, 1, 2)])
def test_column_passes_for_large_groups(NQ, NKV, TQ):
    """More (head, query) columns than one MFMA tile holds: Qwen2.5-7B's 28q/4kv
    at 3- and 4-token verify windows (the reference's position-free gate model,
    runtime/kv_cache.py:566 allows 4 queries), 64q/8kv at 4, and groups of 16
    and 48 (2 to 6 passes)."""
    run(1, NQ, NKV, TQ, 128, 16, 700, 60, seed=31 + NQ + TQ)


def test_column_passes_with_batch_and_splits():
    run(3, 64, 8, 4, 128, 8, 333, 50, seed=41, num_splits=5)
    run(2, 28, 4, 4, 64, 1, 257, 300, seed=42, num_splits=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("NQ,NKV,TQ", [(4, 2, 3), (28, 4, 4), (16, 1, 4)])
def test_fp32_and_fp16_pages(dtype, NQ, NKV, TQ):
    tol = 2e-5 if dtype == torch.float32 else 2e-3
    run(2, NQ, NKV, TQ, 128, 16, 450, 40, seed=51, dtype=dtype, scale_in=0.3, atol=tol,
        rtol=tol)


@pytest.mark.parametrize("D", [32, 96, 160, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_other_head_dims(D, dtype):
    """Head dims the MFMA kernel does not take (any multiple of 32 up to 256);
    256 at 16 columns asks for 85 KB of LDS."""
    tol = 2e-5 if dtype == torch.float32 else 2e-2
    run(1, 16, 2, 2, D, 8, 300, 50, seed=61 + D, dtype=dtype, scale_in=0.3, atol=tol,
        rtol=tol if dtype == torch.float32 else RTOL)


def test_bf16_tables_on_the_mfma_kernel():
    run(2, 8, 2, 2, 128, 16, 600, 50, seed=71, table_dtype=torch.bfloat16)
    run(1, 28, 4, 4, 64, 4, 200, 60, seed=72, table_dtype=torch.bfloat16)


def test_int64_indices_are_accepted():
    """The reference casts the table and positions to int32
    (runtime/pic_attention.py:223-224)."""
    g = torch.Generator().manual_seed(81)
    q = torch.randn((1, 4, 1, 64), generator=g).to(torch.bfloat16).cuda()
    kp = torch.randn((6, 2, 4, 64), generator=g).to(torch.bfloat16).cuda()
    cos, sin = ops.rope_cache(24, 64, 1e4, device="cuda")
    t32 = torch.tensor([3, 1, 4, 0, 5], dtype=torch.int32, device="cuda")
    k32 = torch.arange(20, dtype=torch.int32, device="cuda")
    q32 = torch.tensor([19], dtype=torch.int32, device="cuda")
    a = ops.position_free_paged_attention(q, kp, kp, t32, k32, q32, cos, sin, scale=0.125)
    b = ops.position_free_paged_attention(q, kp, kp, t32.long(), k32.long(), q32.long(), cos,
                                          sin, scale=0.125)
    assert torch.equal(a, b)


def test_dtype_and_table_errors_match_the_reference():
    q = torch.zeros((1, 4, 1, 64), dtype=torch.bfloat16, device="cuda")
    kp = torch.zeros((3, 2, 4, 64), dtype=torch.bfloat16, device="cuda")
    cos, sin = ops.rope_cache(16, 64, 1e4, device="cuda")
    i32 = lambda *v: torch.tensor(v, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="dtypes must match"):
        ops.position_free_paged_attention(q, kp.float(), kp.float(), i32(0), i32(0), i32(0),
                                          cos, sin, scale=1.0)
    with pytest.raises(ValueError, match="RoPE cache must be FP32 or match"):
        ops.position_free_paged_attention(q, kp, kp, i32(0), i32(0), i32(0), cos.half(),
                                          sin.half(), scale=1.0)
    with pytest.raises(ValueError, match="RoPE cache must be FP32 or match"):
        ops.position_free_paged_attention(q, kp, kp, i32(0), i32(0), i32(0), cos, sin.bfloat16(),
                                          scale=1.0)


def test_validation_matches_the_reference_errors():
    q = torch.zeros((1, 4, 1, 64), dtype=torch.bfloat16, device="cuda")
    kp = torch.zeros((3, 2, 4, 64), dtype=torch.bfloat16, device="cuda")
    cos, sin = ops.rope_cache(16, 64, 1e4, device="cuda")
    i32 = lambda *v: torch.tensor(v, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="block table"):
        ops.position_free_paged_attention(q, kp, kp, i32(0), i32(*range(8)), i32(7), cos, sin,
                                          scale=1.0)
    with pytest.raises(ValueError, match="RoPE cache"):
        ops.position_free_paged_attention(q, kp, kp, i32(0), i32(0), i32(0),
                                          cos[:, :16].contiguous(), sin[:, :16].contiguous(),
                                          scale=1.0)
    with pytest.raises(ValueError, match="geometry"):
        ops.position_free_paged_attention(q, kp, kp, i32(0), i32(0), i32(0, 1), cos, sin,
                                          scale=1.0)


def test_pool_cache_sharing_matches_the_oracle():
    """PositionFreeKVCache over a shared pool: a second request reuses the first
    one's prefix pages by reference; both attend through the kernel and match
    the oracle over their own logical tables (runtime/kv_cache.py:555-701)."""
    from voom_amd.position_free import PositionFreeKVCache, PositionFreePagePool
    print("[pf] pool/cache sharing", flush=True)
    L, NKV, NQ, D = 2, 2, 8, 64
    pool = PositionFreePagePool(L, NKV, D, min_capacity=16, device="cuda")
    g = torch.Generator().manual_seed(11)

    def chunk(n):
        return [(torch.randn((1, NKV, n, D), generator=g).to(torch.bfloat16).cuda(),
                 torch.randn((1, NKV, n, D), generator=g).to(torch.bfloat16).cuda())
                for _ in range(L)]

    a = PositionFreeKVCache(pool)
    for n in (40, 25):
        for layer, (k, v) in enumerate(chunk(n)):
            a.update_unrotated(layer, k, v)
    b = PositionFreeKVCache.share_prefix(a, 50)
    for layer, (k, v) in enumerate(chunk(30)):
        b.update_unrotated(layer, k, v)
    assert pool.capacity > 16                      # grew geometrically, ids kept
    for cache in (a, b):
        for layer in range(L):
            TQ = 2
            q = torch.randn((1, NQ, TQ, D), generator=g).to(torch.bfloat16)
            qpos = torch.tensor([cache.offset - 5, cache.offset - 1], dtype=torch.int32)
            out = cache.paged_attention(layer, q.cuda(), qpos, theta=10000.0, scale=D ** -0.5)
            torch.cuda.synchronize()
            kp, vp = pool.pages(layer)
            cos, sin = pool.rope(cache.offset, 10000.0)
            ref = opf.attention(q.float().numpy(), kp.float().cpu().numpy(),
                                vp.float().cpu().numpy(),
                                np.asarray(cache.page_ids, dtype=np.int64),
                                np.arange(cache.offset), qpos.numpy().astype(np.int64),
                                cos.cpu().numpy(), sin.cpu().numpy(), D ** -0.5)
            np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    a.release()
    Kb, _ = b.gather_unrotated(1)                  # shared pages survive a's release
    assert Kb.shape == (1, NKV, 80, D)
    b.release()
    assert pool.live_pages == 0


@pytest.mark.parametrize("yarn", [False, True])
def test_matches_the_rotated_page_cache(yarn):
    """The reference's dense-versus-shared check (tests/test_kv_cache.py:359-447):
    the same q, k, v through PositionFreeKVCache (unrotated keys, RoPE in the
    kernel) and through PagedKVCache (keys rotated on the host in fp32, the
    GQA kernel) -- a 7-token causal prefill, then one decode token -- with
    plain RoPE and with static YaRN (explicit denominators; q and k scaled by
    mscale before rotation, so the shared cache stores the scaled, unrotated
    key).  Bar: 2e-2, the reference's tolerance for its decode comparison."""
    from voom_amd.kv_paged import PagedKVCache
    from voom_amd.position_free import PositionFreeKVCache, PositionFreePagePool
    from voom_amd.synthetic import apply_rope_neox
    print(f"[pf] against the rotated page cache, yarn={yarn}", flush=True)
    NKV, NQ, D, T, theta = 2, 4, 64, 7, 10000.0  # 2 heads x 7 queries <= 16 columns
    half = D // 2
    g = torch.Generator().manual_seed(741)

    def rnd(*shape):
        return (torch.randn(shape, generator=g) * 0.5).to(torch.bfloat16)

    q, k, v = rnd(1, NQ, T + 1, D), rnd(1, NKV, T + 1, D), rnd(1, NKV, T + 1, D)
    den, mscale = None, 1.0
    if yarn:
        den = theta ** (torch.arange(half, dtype=torch.float32) / half)
        den = den * torch.linspace(1.0, 4.0, half)
        mscale = 1.1
    k_store = (k.float() * mscale).to(torch.bfloat16)  # scaled, unrotated
    cos, sin = ops.rope_cache(T + 1, D, theta, denominators=den, device="cuda")
    cos, sin = cos.cpu(), sin.cpu()
    q_rot = apply_rope_neox(q.float() * mscale, cos, sin).to(torch.bfloat16)
    k_rot = apply_rope_neox(k_store, cos, sin).to(torch.bfloat16)
    scale = D ** -0.5

    pool = PositionFreePagePool(1, NKV, D, min_capacity=16, device="cuda")
    shared = PositionFreeKVCache(pool)
    dense = PagedKVCache(1, 1 << 30, page_positions=64)
    outs = {}
    for name, lo, hi in (("prefill", 0, T), ("decode", T, T + 1)):
        shared.update_unrotated(0, k_store[:, :, lo:hi].cuda(), v[:, :, lo:hi].cuda())
        dense.append(0, k_rot[:, :, lo:hi].cuda(), v[:, :, lo:hi].cuda())
        qpos = torch.arange(lo, hi, dtype=torch.int32)
        got = shared.paged_attention(0, q_rot[:, :, lo:hi].cuda(), qpos, theta=theta,
                                     denominators=den, scale=scale)
        if name == "prefill":
            ref = dense.attend_prefill(0, q_rot[:, :, lo:hi].cuda(), scale)
        else:
            ref = dense.attend(0, q_rot[:, :, lo:hi].cuda(), scale)
        torch.cuda.synchronize()
        outs[name] = (got.float().cpu(), ref.float().cpu().reshape(got.shape))
    assert shared.offset == dense.offset == T + 1
    for name, (got, ref) in outs.items():
        assert torch.allclose(got, ref, rtol=2e-2, atol=2e-2), \
            f"{name}: max |diff| {float((got - ref).abs().max()):.4f}"
    shared.release()
    dense.release()
