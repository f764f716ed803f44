"""Debug bounds checks of the attention calls (ops.set_bounds_checks).

The kernels read slot 0 for an out-of-range slot or page id and clamp a
position outside the RoPE tables, so a caller's bug gives plausible numbers.
With the checks on, the call raises ValueError instead, as the reference's
page pool and kernel wrapper do (runtime/kv_cache.py:305-310,357-476;
runtime/pic_attention.py:197-213).  Every call here runs to completion on the
GPU with in-bounds reads; only the host decides to raise."""
import pytest
import torch

from voom_amd import ops
from voom_amd.page_pool import v_slot_shape

pytestmark = pytest.mark.gpu


@pytest.fixture
def checks_on():
    ops.set_bounds_checks(True)
    try:
        yield
    finally:
        ops.set_bounds_checks(False)


def _gqa_inputs(seed=0, B=2, NQ=8, NKV=2, D=128, PT=64, slots=12, max_pages=4):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, NQ, D), generator=g).to(torch.bfloat16).cuda()
    k = torch.randn((slots, NKV, PT, D), generator=g).to(torch.bfloat16).cuda()
    v = torch.randn((slots,) + v_slot_shape(NKV, D, PT), generator=g).to(torch.bfloat16).cuda()
    table = torch.randperm(slots, generator=g)[:B * max_pages].reshape(B, max_pages)
    table = table.to(torch.int32).cuda()
    ctx = torch.tensor([150, 256], dtype=torch.int32, device="cuda")
    return q, k, v, table, ctx


def test_gqa_rejects_spilled_and_oversize_slots(checks_on):
    print("[bounds] gqa", flush=True)
    q, k, v, table, ctx = _gqa_inputs()
    ops.set_bounds_checks(False)
    want = ops.paged_gqa_decode(q, k, v, table, ctx)
    ops.set_bounds_checks(True)
    got = ops.paged_gqa_decode(q, k, v, table, ctx)   # valid: no error, same bits
    assert torch.equal(got, want)
    bad = table.clone()
    bad[0, 2] = -1                                     # a spilled column inside ctx 150
    with pytest.raises(ValueError, match="slot ids outside"):
        ops.paged_gqa_decode(q, k, v, bad, ctx)
    bad = table.clone()
    bad[1, 3] = k.shape[0]                             # one past the pool
    with pytest.raises(ValueError, match="slot ids outside"):
        ops.paged_gqa_decode(q, k, v, bad, ctx)
    bad = table.clone()
    bad[0, 3] = -1                                     # past sequence 0's context: fine
    ops.paged_gqa_decode(q, k, v, bad, ctx)
    with pytest.raises(ValueError, match="context lengths"):
        ops.paged_gqa_decode(q, k, v, table, torch.tensor([150, 257], dtype=torch.int32,
                                                          device="cuda"))


def test_checks_off_reads_slot_zero_without_error():
    print("[bounds] off", flush=True)
    q, k, v, table, ctx = _gqa_inputs(seed=1)
    bad = table.clone()
    bad[0, 0] = -1
    out = ops.paged_gqa_decode(q, k, v, bad, ctx)      # completes; no check
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


def test_mla_dense_and_sparse(checks_on):
    print("[bounds] mla", flush=True)
    g = torch.Generator().manual_seed(2)
    B, H, PT, slots, max_pages = 2, 64, 64, 10, 4
    q = torch.randn((B, H, 576), generator=g).to(torch.bfloat16).cuda()
    lat = torch.randn((slots, PT, 576), generator=g).to(torch.bfloat16).cuda()
    table = torch.arange(B * max_pages, dtype=torch.int32).reshape(B, max_pages).cuda()
    ctx = torch.tensor([200, 100], dtype=torch.int32, device="cuda")
    ops.mla_latent_decode(q, lat, table, ctx, scale=0.07)
    bad = table.clone()
    bad[1, 1] = -1
    with pytest.raises(ValueError, match="slot ids outside"):
        ops.mla_latent_decode(q, lat, bad, ctx, scale=0.07)
    sel = torch.tensor([[0, 5, 130, 199], [3, 64, 99, 0]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([4, 3], dtype=torch.int32, device="cuda")
    ops.mla_sparse_decode(q, lat, table, sel, lens, scale=0.07)
    with pytest.raises(ValueError, match="slot ids outside"):
        ops.mla_sparse_decode(q, lat, bad, sel, lens, scale=0.07)   # position 64 -> column 1
    far = sel.clone()
    far[0, 3] = max_pages * PT
    with pytest.raises(ValueError, match="positions outside"):
        ops.mla_sparse_decode(q, lat, table, far, lens, scale=0.07)
    with pytest.raises(ValueError, match="selection counts"):
        ops.mla_sparse_decode(q, lat, table, sel, torch.tensor([5, 3], dtype=torch.int32,
                                                               device="cuda"), scale=0.07)


def test_position_free_pages_and_positions(checks_on):
    print("[bounds] position-free", flush=True)
    g = torch.Generator().manual_seed(3)
    q = torch.randn((1, 4, 2, 64), generator=g).to(torch.bfloat16).cuda()
    kp = torch.randn((6, 2, 4, 64), generator=g).to(torch.bfloat16).cuda()
    cos, sin = ops.rope_cache(24, 64, 1e4, device="cuda")
    table = torch.tensor([3, 1, 4, 0, 5], dtype=torch.int32, device="cuda")
    kpos = torch.arange(20, dtype=torch.int32, device="cuda")
    qpos = torch.tensor([18, 19], dtype=torch.int32, device="cuda")
    ops.position_free_paged_attention(q, kp, kp, table, kpos, qpos, cos, sin, scale=0.125)
    for bad_id in (-1, 6):
        bad = table.clone()
        bad[2] = bad_id
        with pytest.raises(ValueError, match="page ids outside"):
            ops.position_free_paged_attention(q, kp, kp, bad, kpos, qpos, cos, sin, scale=0.125)
    far = kpos.clone()
    far[7] = 24
    with pytest.raises(ValueError, match="key positions"):
        ops.position_free_paged_attention(q, kp, kp, table, far, qpos, cos, sin, scale=0.125)
