"""GPU parity of the byte-plane kernels and page helpers (bit-exact)."""
import numpy as np
import pytest
import torch

from oracle import byteplane as ob
from voom_amd import ops
from voom_amd.page_pool import v_pages_to_tokens, v_slot_shape

pytestmark = pytest.mark.gpu


def test_split_merge_every_bit_pattern():
    print("[codec] exhaustive 65536 patterns", flush=True)
    e = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    e = e[np.random.default_rng(0).permutation(e.size)]
    d = torch.from_numpy(e.view(np.int16).copy()).cuda()
    lo, hi = ops.byteplane_split(d)
    back = torch.empty_like(d)
    ops.byteplane_merge(lo, hi, back)
    torch.cuda.synchronize()
    rl, rh = ob.split(e)
    assert np.array_equal(lo.cpu().numpy(), rl)
    assert np.array_equal(hi.cpu().numpy(), rh)
    assert np.array_equal(back.cpu().numpy().view(np.uint16), e)


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1000, 4096 + 13, 3 * 2 ** 20 + 5])
def test_ragged_lengths(n):
    print(f"[codec] n={n}", flush=True)
    raw = np.random.default_rng(n).integers(0, 65536, size=n, dtype=np.uint32).astype(np.uint16)
    d = torch.from_numpy(raw.view(np.int16).copy()).cuda()
    lo, hi = ops.byteplane_split(d)
    back = torch.empty_like(d)
    ops.byteplane_merge(lo, hi, back)
    torch.cuda.synchronize()
    rl, rh = ob.split(raw)
    assert np.array_equal(lo.cpu().numpy(), rl) and np.array_equal(hi.cpu().numpy(), rh)
    assert np.array_equal(back.cpu().numpy().view(np.uint16), raw)


def test_slot_gather_split_and_scatter_merge():
    print("[codec] slot gather/scatter", flush=True)
    rng = np.random.default_rng(7)
    slots_total, slot_elems = 37, 8 * 64 * 128
    pool_np = rng.integers(0, 65536, size=(slots_total, slot_elems), dtype=np.uint32).astype(np.uint16)
    pool = torch.from_numpy(pool_np.view(np.int16).copy()).cuda()
    pick = rng.choice(slots_total, size=11, replace=False).astype(np.int32)
    slots = torch.from_numpy(pick).cuda()
    lo = torch.empty(11 * slot_elems, dtype=torch.uint8, device="cuda")
    hi = torch.empty_like(lo)
    ops.byteplane_split_slots(pool, slots, lo, hi)
    torch.cuda.synchronize()
    rl, rh = ob.split(pool_np[pick].reshape(-1))
    assert np.array_equal(lo.cpu().numpy(), rl) and np.array_equal(hi.cpu().numpy(), rh)
    dest = torch.zeros_like(pool)
    target = rng.choice(slots_total, size=11, replace=False).astype(np.int32)
    ops.byteplane_merge_slots(lo, hi, dest, torch.from_numpy(target).cuda())
    torch.cuda.synchronize()
    got = dest.cpu().numpy().view(np.uint16)
    assert np.array_equal(got[target], pool_np[pick])
    untouched = np.setdiff1d(np.arange(slots_total), target)
    assert np.all(got[untouched] == 0)


def test_append_then_gather_round_trips():
    print("[pages] append/gather", flush=True)
    B, NKV, D, PT, S = 3, 2, 128, 64, 150
    pages = -(-S // PT)
    slots = B * pages + 4
    perm = np.random.default_rng(3).permutation(slots)[: B * pages].reshape(B, pages)
    table = torch.from_numpy(perm.astype(np.int32)).cuda()
    kp = torch.zeros((slots, NKV, PT, D), dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros((slots,) + v_slot_shape(NKV, D, PT), dtype=torch.bfloat16, device="cuda")
    k = torch.randn((B, NKV, S, D), device="cuda").to(torch.bfloat16)
    v = torch.randn((B, NKV, S, D), device="cuda").to(torch.bfloat16)
    # append in three uneven steps, as prefill chunk + decode tokens would
    cut = [0, 100, 149, 150]
    for a, b in zip(cut[:-1], cut[1:]):
        pos = torch.full((B,), a, dtype=torch.int32, device="cuda")
        ops.append_kv(k[:, :, a:b].contiguous(), v[:, :, a:b].contiguous(), kp, vp, table, pos)
    kg, vg = ops.gather_kv(kp, vp, table, S)
    torch.cuda.synchronize()
    assert torch.equal(kg, k) and torch.equal(vg, v)
    # V really is stored as V^T blocks of 32 tokens: token 37 of page 0 is
    # column 5 of block 1
    assert torch.equal(vp[int(perm[1, 0]), 1, 1, :, 5], v[1, 1, 37])
    assert torch.equal(v_pages_to_tokens(vp[int(perm[1, 0])].unsqueeze(0)), v[1:2, :, :PT])
