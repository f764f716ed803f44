"""Host-side invariants of the position-free pool and cache (CPU tensors):
the refcount / write-once / sharing rules of runtime/kv_cache.py:255-701."""
import pytest
import torch

from voom_amd.position_free import PositionFreeKVCache, PositionFreePagePool


def kv(L, NKV=2, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((1, NKV, L, D), generator=g).to(torch.bfloat16)
    v = torch.randn((1, NKV, L, D), generator=g).to(torch.bfloat16)
    return k, v


def test_allocate_write_gather_and_growth():
    pool = PositionFreePagePool(2, 2, 8, min_capacity=4, device="cpu")
    cache = PositionFreeKVCache(pool)
    ks = []
    for chunk in (3, 4, 2):
        k, v = kv(chunk, seed=chunk)
        ks.append((k, v))
        for layer in range(2):
            cache.update_unrotated(layer, k, v)
    assert cache.offset == 9 and cache.is_complete and pool.capacity >= 9
    K, V = cache.gather_unrotated(1)
    assert torch.equal(K, torch.cat([k for k, _ in ks], 2))
    assert torch.equal(V, torch.cat([v for _, v in ks], 2))
    assert cache.block_table().tolist() == list(cache.page_ids)
    assert cache.key_positions().tolist() == list(range(9))


def test_sharing_refcounts_and_recycling():
    pool = PositionFreePagePool(1, 2, 8, device="cpu")
    a = PositionFreeKVCache(pool)
    a.update_unrotated(0, *kv(5))
    b = PositionFreeKVCache.share_prefix(a, 3)
    b.update_unrotated(0, *kv(2, seed=9))
    shared = a.page_ids[:3]
    assert b.page_ids[:3] == shared
    assert all(pool.reference_count(p) == 2 for p in shared)
    a.release()
    assert all(pool.reference_count(p) == 1 for p in shared)
    assert pool.live_pages == 5          # 3 shared + b's 2 own
    Kb, _ = b.gather_unrotated(0)
    assert Kb.shape[2] == 5
    b.release()
    assert pool.live_pages == 0 and pool.free_pages == 7
    c = PositionFreeKVCache(pool)
    c.update_unrotated(0, *kv(4))
    assert set(c.page_ids) <= set(range(7))   # recycled ids


def test_invariants_raise_like_the_reference():
    pool = PositionFreePagePool(2, 2, 8, device="cpu")
    cache = PositionFreeKVCache(pool)
    k, v = kv(3)
    cache.update_unrotated(0, k, v)
    with pytest.raises(ValueError, match="incomplete"):
        PositionFreeKVCache.share_prefix(cache, 2)   # layer 1 not written yet
    with pytest.raises(ValueError, match="written twice"):
        pool.write(0, cache.page_ids, k, v)
    with pytest.raises(ValueError, match="same complete token span"):
        cache.update_unrotated(1, *kv(2))
    cache.update_unrotated(1, k, v)
    other = PositionFreeKVCache.share_prefix(cache, 3)
    with pytest.raises(ValueError, match="exclusively writable"):
        pool.write(0, other.page_ids, k, v)      # shared pages are read-only
    other.release()
    cache.release()
    with pytest.raises(RuntimeError, match="released twice"):
        pool.release([cache_id for cache_id in range(1)])
    with pytest.raises(RuntimeError, match="released"):
        cache.gather_unrotated(0)
    with pytest.raises(ValueError):
        pool.allocate(-1)


# ---- the reference's position-free cache tests (tests/test_kv_cache.py:222-335) ----

from voom_amd.position_free import ReusedRange, ToolPICPlan  # noqa: E402


def values_of(layer: int, width: int, dim: int = 32):
    keys = (torch.arange(width * dim, dtype=torch.float32).reshape(1, 1, width, dim)
            + layer * 10_000)
    return keys, keys + 1000


def f32_pool(layers, nkv, dim, **kw):
    return PositionFreePagePool(layers, nkv, dim, device="cpu", dtype=torch.float32, **kw)


def test_pic_plan_shares_pages_and_releases_by_reference():
    pool = f32_pool(2, 1, 32, min_capacity=8)
    source = PositionFreeKVCache(pool)
    for layer in range(2):
        source.update_unrotated(layer, *values_of(layer, 4))
    assert source.is_complete and pool.live_pages == 4
    plan = ToolPICPlan(reused=(ReusedRange(0, 1, 0, "tool_capsule"),
                               ReusedRange(2, 4, 1, "tool_capsule")),
                       selected_positions=(1, 4), exact_prefix_tokens=0,
                       capsule_tokens_reused=3, capsule_tokens_repaired=0)
    dest = PositionFreeKVCache.from_pic_plan(source, plan, 5)
    # four source pages plus two new selected pages
    assert pool.live_pages == 6
    assert dest.page_ids[0] == source.page_ids[0]
    assert dest.page_ids[2:4] == source.page_ids[1:3]
    for page_id in (dest.page_ids[0], *dest.page_ids[2:4]):
        assert pool.reference_count(page_id) == 2
    assert not dest.is_complete
    for layer in range(2):
        keys, vals = values_of(layer + 10, 2)
        dest.write_selected(layer, (1, 4), keys, vals)
    assert dest.is_complete
    source.release()
    assert pool.live_pages == 5
    assert all(pool.reference_count(p) == 1 for p in dest.page_ids)
    gathered, _ = dest.gather_unrotated(1)
    assert float(gathered[0, 0, 0, 0]) == 10_000
    assert float(gathered[0, 0, 2, 0]) == 10_032
    assert float(gathered[0, 0, 1, 0]) == 110_000  # the selected page's own write
    dest.release()
    assert pool.live_pages == 0 and pool.free_pages == 6


def test_trim_recycles_only_unreferenced_tail_pages():
    pool = f32_pool(1, 1, 32, min_capacity=4)
    source = PositionFreeKVCache(pool)
    source.update_unrotated(0, *values_of(0, 4))
    shared = source.page_ids[:2]
    pool.retain(shared)
    source.trim(2)
    assert pool.live_pages == 2 and source.offset == 2
    assert all(pool.reference_count(p) == 2 for p in shared)
    source.release()
    assert all(pool.reference_count(p) == 1 for p in shared)
    pool.release(shared)
    assert pool.live_pages == 0


def test_live_counter_tracks_reference_transitions():
    pool = f32_pool(1, 1, 32, min_capacity=8)
    cache = PositionFreeKVCache(pool)
    cache.update_unrotated(0, *values_of(0, 5))
    assert pool.live_pages == 5 == int((pool._refs[:pool._high] > 0).sum())
    shared = cache.page_ids[1:4]
    pool.retain(shared)
    assert pool.live_pages == 5
    pool.release(shared)
    assert pool.live_pages == 5
    cache.trim(2)
    assert pool.live_pages == 2
    cache.release()
    assert pool.live_pages == 0
    pool.close()
    assert pool.live_pages == 0


def test_failed_plan_restores_the_pool():
    pool = f32_pool(1, 1, 32, min_capacity=8)
    source = PositionFreeKVCache(pool)
    source.update_unrotated(0, *values_of(0, 2))
    bad = ToolPICPlan(reused=(), selected_positions=(0, 0), exact_prefix_tokens=0,
                      capsule_tokens_reused=0, capsule_tokens_repaired=2)
    with pytest.raises(ValueError, match="invalid PIC selected position"):
        PositionFreeKVCache.from_pic_plan(source, bad, 2)
    assert pool.live_pages == 2 and pool.free_pages == 2
    overlap = ToolPICPlan(reused=(ReusedRange(0, 2, 0, "x"),), selected_positions=(1,),
                          exact_prefix_tokens=0, capsule_tokens_reused=2,
                          capsule_tokens_repaired=1)
    with pytest.raises(ValueError, match="overlapping PIC destination"):
        PositionFreeKVCache.from_pic_plan(source, overlap, 2)
    gap = ToolPICPlan(reused=(), selected_positions=(0,), exact_prefix_tokens=0,
                      capsule_tokens_reused=0, capsule_tokens_repaired=1)
    with pytest.raises(ValueError, match="uncovered positions"):
        PositionFreeKVCache.from_pic_plan(source, gap, 3)
    past = ToolPICPlan(reused=(ReusedRange(1, 3, 1, "x"),), selected_positions=(0,),
                       exact_prefix_tokens=0, capsule_tokens_reused=2,
                       capsule_tokens_repaired=1)
    with pytest.raises(ValueError, match="invalid PIC reused position layout"):
        PositionFreeKVCache.from_pic_plan(source, past, 3)
    assert pool.live_pages == 2 and all(pool.reference_count(p) == 1 for p in source.page_ids)


def test_write_selected_and_trim_errors():
    pool = f32_pool(1, 1, 32)
    source = PositionFreeKVCache(pool)
    source.update_unrotated(0, *values_of(0, 3))
    plan = ToolPICPlan(reused=(ReusedRange(0, 2, 0, "x"),), selected_positions=(2,),
                       exact_prefix_tokens=0, capsule_tokens_reused=2, capsule_tokens_repaired=1)
    dest = PositionFreeKVCache.from_pic_plan(source, plan, 3)
    with pytest.raises(ValueError, match="shape mismatch"):
        dest.write_selected(0, (2,), *values_of(0, 2))
    with pytest.raises(ValueError, match="outside destination"):
        dest.write_selected(0, (7,), *values_of(0, 1))
    dest.write_selected(0, (2,), *values_of(0, 1))
    with pytest.raises(ValueError, match="already completed"):
        dest.write_selected(0, (2,), *values_of(0, 1))
    with pytest.raises(ValueError, match="cannot grow"):
        dest.trim(4)
    with pytest.raises(ValueError, match="integer"):
        dest.trim(1.0)
    incomplete = PositionFreeKVCache(f32_pool(2, 1, 32))
    incomplete.update_unrotated(0, *values_of(0, 1))
    with pytest.raises(ValueError, match="source position-free cache is incomplete"):
        PositionFreeKVCache.from_pic_plan(incomplete, plan, 3)


def test_release_is_atomic_and_reserve_growth_prevents_regrowth():
    pool = f32_pool(1, 1, 32, min_capacity=4)
    cache = PositionFreeKVCache(pool)
    cache.update_unrotated(0, *values_of(0, 3))
    ids = cache.page_ids
    with pytest.raises(RuntimeError, match="released twice"):
        pool.release([ids[0], ids[1], ids[1]])  # ids[1] has one reference
    assert all(pool.reference_count(p) == 1 for p in ids)  # nothing changed
    cache.reserve_growth(40)
    cap = pool.capacity
    assert cap >= 43
    for _ in range(8):
        cache.update_unrotated(0, *values_of(0, 5))
    assert pool.capacity == cap and cache.offset == 43
    assert cache.block_table().tolist() == list(cache.page_ids)
    assert cache.key_positions().tolist() == list(range(43))
    cache.trim(10)
    assert cache.block_table().tolist() == list(cache.page_ids)[:10]
    cache.update_unrotated(0, *values_of(0, 2))
    assert cache.block_table().tolist() == list(cache.page_ids)


def test_recycled_ids_come_out_in_the_reference_order():
    """The reference frees a page at the occurrence that drops its last
    reference (runtime/kv_cache.py:402-414) and hands out _free[-k:] in list
    order (:367-371): pin the exact ids, repeated releases included."""
    pool = PositionFreePagePool(1, 2, 8, device="cpu")
    ids = pool.allocate(6)
    assert ids == (0, 1, 2, 3, 4, 5)
    pool.release([1, 3, 2])                  # free list [1, 3, 2]
    assert pool.allocate(2) == (3, 2)        # _free[-2:]
    assert pool.allocate(2) == (1, 6)        # [1] + one fresh id
    k, v = kv(4)
    pool.write(0, [0, 3, 4, 5], k, v)
    pool.retain([4])                         # page 4 held twice
    pool.release([4, 5, 4])                  # 5 dies first, 4 at its second occurrence
    assert pool.allocate(1) == (4,)
    assert pool.allocate(1) == (5,)
