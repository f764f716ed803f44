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
