"""Config 3 at its stated size: 32 layers x 32768 tokens x 8 KV heads x 128
(4 GiB of bf16 K/V, K ~ N(0,1) with 4 outlier channels per head scaled x20,
V ~ N(0,0.5)); the budget evicts the oldest 50 % of the pages in the
reference's order (runtime/kv_paged.py:216-240) through the byte-plane split
into pinned host memory; the pages are reloaded into seeded-random different
pool slots; all 4 GiB are compared bitwise (the reference's own bar for a
spilled page, tests/test_kv_spill_compress.py:47-50)."""
import numpy as np
import pytest
import torch

from voom_amd import ops
from voom_amd.kv_paged import PagedKVCache

pytestmark = pytest.mark.gpu


def test_config3_full_size_spill_reload_is_bit_exact():
    L, S, NKV, D, PT = 32, 32768, 8, 128, 64
    n_pages = S // PT
    print("[config3] building 32 x 32768-token layers", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(6)
    outlier = torch.ones((1, NKV, 1, D), device="cuda")
    for h in range(NKV):
        chans = np.random.default_rng(6 + h).choice(D, size=4, replace=False)
        outlier[0, h, 0, torch.from_numpy(chans).cuda()] = 20.0
    kv = PagedKVCache(num_layers=L, max_bytes=1 << 62, page_positions=PT, resident_pages=1,
                      initial_slots=n_pages)
    orig = []
    for layer in range(L):
        k = (torch.randn((1, NKV, S, D), generator=gen, device="cuda") * outlier
             ).to(torch.bfloat16)
        v = (torch.randn((1, NKV, S, D), generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
        kv.append(layer, k, v)
        orig.append((k.view(torch.int16), v.view(torch.int16)))
    spill_bytes = L * (n_pages // 2) * kv.page_nbytes
    assert spill_bytes == 2 << 30
    kv.arena.reserve(spill_bytes + (64 << 20))
    old_slots = {(l, i): list(kv._pages[l][i].slots) for l in range(L) for i in range(n_pages)}
    print("[config3] evicting 50 % through the budget", flush=True)
    kv.max_bytes = kv.nbytes() - spill_bytes
    assert kv.spill() == L * (n_pages // 2)
    # the reference order: the oldest half of every layer, nothing else
    for layer in range(L):
        res = [p.resident for p in kv._pages[layer]]
        assert not any(res[:n_pages // 2]) and all(res[n_pages // 2:])
    assert kv.nbytes() == kv.max_bytes
    # reload into different slots: shuffle each pool's free list (seed 7)
    rng = np.random.default_rng(7)
    for layer in range(L):
        free = kv._pools[layer]._free
        free[:] = [free[j] for j in rng.permutation(len(free))]
    print("[config3] reloading", flush=True)
    assert kv.reload() == L * (n_pages // 2)
    torch.cuda.synchronize()
    moved = sum(kv._pages[l][i].slots != old_slots[(l, i)]
                for l in range(L) for i in range(n_pages // 2))
    assert moved >= 0.9 * L * (n_pages // 2), moved
    print("[config3] comparing 4 GiB bitwise", flush=True)
    for layer in range(L):
        pool = kv._pools[layer]
        k2, v2 = ops.gather_kv(pool.k, pool.v, kv._tables[layer], S)
        assert torch.equal(k2.view(torch.int16), orig[layer][0]), f"layer {layer} K"
        assert torch.equal(v2.view(torch.int16), orig[layer][1]), f"layer {layer} V"
    assert kv.stats.spills == kv.stats.reloads == L * (n_pages // 2)
    kv.release()
    del orig
    torch.cuda.empty_cache()
