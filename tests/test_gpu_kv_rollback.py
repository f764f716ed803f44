"""GPU tests of the cache's rollback and of attention over many spilled chunks.

* trim / trim_layer_lengths roll the paged KV and latent caches back exactly
  as the reference's KVCache.trim does (runtime/kv_cache.py:107-179): the
  first ``length`` positions stay bit-identical, later appends continue from
  there, and pages spilled past the cut are dropped.
* attend over spilled pages that stream in as many chunks keeps an fp32
  running state (runtime/glm.py:165-196 keeps fp32 across key tiles).
* an upload started ahead of a layer's attention keeps its staging buffer
  until it is merged, even when a spill runs in between.
"""
import numpy as np
import pytest
import torch

from oracle import paged_attention as opa
from voom_amd.kv_paged import PagedKVCache

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def bits(t):
    return t.contiguous().view(torch.int16)


def randn_bf16(shape, gen):
    return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)


def oracle(q, K, V, scale):
    out = [opa.sdpa_decode(q[b, :, 0].float().cpu().numpy(), K[b].float().cpu().numpy(),
                           V[b].float().cpu().numpy(), scale, dtype=np.float64)
           for b in range(q.shape[0])]
    return np.stack(out)[:, :, None, :]


@pytest.mark.parametrize("spill_cut", [False, True])
def test_trim_rolls_back_and_appends_continue(spill_cut):
    print(f"[trim] kv cache spill_cut={spill_cut}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(21)
    B, NQ, NKV, D, PT, layers = 2, 8, 2, 128, 64, 2
    kv = PagedKVCache(num_layers=layers, max_bytes=1 << 40, page_positions=PT,
                      resident_pages=1)
    ks = [randn_bf16((B, NKV, 300, D), gen) for _ in range(layers)]
    vs = [randn_bf16((B, NKV, 300, D), gen) for _ in range(layers)]
    for layer in range(layers):
        kv.append(layer, ks[layer], vs[layer])
    # page 2 (tokens 128..191) will hold the cut at 150; spill it and a page
    # wholly past the cut
    if spill_cut:
        kv.spill([(l, i) for l in range(layers) for i in (0, 2, 3)])
    kv.trim(150)
    assert kv.offset == 150 and kv.layer_lengths() == (150, 150)
    assert len(kv._pages[0]) == 2
    assert all(p.resident == (not spill_cut or p.index != 0) for p in kv._pages[0])
    new_k = [randn_bf16((B, NKV, 90, D), gen) for _ in range(layers)]
    new_v = [randn_bf16((B, NKV, 90, D), gen) for _ in range(layers)]
    for layer in range(layers):
        kv.append(layer, new_k[layer], new_v[layer])
    assert kv.offset == 240
    for layer in range(layers):
        K, V = kv.gather(layer)
        want_k = torch.cat([ks[layer][:, :, :150], new_k[layer]], 2)
        want_v = torch.cat([vs[layer][:, :, :150], new_v[layer]], 2)
        assert torch.equal(bits(K), bits(want_k)) and torch.equal(bits(V), bits(want_v))
        q = randn_bf16((B, NQ, 1, D), gen)
        out = kv.attend(layer, q)
        torch.cuda.synchronize()
        np.testing.assert_allclose(out.float().cpu().numpy(),
                                   oracle(q, want_k, want_v, D ** -0.5), atol=ATOL, rtol=RTOL)
    kv.release()


def test_trim_layer_lengths_and_errors():
    print("[trim] per-layer lengths, latent cache", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(22)
    B, R, PT = 2, 576, 64
    kv = PagedKVCache(num_layers=3, max_bytes=1 << 40, page_positions=PT, resident_pages=1)
    lats = [randn_bf16((B, 200, R), gen) for _ in range(3)]
    for layer in range(3):
        kv.append_latent(layer, lats[layer])
    kv.spill([(1, 1)])
    with pytest.raises(ValueError, match="cannot grow"):
        kv.trim_layer_lengths([201, 10, 10])
    with pytest.raises(ValueError, match="invalid"):
        kv.trim_layer_lengths([10, 10])
    with pytest.raises(ValueError):
        kv.trim(-1)
    kv.trim_layer_lengths([200, 100, 64])
    assert kv.layer_lengths() == (200, 100, 64)
    for layer, n in enumerate((200, 100, 64)):
        got = kv.gather_latent(layer)
        assert torch.equal(bits(got), bits(lats[layer][:, :n]))
    kv.trim(0)
    assert kv.layer_lengths() == (0, 0, 0) and kv.nbytes() == 0
    more = randn_bf16((B, 70, R), gen)
    for layer in range(3):
        kv.append_latent(layer, more)
    assert torch.equal(bits(kv.gather_latent(2)), bits(more))
    kv.release()


def test_trim_calls_the_attached_dsa_state():
    print("[trim] dsa state follows", flush=True)
    seen = []

    class Probe:
        def trim(self, length):
            seen.append(length)

    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=64)
    kv.dsa = Probe()
    kv.append_latent(0, torch.zeros((1, 10, 576), dtype=torch.bfloat16, device="cuda"))
    kv.trim(4)
    assert seen == [4] and kv.offset == 4


def test_reserve_refuses_spilled_pages():
    print("[reserve] spilled pages", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(23)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=64)
    kv.append(0, randn_bf16((1, 2, 200, 64), gen), randn_bf16((1, 2, 200, 64), gen))
    kv.spill([(0, 0)])
    with pytest.raises(ValueError, match="spilled"):
        kv.reserve(300)
    kv.reload()
    kv.reserve(300)
    kv.release()


def test_many_one_page_chunks_keep_an_fp32_running_state():
    print("[chunks] 40 one-page chunks", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(24)
    B, NQ, NKV, D, PT, S = 2, 8, 2, 128, 64, 64 * 44 + 17
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1,
                      prefetch=False)
    k = randn_bf16((B, NKV, S, D), gen)
    v = randn_bf16((B, NKV, S, D), gen)
    kv.append(0, k, v)
    q = randn_bf16((B, NQ, 1, D), gen)
    resident = kv.attend(0, q).clone()
    kv._ring.nbytes = kv.page_nbytes  # one page per staging chunk
    assert kv.spill([(0, i) for i in range(40)]) == 40
    out = kv.attend(0, q)
    torch.cuda.synchronize()
    ref = oracle(q, k, v, D ** -0.5)
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
    # 41 folds cost no more than the bf16 rounding of the parts: within a few
    # bf16 ulps of the output scale, as the one-call resident result is
    scale_ = np.abs(ref).max()
    err_chunked = np.abs(got - ref).max()
    err_resident = np.abs(resident.float().cpu().numpy() - ref).max()
    assert err_chunked <= 4 * 2 ** -8 * scale_, (err_chunked, scale_)
    assert err_chunked <= 4 * err_resident + 2 ** -9 * scale_, (err_chunked, err_resident)
    kv.release()


def test_prefetched_buffer_survives_a_spill_before_its_merge():
    """attend(0) starts layer 1's upload; a spill runs before attend(1); the
    layer's second chunk must not be staged into the prefetched buffer while
    that buffer still waits for its merge."""
    print("[ring] prefetch + spill + multi-chunk attend", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(25)
    B, NQ, NKV, D, PT, layers, S = 2, 8, 2, 128, 64, 2, 64 * 12
    kv = PagedKVCache(num_layers=layers, max_bytes=1 << 40, page_positions=PT,
                      resident_pages=1)
    ks = [randn_bf16((B, NKV, S, D), gen) for _ in range(layers)]
    vs = [randn_bf16((B, NKV, S, D), gen) for _ in range(layers)]
    for layer in range(layers):
        kv.append(layer, ks[layer], vs[layer])
    kv._ring.nbytes = 2 * kv.page_nbytes  # two pages per chunk
    kv.spill([(l, i) for l in range(layers) for i in range(6)])  # 3 chunks per layer
    for step in range(3):
        qs = [randn_bf16((B, NQ, 1, D), gen) for _ in range(layers)]
        out0 = kv.attend(0, qs[0])          # ends by starting layer 1's first upload
        kv.spill([(0, 6 + step)])           # takes a staging buffer in between
        out1 = kv.attend(1, qs[1])          # merges the prefetch, stages chunks 2 and 3
        torch.cuda.synchronize()
        for layer, q, out in ((0, qs[0], out0), (1, qs[1], out1)):
            np.testing.assert_allclose(out.float().cpu().numpy(),
                                       oracle(q, ks[layer], vs[layer], D ** -0.5),
                                       atol=ATOL, rtol=RTOL)
    assert kv.prefetch_hits > 0
    kv.release()


def steady_marks(kv):
    """(device bytes allocated, arena capacity, arena bytes in use) after a
    collection, so that objects other tests left behind are not freed midway."""
    import gc

    gc.collect()
    torch.cuda.synchronize()
    return torch.cuda.memory_allocated(), kv.arena.capacity, kv.arena.used_bytes


def assert_steady(marks):
    # from the second cycle on the arena is unchanged; device memory is the
    # same over the last three cycles (a leak grows it every cycle) and has
    # grown by at most the bounded memo of index tensors (256 small entries)
    assert all(m[1:] == marks[1][1:] for m in marks[1:]), marks
    assert marks[-1] == marks[-2] == marks[-3], marks
    assert marks[-1][0] - marks[1][0] <= 1 << 16, marks


def test_repeated_spill_reload_cycles_hold_memory_steady():
    """A serving loop spills and reloads the same cache again and again.  After
    the first cycle, device memory, the pinned arena's capacity and its used
    bytes are the same at the end of every cycle; attention over the spilled
    pages (streamed in per call) repeats bit for bit and matches the oracle,
    and after each reload it equals the all-resident result bit for bit."""
    print("[kv] repeated spill/reload cycles", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(21)
    B, NKV, NQ, D, PT, L = 2, 4, 16, 128, 64, 2
    kv = PagedKVCache(num_layers=L, max_bytes=1 << 40, page_positions=PT)
    ks, vs = [], []
    for layer in range(L):
        k = randn_bf16((B, NKV, 5 * PT + 17, D), gen)
        v = randn_bf16((B, NKV, 5 * PT + 17, D), gen)
        kv.append(layer, k, v)
        ks.append(k)
        vs.append(v)
    q = randn_bf16((B, NQ, 1, D), gen)
    resident = [kv.attend(layer, q) for layer in range(L)]
    torch.cuda.synchronize()
    spilled_ref = None
    marks = []
    for cycle in range(6):
        assert kv.spill([(layer, i) for layer in range(L) for i in range(4)]) == 4 * L
        spilled = [kv.attend(layer, q) for layer in range(L)]
        torch.cuda.synchronize()
        if spilled_ref is None:
            spilled_ref = spilled
            for layer in range(L):
                np.testing.assert_allclose(spilled[layer].float().cpu().numpy(),
                                           oracle(q, ks[layer], vs[layer], D ** -0.5),
                                           atol=ATOL, rtol=RTOL)
        for a, b in zip(spilled, spilled_ref):
            assert torch.equal(bits(a), bits(b)), f"cycle {cycle}: spilled attention changed"
        assert kv.reload() == 4 * L
        again = [kv.attend(layer, q) for layer in range(L)]
        torch.cuda.synchronize()
        for a, b in zip(again, resident):
            assert torch.equal(bits(a), bits(b)), f"cycle {cycle}: reloaded attention changed"
        marks.append(steady_marks(kv))
    assert_steady(marks)
    kv.release()


@pytest.mark.parametrize("compress", [False, True])
def test_repeated_latent_spill_reload_cycles_hold_memory_steady(compress):
    """The same soak over a latent (absorbed-MLA) cache, with and without the
    zstd high planes: steady device and pinned memory after the first cycle,
    attend_mla bit-stable over spilled pages and bit-identical to the
    all-resident result after each reload."""
    from voom_amd import ops
    print(f"[kv-latent] repeated spill/reload cycles compress={compress}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(22)
    B, H, dn, dv, C, dr, PT = 2, 64, 128, 128, 512, 64, 64
    kv_b = (torch.randn((H * (dn + dv), C), generator=gen, device="cuda") * C ** -0.5
            ).to(torch.bfloat16)
    w_uk, w_uv_t = ops.split_kv_b(kv_b, H, dn, dv)
    w_uk, w_uv_t = ops.pack_head_weights(w_uk), ops.pack_head_weights(w_uv_t)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT,
                      compress_spill=compress)
    kv.append_latent(0, randn_bf16((B, 6 * PT + 5, C + dr), gen))
    q_nope = randn_bf16((B, H, dn), gen)
    q_rope = randn_bf16((B, H, dr), gen)
    scale = (dn + dr) ** -0.5
    resident = kv.attend_mla(0, q_nope, q_rope, w_uk, w_uv_t, scale)
    torch.cuda.synchronize()
    spilled_ref = None
    marks = []
    for cycle in range(5):
        assert kv.spill([(0, i) for i in (0, 2, 3, 5)]) == 4
        spilled = kv.attend_mla(0, q_nope, q_rope, w_uk, w_uv_t, scale)
        torch.cuda.synchronize()
        if spilled_ref is None:
            spilled_ref = spilled
            np.testing.assert_allclose(spilled.float().cpu().numpy(),
                                       resident.float().cpu().numpy(), atol=ATOL, rtol=RTOL)
        assert torch.equal(bits(spilled), bits(spilled_ref)), f"cycle {cycle}"
        assert kv.reload() == 4
        again = kv.attend_mla(0, q_nope, q_rope, w_uk, w_uv_t, scale)
        torch.cuda.synchronize()
        assert torch.equal(bits(again), bits(resident)), f"cycle {cycle}"
        kv._wait_host_work()  # background zstd jobs of this cycle
        marks.append(steady_marks(kv))
    assert_steady(marks)
    kv.release()
