"""GPU tests of the PagedKVCache drop-in (append/spill/reload/attend + the
reference protocol), mirroring tests/test_kv_spill_compress.py:22-60 of the
reference and checking attention against the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import paged_attention as opa
from voom_amd import ops
from voom_amd.kv_paged import PagedKVCache

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def bits(t):
    return t.contiguous().view(torch.int16)


def rand_bf16(shape, gen):
    # arbitrary 16-bit patterns: NaN payloads, infinities, subnormals included
    return torch.randint(-32768, 32768, shape, generator=gen, dtype=torch.int32,
                         device="cuda").to(torch.int16).view(torch.bfloat16)


@pytest.mark.parametrize("compress", [False, True])
def test_spilled_page_round_trips_byte_identical(compress):
    print(f"[kv] reference unit geometry compress={compress}", flush=True)
    kv = PagedKVCache(num_layers=2, max_bytes=1, spill_dir=None, page_positions=4,
                      resident_pages=0, compress_spill=compress)
    gen = torch.Generator(device="cuda").manual_seed(0)
    ref_k, ref_v = [], []
    for layer in range(2):
        k = rand_bf16((1, 2, 4, 8), gen)
        v = rand_bf16((1, 2, 4, 8), gen)
        ref_k.append(k)
        ref_v.append(v)
        kv.update(layer, k, v)
    for layer in range(2):
        kv.update(layer, rand_bf16((1, 2, 1, 8), gen), rand_bf16((1, 2, 1, 8), gen))
    assert kv.stats.spills > 0
    page = kv._pages[0][0]
    assert not page.resident
    lk, lv = page.load()
    torch.cuda.synchronize()
    assert lk.dtype == torch.bfloat16
    assert torch.equal(bits(lk), bits(ref_k[0])) and torch.equal(bits(lv), bits(ref_v[0]))
    if compress:
        assert kv.stats.spill_bytes_compressed > 0 and "compress" in kv.stats.summary()
    kv.release()
    assert kv.offset == 0 and kv.nbytes() == 0


def test_update_returns_everything_appended_even_after_spills():
    print("[kv] update() concatenation", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(1)
    B, NKV, D, PT = 2, 2, 64, 32
    kv = PagedKVCache(num_layers=3, max_bytes=3 * B * NKV * D * 4 * PT * 2,
                      page_positions=PT, resident_pages=1)
    ks = [[] for _ in range(3)]
    vs = [[] for _ in range(3)]
    for chunk in (70, 1, 1, 33, 1, 64, 1):
        for layer in range(3):
            k = rand_bf16((B, NKV, chunk, D), gen)
            v = rand_bf16((B, NKV, chunk, D), gen)
            ks[layer].append(k)
            vs[layer].append(v)
            K, V = kv.update(layer, k, v)
            torch.cuda.synchronize()
            assert torch.equal(bits(K), bits(torch.cat(ks[layer], dim=2)))
            assert torch.equal(bits(V), bits(torch.cat(vs[layer], dim=2)))
    assert kv.stats.spills > 0 and kv.stats.reloads > 0
    assert kv.offset == 171
    # the newest closed page of each layer stays resident
    for layer in range(3):
        assert kv._pages[layer][-1].resident


class count_staged_copies:
    """Counts the host -> staging-buffer transfers of a block: strided ones
    (ops.copy_rows) and plain tensor copies into a staging buffer."""

    def __init__(self, kv):
        self.kv = kv
        self.calls = []

    def __enter__(self):
        kv, calls = self.kv, self.calls
        self.real_rows, self.real_copy = ops.copy_rows, torch.Tensor.copy_

        def rows(*args, **kwargs):
            calls.append(("rows", args[5]))
            return self.real_rows(*args, **kwargs)

        def copy(dst, src, *args, **kwargs):
            ring = {b.untyped_storage().data_ptr() for b in kv._ring.bufs if b is not None}
            if (src.device.type == "cpu" and dst.device.type == "cuda"
                    and dst.untyped_storage().data_ptr() in ring):
                calls.append(("copy", src.numel()))
            return self.real_copy(dst, src, *args, **kwargs)

        ops.copy_rows, torch.Tensor.copy_ = rows, copy
        return calls

    def __exit__(self, *exc):
        ops.copy_rows, torch.Tensor.copy_ = self.real_rows, self.real_copy
        return False


@pytest.mark.parametrize("pages_per_chunk", [3, 7])
@pytest.mark.parametrize("verify", [True, False])
def test_staging_chunks_that_cut_a_host_record(pages_per_chunk, verify):
    """Pages spilled in one call share one host record.  Staging chunks
    smaller than that record, with two of its pages reloaded in between, take
    runs of its pages that start inside it; each run moves with one copy per
    plane (and per checksum row).  gather() returns every byte appended,
    attend() matches the oracle, and a chunk takes a handful of copies."""
    print(f"[kv] chunks of {pages_per_chunk} pages cut a record, verify={verify}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(31 + pages_per_chunk)
    B, NQ, NKV, D, PT, S = 2, 8, 2, 64, 32, 32 * 23 + 5
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1,
                      prefetch=False, verify_spills=verify)
    k = torch.randn((B, NKV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, NKV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    kv.append(0, k, v)
    assert kv.spill([(0, i) for i in range(20)]) == 20
    record = kv._pages[0][0].host
    assert all(kv._pages[0][i].host is record for i in range(20)) and record.chunk >= 20
    assert kv.reload([(0, 5), (0, 6)]) == 2
    # a staged page takes the record's bytes per page (checksums included)
    kv._ring.nbytes = pages_per_chunk * record.page_bytes
    with count_staged_copies(kv) as copies:
        K, V = kv.gather(0)
    torch.cuda.synchronize()
    assert torch.equal(bits(K), bits(k)) and torch.equal(bits(V), bits(v))
    # the 18 spilled pages in chunks of n; a run ends at a chunk's end or at
    # the reloaded pages 5-6, and takes 2 tensors x 2 planes (+ 2 checksum
    # rows when verified) copies; page by page it would be that many per page
    spilled = [i for i in range(20) if i not in (5, 6)]
    runs = 0
    for c0 in range(0, len(spilled), pages_per_chunk):
        cp = spilled[c0:c0 + pages_per_chunk]
        runs += 1 + sum(1 for a, b in zip(cp, cp[1:]) if b != a + 1)
    per_run = 6 if verify else 4
    assert len(copies) == runs * per_run, (len(copies), runs)
    q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    out = kv.attend(0, q)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), attn_oracle(q, k, v, D ** -0.5),
                               atol=ATOL, rtol=RTOL)
    kv.release()


@pytest.mark.parametrize("verify", [True, False])
def test_pages_spilled_one_at_a_time_upload_as_strided_runs(verify):
    """The budget spills one page at a time as a decode grows, so each spilled
    page sits in a record of its own, one after another in the arena.  Their
    planes lie at a constant host stride: a staged chunk moves each plane (and
    checksum row) of such a run as one strided transfer instead of one copy
    per page, and the bytes come back exactly."""
    print(f"[kv] one-page records, verify={verify}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(41)
    B, NQ, NKV, D, PT, S = 2, 8, 2, 64, 32, 32 * 34 + 9
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1,
                      prefetch=False, verify_spills=verify)
    k = torch.randn((B, NKV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, NKV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    kv.append(0, k, v)
    for i in range(30):
        assert kv.spill([(0, i)]) == 1
    hosts = [kv._pages[0][i].host for i in range(30)]
    assert len({id(h) for h in hosts}) == 30  # 30 records of one page
    with count_staged_copies(kv) as copies:
        K, V = kv.gather(0)
    torch.cuda.synchronize()
    assert torch.equal(bits(K), bits(k)) and torch.equal(bits(V), bits(v))
    per_run = 6 if verify else 4
    # page by page: 30 * per_run copies; evenly spaced records: one run (a
    # new arena slab would start a second)
    assert len(copies) <= 2 * per_run, copies
    assert all(kind == "rows" for kind, _ in copies) and sum(n for _, n in copies) == 30 * per_run
    q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    out = kv.attend(0, q)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), attn_oracle(q, k, v, D ** -0.5),
                               atol=ATOL, rtol=RTOL)
    # reload(): runs this short go through the staging ring as well (a record
    # kernel launch per page would move too little each)
    with count_staged_copies(kv) as copies:
        assert kv.reload() == 30
    torch.cuda.synchronize()
    assert copies and all(kind == "rows" for kind, _ in copies)
    K, V = kv.gather(0)
    torch.cuda.synchronize()
    assert torch.equal(bits(K), bits(k)) and torch.equal(bits(V), bits(v))
    kv.release()


def attn_oracle(q, K, V, scale):
    """Reference decode over the concatenated K/V [B, NKV, S, D]."""
    B = q.shape[0]
    out = []
    for b in range(B):
        out.append(opa.sdpa_decode(q[b, :, 0].float().cpu().numpy(), K[b].float().cpu().numpy(),
                                   V[b].float().cpu().numpy(), scale))
    return np.stack(out)[:, :, None, :]


@pytest.mark.parametrize("budget_pages", [None, 3])
def test_attend_matches_oracle_with_and_without_spills(budget_pages):
    print(f"[kv] attend budget_pages={budget_pages}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(2)
    B, NQ, NKV, D, PT, layers = 3, 16, 4, 128, 64, 2
    page_bytes = B * NKV * D * 4 * PT
    max_bytes = 1 << 40 if budget_pages is None else budget_pages * page_bytes
    kv = PagedKVCache(num_layers=layers, max_bytes=max_bytes, page_positions=PT,
                      resident_pages=1)
    ks = [[] for _ in range(layers)]
    vs = [[] for _ in range(layers)]
    for chunk in (300, 1, 1, 1, 130, 1):
        for layer in range(layers):
            k = torch.randn((B, NKV, chunk, D), generator=gen, device="cuda").to(torch.bfloat16)
            v = torch.randn((B, NKV, chunk, D), generator=gen, device="cuda").to(torch.bfloat16)
            ks[layer].append(k)
            vs[layer].append(v)
            kv.append(layer, k, v)
        for layer in range(layers):
            q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
            out = kv.attend(layer, q)
            torch.cuda.synchronize()
            ref = attn_oracle(q, torch.cat(ks[layer], 2), torch.cat(vs[layer], 2), D ** -0.5)
            np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    if budget_pages is not None:
        assert kv.stats.spills > 0 and kv.stats.reloads > 0
        assert any(not p.resident for p in kv._pages[0])


def test_reload_restores_pages_bitwise_and_attention():
    print("[kv] explicit spill + reload", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(3)
    B, NQ, NKV, D, PT = 2, 8, 2, 128, 64
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1)
    k = rand_bf16((B, NKV, 500, D), gen)
    v = torch.randn((B, NKV, 500, D), generator=gen, device="cuda").to(torch.bfloat16)
    kf = torch.randn((B, NKV, 500, D), generator=gen, device="cuda").to(torch.bfloat16)
    kv.append(0, kf, v)
    q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    before = kv.attend(0, q).clone()
    originals = [tuple(t.clone() for t in p.load()) for p in kv._pages[0]]
    n = kv.spill([(0, i) for i in range(0, 7, 2)])
    assert n == 4 and not kv._pages[0][0].resident
    spilled_out = kv.attend(0, q)
    assert kv.reload() == 4
    assert all(p.resident for p in kv._pages[0])
    for p, (ko, vo) in zip(kv._pages[0], originals):
        kl, vl = p.load()
        assert torch.equal(bits(kl), bits(ko)) and torch.equal(bits(vl), bits(vo))
    after = kv.attend(0, q)
    torch.cuda.synchronize()
    # same logical pages in new slots: the kernel result is bitwise unchanged
    assert torch.equal(bits(after), bits(before))
    np.testing.assert_allclose(spilled_out.float().cpu().numpy(), before.float().cpu().numpy(),
                               atol=ATOL, rtol=RTOL)
    kv.release()
    assert kv.nbytes() == 0


def test_nbytes_counts_resident_pages_and_tail():
    print("[kv] nbytes accounting", flush=True)
    B, NKV, D, PT = 1, 2, 64, 32
    kv = PagedKVCache(num_layers=2, max_bytes=1 << 40, page_positions=PT)
    x = torch.zeros((B, NKV, 70, D), dtype=torch.bfloat16, device="cuda")
    for layer in range(2):
        kv.append(layer, x, x)
    tok = B * NKV * D * 2 * 2
    assert kv.nbytes() == 2 * 70 * tok
    kv.spill([(0, 0)])
    assert kv.nbytes() == 2 * 70 * tok - PT * tok
    assert kv.offset == 70 and kv.layer_length(0) == 70


# ---- latent (absorbed-MLA) cache -------------------------------------------

def test_latent_update_round_trips_through_spills_bitwise():
    print("[kv-latent] update_latent concatenation + spilled page load", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(4)
    B, R, PT, layers = 2, 576, 64, 2
    kv = PagedKVCache(num_layers=layers, max_bytes=2 * B * R * 2 * PT, page_positions=PT,
                      resident_pages=1)
    chunks = [[] for _ in range(layers)]
    for n in (150, 1, 1, 70, 1):
        for layer in range(layers):
            lat = rand_bf16((B, n, R), gen)
            chunks[layer].append(lat)
            got = kv.update_latent(layer, lat)
            torch.cuda.synchronize()
            assert torch.equal(bits(got), bits(torch.cat(chunks[layer], 1)))
    assert kv.compressed_mla
    assert kv.stats.spills > 0 and kv.stats.reloads > 0
    page = kv._pages[0][0]
    assert not page.resident
    (lat0,) = page.load()
    assert torch.equal(bits(lat0), bits(torch.cat(chunks[0], 1)[:, :PT]))
    with pytest.raises(ValueError):
        kv.attend(0, torch.zeros((B, 8, 1, 64), dtype=torch.bfloat16, device="cuda"))
    kv.release()
    assert kv.nbytes() == 0 and kv.offset == 0


@pytest.mark.parametrize("budget_pages,compress", [(None, False), (2, False), (2, True)])
def test_attend_mla_matches_oracle_with_spills(budget_pages, compress):
    from oracle import mla as omla
    print(f"[kv-latent] attend_mla budget_pages={budget_pages} compress={compress}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    B, H, dn, dv, C, dr, PT = 2, 32, 128, 128, 512, 64, 64
    kv_b = (torch.randn((H * (dn + dv), C), generator=gen, device="cuda") * C ** -0.5
            ).to(torch.bfloat16)
    w_uk, w_uv_t = ops.split_kv_b(kv_b, H, dn, dv)
    page_bytes = B * (C + dr) * 2 * PT
    max_bytes = 1 << 40 if budget_pages is None else budget_pages * page_bytes
    kv = PagedKVCache(num_layers=1, max_bytes=max_bytes, page_positions=PT, resident_pages=1,
                      compress_spill=compress)
    lats = []
    scale = (dn + dr) ** -0.5
    for n in (260, 1, 90, 1):
        lat = torch.randn((B, n, C + dr), generator=gen, device="cuda").to(torch.bfloat16)
        lats.append(lat)
        kv.append_latent(0, lat)
        q_nope = torch.randn((B, H, dn), generator=gen, device="cuda").to(torch.bfloat16)
        q_rope = torch.randn((B, H, dr), generator=gen, device="cuda").to(torch.bfloat16)
        out, wc = kv.attend_mla(0, q_nope, q_rope, w_uk, w_uv_t, scale, return_weighted_c=True)
        torch.cuda.synchronize()
        ref_out, ref_wc = omla.absorbed(
            q_nope.float().cpu().numpy()[:, :, None], q_rope.float().cpu().numpy()[:, :, None],
            torch.cat(lats, 1).float().cpu().numpy(), kv_b.float().cpu().numpy(), dn, dv,
            bf16=True)
        np.testing.assert_allclose(wc.float().cpu().numpy(), ref_wc[:, :, 0], atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref_out[:, :, 0], atol=ATOL,
                                   rtol=RTOL)
    if budget_pages is not None:
        assert kv.stats.spills > 0 and any(not p.resident for p in kv._pages[0])
    if compress:
        assert kv.stats.spill_bytes_compressed > 0


def test_latent_reload_restores_pages_bitwise():
    print("[kv-latent] explicit spill + reload", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(6)
    B, R, PT = 3, 576, 64
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1,
                      compress_spill=True)
    kv.append_latent(0, rand_bf16((B, 400, R), gen))
    originals = [p.load()[0].clone() for p in kv._pages[0]]
    assert kv.spill([(0, 1), (0, 3), (0, 4)]) == 3
    assert kv.nbytes() == (400 - 3 * PT) * B * R * 2
    assert kv.reload() == 3
    for p, o in zip(kv._pages[0], originals):
        assert p.resident and torch.equal(bits(p.load()[0]), bits(o))
    torch.cuda.synchronize()


def test_prefetched_uploads_match_fresh_ones_through_cache_changes():
    print("[kv] cross-layer prefetch vs no prefetch, with spills and reloads between", flush=True)
    B, NQ, NKV, D, PT, layers = 2, 8, 2, 128, 64, 3
    outs = {}
    for prefetch in (True, False):
        gen = torch.Generator(device="cuda").manual_seed(7)
        kv = PagedKVCache(num_layers=layers, max_bytes=1 << 40, page_positions=PT,
                          resident_pages=1, prefetch=prefetch)
        ks = [[] for _ in range(layers)]
        vs = [[] for _ in range(layers)]
        res = []
        for step, n in enumerate((400, 1, 1, 70, 1, 1)):
            for layer in range(layers):
                k = torch.randn((B, NKV, n, D), generator=gen, device="cuda").to(torch.bfloat16)
                v = torch.randn((B, NKV, n, D), generator=gen, device="cuda").to(torch.bfloat16)
                ks[layer].append(k)
                vs[layer].append(v)
                kv.append(layer, k, v)
            if step == 0:
                kv.spill([(l, i) for l in range(layers) for i in range(0, 5)])
            if step == 3:
                kv.reload([(1, 2), (2, 0)])
                kv.spill([(0, 5), (2, 6)])
            for layer in range(layers):
                q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
                out = kv.attend(layer, q)
                res.append(out.clone())
                if prefetch:
                    ref = attn_oracle(q, torch.cat(ks[layer], 2), torch.cat(vs[layer], 2),
                                      D ** -0.5)
                    torch.cuda.synchronize()
                    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL,
                                               rtol=RTOL)
        torch.cuda.synchronize()
        outs[prefetch] = res
        if prefetch:
            assert kv.prefetch_hits > 0
        else:
            assert kv.prefetch_hits == 0
        kv.release()
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(bits(a), bits(b))


# ---- disk tier (spill_dir) -------------------------------------------------

@pytest.mark.parametrize("compress", [False, True])
def test_spill_dir_writes_page_files_like_the_reference(tmp_path, compress):
    # mirrors tests/test_kv_spill_compress.py:22-60 of the reference
    print(f"[kv-disk] reference protocol with spill_dir compress={compress}", flush=True)
    spill_dir = tmp_path / "spill"
    kv = PagedKVCache(num_layers=2, max_bytes=1, spill_dir=spill_dir, page_positions=4,
                      resident_pages=0, compress_spill=compress)
    gen = torch.Generator(device="cuda").manual_seed(0)
    ref_k, ref_v = [], []
    for layer in range(2):
        k = rand_bf16((1, 2, 4, 8), gen)
        v = rand_bf16((1, 2, 4, 8), gen)
        ref_k.append(k)
        ref_v.append(v)
        kv.update(layer, k, v)
    for layer in range(2):
        kv.update(layer, rand_bf16((1, 2, 1, 8), gen), rand_bf16((1, 2, 1, 8), gen))
    assert kv.stats.spills > 0
    page = kv._pages[0][0]
    assert not page.resident
    lk, lv = page.load()
    torch.cuda.synchronize()
    assert torch.equal(bits(lk), bits(ref_k[0])) and torch.equal(bits(lv), bits(ref_v[0]))
    spill_paths = [p.path for pages in kv._pages for p in pages if p.path is not None]
    assert spill_paths and all(path.exists() for path in spill_paths)
    assert page.path.name == "kv_l0_p0.vt"
    kv.release()
    assert kv.offset == 0 and kv.nbytes() == 0
    assert not any(path.exists() for path in spill_paths)


def test_incompressible_high_planes_stay_raw(tmp_path):
    # runtime/warm_tier.py:56,79-81: a page that barely compresses is not kept
    # compressed.  K of random bit patterns has random high bytes (ratio ~1);
    # V of small values has high bytes of a few exponents (ratio well above
    # 1.15).  Both come back bit-exact from the page files alone.
    import json
    import struct

    print("[kv-disk] zstd admission: incompressible high planes stay raw", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(21)
    B, NKV, D, PT = 1, 2, 64, 16
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, spill_dir=tmp_path, page_positions=PT,
                      resident_pages=0, compress_spill=True, host_max_bytes=1)
    k = torch.randint(-32768, 32768, (B, NKV, 2 * PT, D), generator=gen, device="cuda",
                      dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = (torch.randn((B, NKV, 2 * PT, D), generator=gen, device="cuda") * 0.01).to(
        torch.bfloat16)
    kv.append(0, k, v)
    originals = [tuple(t.clone() for t in p.load()) for p in kv._pages[0]]
    kv.spill([(0, 0), (0, 1)])  # host_max_bytes=1: the files are written, host copies dropped
    for i, page in enumerate(kv._pages[0]):
        assert page.path is not None and page.host is None  # on disk only
        with open(page.path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            head = json.loads(f.read(n))
        hz = {t["name"]: t["hi_z"] for t in head["tensors"]}
        assert hz["k"] is None, hz
        assert hz["v_t"] is not None and hz["v_t"] * 1.15 <= head["tensors"][1]["hi"], hz
        lk, lv = page.load()
        torch.cuda.synchronize()
        assert torch.equal(bits(lk), bits(originals[i][0]))
        assert torch.equal(bits(lv), bits(originals[i][1]))
    kv.release()


def test_host_budget_moves_pages_to_disk_and_back(tmp_path):
    print("[kv-disk] host_max_bytes evicts host copies; attend/load/reload from files", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    B, NQ, NKV, D, PT = 2, 8, 2, 128, 64
    page_bytes = B * NKV * D * 4 * PT
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, spill_dir=tmp_path,
                      page_positions=PT, resident_pages=1, compress_spill=True,
                      host_max_bytes=2 * page_bytes)
    k = rand_bf16((B, NKV, 640, D), gen)
    v = torch.randn((B, NKV, 640, D), generator=gen, device="cuda").to(torch.bfloat16)
    kf = torch.randn((B, NKV, 640, D), generator=gen, device="cuda").to(torch.bfloat16)
    kv.append(0, kf, v)
    originals = [tuple(t.clone() for t in p.load()) for p in kv._pages[0]]
    q = torch.randn((B, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    before = kv.attend(0, q).clone()
    # three separate spills: the oldest host blocks go over the host budget
    kv.spill([(0, i) for i in (0, 1, 2)])
    kv.spill([(0, i) for i in (3, 4)])
    kv.spill([(0, i) for i in (5, 6)])
    pages = kv._pages[0]
    assert all(p.path is not None and p.path.exists() for p in pages[:7])
    assert kv.arena.used_bytes <= 2 * page_bytes
    disk_only = [p for p in pages[:7] if p.host is None]
    assert len(disk_only) >= 3
    for p in pages[:7]:
        kl, vl = p.load()
        assert torch.equal(bits(kl), bits(originals[p.index][0]))
        assert torch.equal(bits(vl), bits(originals[p.index][1]))
    spilled_out = kv.attend(0, q)
    torch.cuda.synchronize()
    np.testing.assert_allclose(spilled_out.float().cpu().numpy(),
                               before.float().cpu().numpy(), atol=ATOL, rtol=RTOL)
    files = [p.path for p in pages[:7]]
    assert kv.reload() == 7
    assert all(p.resident and p.path is None for p in pages)
    assert not any(f.exists() for f in files)
    after = kv.attend(0, q)
    torch.cuda.synchronize()
    assert torch.equal(bits(after), bits(before))
    kv.release()


@pytest.mark.parametrize("B,H,offset,L,spill", [(1, 64, 3, 5, False), (1, 128, 0, 64, False),
                                                (2, 64, 150, 40, True)])
def test_attend_mla_prefill_is_causal_absorbed_mla(B, H, offset, L, spill):
    """attend_mla_prefill against oracle/mla.absorbed with L > 1 (the causal
    branch of runtime/glm.py:142-153): the reference known-answer test's
    query window (L = 5 after 3 cached tokens, tests/test_mla_absorbed.py:
    115-222) at the kernel's latent width, a 64-token prompt at 128 heads, and
    a window over spilled pages.  2e-2 abs / 1e-2 rel in bf16."""
    from oracle import mla as omla
    print(f"[kv-latent] attend_mla_prefill B={B} H={H} offset={offset} L={L} spill={spill}",
          flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11 + L)
    dn, dv, C, dr, PT = 128, 128, 512, 64, 64
    kv_b = (torch.randn((H * (dn + dv), C), generator=gen, device="cuda") * C ** -0.5
            ).to(torch.bfloat16)
    w_uk, w_uv_t = ops.split_kv_b(kv_b, H, dn, dv)
    page_bytes = B * (C + dr) * 2 * PT
    kv = PagedKVCache(num_layers=1, max_bytes=(2 * page_bytes if spill else 1 << 40),
                      page_positions=PT, resident_pages=1)
    lat = torch.randn((B, offset + L, C + dr), generator=gen, device="cuda").to(torch.bfloat16)
    if offset:
        kv.append_latent(0, lat[:, :offset])
    kv.append_latent(0, lat[:, offset:])
    if spill:
        assert any(not p.resident for p in kv._pages[0])
    q_nope = torch.randn((B, H, L, dn), generator=gen, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn((B, H, L, dr), generator=gen, device="cuda").to(torch.bfloat16)
    scale = (dn + dr) ** -0.5
    out, wc = kv.attend_mla_prefill(0, q_nope, q_rope, w_uk, w_uv_t, scale,
                                    return_weighted_c=True)
    torch.cuda.synchronize()
    assert out.shape == (B, H, L, dv) and wc.shape == (B, H, L, C)
    ref_out, ref_wc = omla.absorbed(q_nope.float().cpu().numpy(), q_rope.float().cpu().numpy(),
                                    lat.float().cpu().numpy(), kv_b.float().cpu().numpy(), dn, dv,
                                    offset=offset, bf16=True)
    np.testing.assert_allclose(wc.float().cpu().numpy(), ref_wc, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
    kv.release()


def test_attend_mla_prefill_of_one_token_is_attend_mla_bitwise():
    print("[kv-latent] attend_mla_prefill L=1 vs attend_mla", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(12)
    B, H, dn, dv, C, dr, PT = 3, 128, 128, 128, 512, 64, 64
    kv_b = (torch.randn((H * (dn + dv), C), generator=gen, device="cuda") * C ** -0.5
            ).to(torch.bfloat16)
    w_uk, w_uv_t = ops.split_kv_b(kv_b, H, dn, dv)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT)
    kv.append_latent(0, torch.randn((B, 777, C + dr), generator=gen, device="cuda")
                     .to(torch.bfloat16))
    q_nope = torch.randn((B, H, 1, dn), generator=gen, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn((B, H, 1, dr), generator=gen, device="cuda").to(torch.bfloat16)
    scale = (dn + dr) ** -0.5
    a, wa = kv.attend_mla_prefill(0, q_nope, q_rope, w_uk, w_uv_t, scale, return_weighted_c=True)
    b, wb = kv.attend_mla(0, q_nope[:, :, 0], q_rope[:, :, 0], w_uk, w_uv_t, scale,
                          return_weighted_c=True)
    assert torch.equal(bits(a[:, :, 0]), bits(b)) and torch.equal(bits(wa[:, :, 0]), bits(wb))
    kv.release()


def test_side_stream_does_not_queue_behind_the_current_stream():
    """The cache's upload stream is checked against the current stream's
    hardware queue: whatever number of streams the process made before, a
    marker on it completes while work enqueued earlier on the current stream
    is still running (on a shared queue it would wait for that work)."""
    from voom_amd.kv_paged import _side_stream_off_queue

    print("[kv] side stream off the current stream's queue", flush=True)
    dev = torch.device("cuda")
    main = torch.cuda.current_stream()
    scratch = torch.empty(32 << 20, dtype=torch.int32, device="cuda")
    for extra in range(6):
        for _ in range(extra):  # shift where the next new stream lands
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                torch.zeros(8, device="cuda").add_(1)
        torch.cuda.synchronize()
        side = _side_stream_off_queue(dev)
        start, busy_end, marker = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        start.record(main)
        for _ in range(20):
            scratch.fill_(2)
        busy_end.record(main)
        marker.record(side)
        torch.cuda.synchronize()
        busy = start.elapsed_time(busy_end)
        assert busy > 0.1, busy
        assert start.elapsed_time(marker) < 0.5 * busy, (extra, start.elapsed_time(marker), busy)
