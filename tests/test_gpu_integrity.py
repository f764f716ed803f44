"""Spill integrity on the GPU: the split kernel's per-slot checksums equal the
CPU restatement (oracle/page_sums.py); a spilled page whose host bytes, zstd
frame, page file or stored checksum changed is refused on reload with
KVIntegrityError naming the page, on the explicit reload and on attention's
transient reload alike (the pattern of the reference's durability tests,
tests/test_hot_kv_durability.py:142-170, which flip one byte of a stored
payload and expect it to be rejected)."""
import numpy as np
import pytest
import torch

from oracle import page_sums as ops_
from voom_amd import ops
from voom_amd.kv_paged import KVIntegrityError, PagedKVCache

pytestmark = pytest.mark.gpu


def randn_bf16(shape, gen):
    return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)


def rand_bits(shape, gen):
    return torch.randint(-32768, 32768, shape, generator=gen, dtype=torch.int32,
                         device="cuda").to(torch.int16)


@pytest.mark.parametrize("slot_shape", [(2, 64, 128), (64, 576), (4, 8, 8)])
def test_split_and_merge_checksums_match_the_oracle(slot_shape):
    print(f"[sums] slot shape {slot_shape}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(50)
    pool = rand_bits((40,) + slot_shape, gen)
    slots = torch.tensor([7, 0, 39, 12, 12, 5], dtype=torch.int32, device="cuda")
    n, elems = slots.numel(), pool[0].numel()
    lo = torch.empty(n * elems, dtype=torch.uint8, device="cuda")
    hi = torch.empty_like(lo)
    sums = torch.zeros(n, dtype=torch.int32, device="cuda")
    ops.byteplane_split_slots(pool, slots, lo, hi, sums=sums)
    dest = torch.zeros_like(pool)
    back = torch.zeros(n, dtype=torch.int32, device="cuda")
    tgt = torch.tensor([1, 2, 3, 4, 5, 6], dtype=torch.int32, device="cuda")
    ops.byteplane_merge_slots(lo, hi, dest, tgt, sums=back)
    torch.cuda.synchronize()
    want = ops_.slot_sums(pool.cpu().numpy().view(np.uint16), slots.cpu().numpy())
    assert np.array_equal(sums.cpu().numpy(), want)
    assert np.array_equal(back.cpu().numpy(), want)
    status = torch.zeros(2, dtype=torch.int32, device="cuda")
    ops.page_sums_verify(sums, back, 7, status)
    assert status.tolist() == [0, 0]
    back[3] += 1
    back[5] -= 1
    ops.page_sums_verify(sums, back, 9, status)
    ops.page_sums_verify(sums, back, 11, status)
    assert status.tolist() == [4, 9]


def make_cache(gen, **kw):
    kv = PagedKVCache(num_layers=2, max_bytes=1 << 40, page_positions=64, resident_pages=1,
                      **kw)
    data = []
    for layer in range(2):
        k = randn_bf16((2, 2, 400, 128), gen)
        v = randn_bf16((2, 2, 400, 128), gen)
        kv.append(layer, k, v)
        data.append((k, v))
    return kv, data


@pytest.mark.parametrize("record_run_bytes", [0, 1 << 40])  # record kernels / staging ring
def test_corrupt_host_byte_is_refused_on_reload(record_run_bytes):
    print(f"[integrity] host arena byte flip, record_run_bytes={record_run_bytes}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(51)
    kv, _ = make_cache(gen)
    kv.record_run_bytes = record_run_bytes
    kv.spill([(1, i) for i in (0, 1, 2, 3)])
    torch.cuda.synchronize()
    p = kv._pages[1][2]
    plane = p.host.part(1, p.host_j)  # low plane of V^T
    plane[1000] ^= 0x10
    with pytest.raises(KVIntegrityError, match=r"layer 1, pages \[0, 1, 2, 3\]"):
        kv.reload()
    # the error is cleared once raised; clean pages reload quietly afterwards
    kv.spill([(0, 1)])
    assert kv.reload() == 1
    kv.release()


@pytest.mark.parametrize("record_run_bytes", [0, 1 << 40])  # record kernels / staging ring
def test_corrupt_checksum_word_is_refused(record_run_bytes):
    print(f"[integrity] stored checksum changed, record_run_bytes={record_run_bytes}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(52)
    kv, _ = make_cache(gen)
    kv.record_run_bytes = record_run_bytes
    kv.spill([(0, 3)])
    torch.cuda.synchronize()
    p = kv._pages[0][3]
    p.host.sums(p.host_j)[0, 1] += 1
    with pytest.raises(KVIntegrityError):
        kv.reload()
    kv.release()


def test_attention_reload_reports_at_the_next_call():
    print("[integrity] transient reload inside attend", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(53)
    kv, _ = make_cache(gen, prefetch=False)
    kv.spill([(0, i) for i in range(4)])
    torch.cuda.synchronize()
    q = randn_bf16((2, 8, 1, 128), gen)
    kv.attend(0, q)
    kv.check_integrity()  # clean
    p = kv._pages[0][1]
    p.host.part(2, p.host_j)[5] ^= 0x80  # high plane of K
    kv.attend(0, q)
    with pytest.raises(KVIntegrityError, match="layer 0"):
        kv.check_integrity()
    kv.release()


def test_damaged_zstd_frame_in_a_page_file_is_refused(tmp_path):
    print("[integrity] damaged zstd frame in a page file", flush=True)
    import struct

    gen = torch.Generator(device="cuda").manual_seed(54)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, spill_dir=tmp_path, page_positions=64,
                      resident_pages=1, compress_spill=True, host_max_bytes=1)
    kv.append(0, randn_bf16((2, 2, 400, 128), gen), randn_bf16((2, 2, 400, 128), gen))
    kv.spill([(0, 0), (0, 1)])
    p = kv._pages[0][1]
    assert p.host is None and p.path is not None  # on disk only, high planes compressed
    raw = bytearray(p.path.read_bytes())
    (hlen,) = struct.unpack("<Q", raw[:8])
    raw[8 + hlen + 40] ^= 0xFF  # inside the first tensor's zstd frame
    p.path.write_bytes(bytes(raw))
    with pytest.raises(KVIntegrityError, match="layer 0"):
        kv.reload()
    assert kv.stats.spill_bytes_compressed > 0
    kv.release()


@pytest.mark.parametrize("damage", ["flip", "truncate"])
def test_damaged_page_file_is_refused(tmp_path, damage):
    print(f"[integrity] page file {damage}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(55)
    page_bytes = 2 * 2 * 128 * 4 * 64
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, spill_dir=tmp_path, page_positions=64,
                      resident_pages=1, host_max_bytes=page_bytes)
    kv.append(0, randn_bf16((2, 2, 400, 128), gen), randn_bf16((2, 2, 400, 128), gen))
    kv.spill([(0, 0), (0, 1)])
    kv.spill([(0, 2), (0, 3)])
    pages = kv._pages[0]
    disk_only = [p for p in pages[:4] if p.host is None]
    assert disk_only
    path = disk_only[0].path
    raw = bytearray(path.read_bytes())
    if damage == "flip":
        raw[-100] ^= 0x01  # inside the last low plane: same size, wrong bytes
    else:
        raw = raw[:-100]
    path.write_bytes(bytes(raw))
    with pytest.raises(KVIntegrityError, match="layer 0") as err:
        kv.reload()
    assert str(disk_only[0].index) in str(err.value)
    kv.release()
