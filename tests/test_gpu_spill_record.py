"""The spill-record kernels (voom_spill_record / voom_reload_record): the split
writes byte planes and checksums straight into a pinned host record, the merge
reads them back from it.  The record must equal, byte for byte, the staging
layout the slot codec produces (voom_byteplane_split_slots, whose planes are
pinned to the reference's lo = raw[0::2], hi = raw[1::2], formats/packed.py:
49-50, and whose checksums are pinned to oracle/page_sums.py); the merge must
restore the slots bitwise and count every damaged slot."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import page_sums as osums
from voom_amd import _lib, ops
from voom_amd.kv_paged import PagedKVCache

pytestmark = pytest.mark.gpu


def rand_bits(shape, gen):
    return torch.randint(-32768, 32768, shape, generator=gen, dtype=torch.int32,
                         device="cuda").to(torch.int16)


def staged_record(pools, slots):
    """The record as the slot codec stages it: low planes of every tensor, then
    high planes, then int32 [T, n] checksums."""
    n = slots.numel()
    lows, highs, sums = [], [], []
    for pool in pools:
        half = pool[0].numel()
        lo = torch.empty(n * half, dtype=torch.uint8, device="cuda")
        hi = torch.empty_like(lo)
        s = torch.zeros(n, dtype=torch.int32, device="cuda")
        ops.byteplane_split_slots(pool, slots, lo, hi, sums=s)
        lows.append(lo)
        highs.append(hi)
        sums.append(s.view(torch.uint8))
    return torch.cat(lows + highs + sums)


GEOMS = [[(2, 64, 128)], [(2, 64, 128), (2, 2, 128, 32)], [(64, 576)], [(4, 8, 8)],
         [(4, 8, 8), (1, 32), (3, 64), (2, 96)]]


@pytest.mark.parametrize("geom", GEOMS)
def test_record_equals_the_staged_codec_and_round_trips(geom):
    print(f"[record] geometry {geom}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(60 + len(geom))
    pools = [rand_bits((50,) + shp, gen) for shp in geom]
    slots = torch.tensor([7, 0, 49, 12, 12, 5, 33], dtype=torch.int32, device="cuda")
    n = slots.numel()
    rec = torch.full((ops.record_bytes(pools, n, True),), 0xAB, dtype=torch.uint8,
                     pin_memory=True)
    ops.spill_record(pools, slots, rec, sums=True)
    want = staged_record(pools, slots)
    torch.cuda.synchronize()
    assert torch.equal(rec, want.cpu())
    # checksums against the CPU restatement
    sums = rec[-4 * n * len(pools):].view(torch.int32).view(len(pools), n).numpy()
    for t, pool in enumerate(pools):
        ref = osums.slot_sums(pool.cpu().numpy().view(np.uint16), slots.cpu().numpy())
        assert np.array_equal(sums[t], ref)
    # reload into other slots of fresh pools, verified
    dest = [torch.zeros_like(p) for p in pools]
    tgt = torch.tensor([1, 2, 3, 4, 6, 8, 10], dtype=torch.int32, device="cuda")
    status = torch.zeros(2, dtype=torch.int32, device="cuda")
    ops.reload_record(rec, dest, tgt, tag=5, status=status)
    torch.cuda.synchronize()
    assert status.tolist() == [0, 0]
    for pool, d in zip(pools, dest):
        assert torch.equal(d[tgt.long()], pool[slots.long()])
        untouched = torch.ones(50, dtype=torch.bool)
        untouched[tgt.long().cpu()] = False
        assert bool((d[untouched.cuda()] == 0).all())


def test_sub_range_of_a_device_record():
    print("[record] sub-range of a larger device record", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(70)
    pools = [rand_bits((20, 2, 64, 128), gen), rand_bits((20, 2, 2, 128, 32), gen)]
    all_slots = torch.arange(10, dtype=torch.int32, device="cuda") * 2
    full = torch.empty(ops.record_bytes(pools, 10, True), dtype=torch.uint8, device="cuda")
    ops.spill_record(pools, all_slots, full, sums=True)
    # the same record written in three pieces equals the one-shot record
    pieces = torch.full_like(full, 0x5A)
    host_slots = all_slots.cpu().pin_memory()  # read by the kernel from host memory
    for a, b in ((0, 3), (3, 4), (4, 10)):
        ops.spill_record(pools, host_slots[a:b], pieces, rec_slots=10, first=a, sums=True)
    torch.cuda.synchronize()
    assert torch.equal(pieces, full)
    # reload slots 4..7 of the record only
    dest = [torch.zeros_like(p) for p in pools]
    tgt = torch.tensor([19, 0, 3, 11], dtype=torch.int32, device="cuda")
    status = torch.zeros(2, dtype=torch.int32, device="cuda")
    ops.reload_record(full, dest, tgt, rec_slots=10, first=4, tag=3, status=status)
    torch.cuda.synchronize()
    assert status.tolist() == [0, 0]
    for pool, d in zip(pools, dest):
        assert torch.equal(d[tgt.long()], pool[all_slots[4:8].long()])


def test_reload_counts_each_damaged_slot():
    print("[record] damaged plane bytes and checksum words", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(71)
    pools = [rand_bits((16, 4, 64, 32), gen), rand_bits((16, 4, 2, 32, 32), gen)]
    slots = torch.arange(8, dtype=torch.int32, device="cuda")
    n, half = 8, pools[0][0].numel()
    rec = torch.empty(ops.record_bytes(pools, n, True), dtype=torch.uint8, pin_memory=True)
    ops.spill_record(pools, slots, rec, sums=True)
    torch.cuda.synchronize()
    rec[3 * half + 17] ^= 0x01            # tensor 0, low plane of slot 3
    rec[2 * n * half + 5 * half] ^= 0x80  # tensor 0, high plane of slot 5
    rec[4 * n * half + 4 * n + 4 * 6] ^= 0x02  # tensor 1's checksum of slot 6
    status = torch.zeros(2, dtype=torch.int32, device="cuda")
    ops.reload_record(rec, [torch.zeros_like(p) for p in pools], slots, tag=9, status=status)
    torch.cuda.synchronize()
    assert status.tolist() == [3, 9]


def test_refuses_pageable_short_and_misaligned_records():
    print("[record] pageable / short / misaligned records refused before any launch", flush=True)
    pools = [torch.zeros((4, 64, 32), dtype=torch.bfloat16, device="cuda")]
    slots = torch.arange(4, dtype=torch.int32, device="cuda")
    need = ops.record_bytes(pools, 4, True)
    ptrs = (ctypes.c_void_p * 1)(pools[0].data_ptr())
    sbytes = (ctypes.c_size_t * 1)(64 * 32 * 2)
    counts = (ctypes.c_int * 1)(4)
    stream = torch.cuda.current_stream().cuda_stream

    def spill(ptr, first=0):
        _lib.call("voom_spill_record", ctypes.cast(ptrs, ctypes.c_void_p),
                  ctypes.addressof(sbytes), ctypes.addressof(counts), 1, slots.data_ptr(), 4,
                  ptr, 4, first, 1, stream)

    pageable = np.zeros(need + 64, dtype=np.uint8)
    with pytest.raises(ValueError, match="pinned host or device memory"):
        spill(pageable.ctypes.data)
    # a record whose last 64 bytes lie past the end of an exact pinned allocation
    hip = ctypes.CDLL("libamdhip64.so")
    base = ctypes.c_void_p()
    size = 1 << 20
    assert hip.hipHostMalloc(ctypes.byref(base), ctypes.c_size_t(size), 0) == 0
    try:
        with pytest.raises(ValueError, match="past the end of its allocation"):
            spill(base.value + size - need + 64)
    finally:
        hip.hipHostFree(base)
    ok = torch.empty(need + 256, dtype=torch.uint8, pin_memory=True)
    pageable_slots = np.arange(4, dtype=np.int32)
    with pytest.raises(ValueError, match="slot list must be pinned host or device memory"):
        _lib.call("voom_spill_record", ctypes.cast(ptrs, ctypes.c_void_p),
                  ctypes.addressof(sbytes), ctypes.addressof(counts), 1,
                  pageable_slots.ctypes.data, 4, ok.data_ptr(), 4, 0, 1, stream)
    with pytest.raises(ValueError, match="16-byte aligned"):
        spill(ok.data_ptr() + 8)
    with pytest.raises(ValueError, match="outside the record"):
        spill(ok.data_ptr(), first=1)
    with pytest.raises(ValueError):
        ops.spill_record(pools, slots, torch.empty(need, dtype=torch.uint8), sums=True)
    spill(ok.data_ptr())  # a well-formed call still goes through
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", ["kv", "latent"])
def test_cache_record_path_equals_the_staged_path(kind):
    """PagedKVCache through the record kernels and through the staging ring and
    copy engine: identical host records, identical reloaded pools."""
    print(f"[record] cache paths agree ({kind})", flush=True)
    caches = []
    for direct in (True, False):
        gen = torch.Generator(device="cuda").manual_seed(72)
        kv = PagedKVCache(num_layers=2, max_bytes=1 << 40, page_positions=64, resident_pages=1)
        kv.direct_host = direct
        kv.record_run_bytes = 0  # every run through the record kernels when direct
        for layer in range(2):
            if kind == "kv":
                kv.append(layer, rand_bits((2, 2, 400, 128), gen).view(torch.bfloat16),
                          rand_bits((2, 2, 400, 128), gen).view(torch.bfloat16))
            else:
                kv.append_latent(layer, rand_bits((2, 300, 576), gen).view(torch.bfloat16))
        kv.spill([(1, 0), (1, 2), (1, 3), (0, 1)])
        torch.cuda.synchronize()
        caches.append(kv)
    a, b = caches
    for layer, idx in ((1, 0), (1, 2), (1, 3), (0, 1)):
        pa, pb = a._pages[layer][idx], b._pages[layer][idx]
        T = len(pa.host.parts)
        for w in range(2 * T):
            assert torch.equal(pa.host.part(w, pa.host_j), pb.host.part(w, pb.host_j))
        assert torch.equal(pa.host.sums(pa.host_j), pb.host.sums(pb.host_j))
    # partial reload (one page of a record), then the rest
    assert a.reload([(1, 2)]) == b.reload([(1, 2)]) == 1
    assert a.reload() == b.reload() == 3
    torch.cuda.synchronize()
    for layer in range(2):
        if kind == "kv":
            ga, gb = a.gather(layer), b.gather(layer)
        else:
            ga, gb = (a.gather_latent(layer),), (b.gather_latent(layer),)
        for x, y in zip(ga, gb):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    a.release()
    b.release()
