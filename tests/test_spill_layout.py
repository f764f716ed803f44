"""Host-side layout of spill blocks and records (no GPU): records start on
256-byte boundaries, a block holds exactly its records, and the record size the
kernels expect (ops.record_bytes) is the per-page record size the cache plans
with (record_page_bytes) times the pages."""
import pytest

from voom_amd import ops
from voom_amd.kv_paged import block_bytes, record_page_bytes, record_stride
from voom_amd.page_pool import DevicePagePool


@pytest.mark.parametrize("n,chunk,page_bytes", [(256, 1023, 262152), (3000, 1023, 262152),
                                                (7, 3, 4104), (1, 1, 72), (9, 3, 1000)])
def test_records_are_aligned_and_packed(n, chunk, page_bytes):
    stride = record_stride(chunk, page_bytes)
    assert stride % 256 == 0 and 0 <= stride - chunk * page_bytes < 256
    n_rec = -(-n // chunk)
    last = n - (n_rec - 1) * chunk
    # the last record ends exactly at the block's end
    assert block_bytes(n, chunk, page_bytes) == (n_rec - 1) * stride + last * page_bytes
    for r in range(n_rec):
        assert (r * stride) % 256 == 0


@pytest.mark.parametrize("B", [1, 3])
def test_record_bytes_match_the_cache_plan(B):
    pool = DevicePagePool.kv(8, 128, 64, capacity=4, device="cpu")
    parts = [B * pool.tensor_slot_bytes(t) // 2 for t in range(2)]
    nsum = B * 2
    pages = 5
    assert ops.record_bytes(pool.tensors, pages * B, True) == \
        pages * record_page_bytes(parts, nsum)
    assert ops.record_bytes(pool.tensors, pages * B, False) == \
        pages * record_page_bytes(parts, 0)
    lat = DevicePagePool.rows(64, 576, capacity=2, device="cpu")
    assert ops.record_bytes(lat.tensors, 4, True) == 4 * (64 * 576 * 2 + 4)
