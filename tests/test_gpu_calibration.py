"""The calibration kernels bench.py times for its floors read every byte they
claim to: the XOR folded into their sinks equals the XOR of the 32-bit words
of the same bytes computed on the host (voom_stream_read, voom_gather_read),
and voom_tile_read stores each wavefront's fold into that wavefront's rows."""
import numpy as np
import pytest
import torch

from voom_amd import calibrate, ops

pytestmark = pytest.mark.gpu


def xor_words(t: torch.Tensor) -> int:
    w = t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32)
    return int(np.bitwise_xor.reduce(w.ravel(), initial=np.uint32(0)))


def sink_xor(sink: torch.Tensor) -> int:
    return xor_words(sink)


@pytest.mark.parametrize("nbytes,wgs", [(1 << 20, 512), ((1 << 20) + 48, 7), (16, 3)])
def test_stream_read_reads_every_word(nbytes, wgs):
    g = torch.Generator(device="cuda").manual_seed(nbytes)
    buf = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=g)
    sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
    calibrate.stream_read(buf, sink, workgroups=wgs)
    torch.cuda.synchronize()
    assert sink_xor(sink) == xor_words(buf)


@pytest.mark.parametrize("row_kib,two", [(1, False), (2, True), (4, True), (3, False)])
def test_gather_read_reads_the_listed_rows(row_kib, two):
    g = torch.Generator(device="cuda").manual_seed(row_kib)
    rows = 300
    base = torch.randint(0, 256, (rows, 1024 * row_kib), dtype=torch.uint8, device="cuda",
                         generator=g)
    base2 = torch.randint(0, 256, base.shape, dtype=torch.uint8, device="cuda",
                          generator=g) if two else None
    idx = torch.randint(0, rows, (1000,), dtype=torch.int32, device="cuda", generator=g)
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    calibrate.gather_read(base, idx, sink, base2=base2, workgroups=64)
    torch.cuda.synchronize()
    want = xor_words(base[idx.long()])
    if two:
        want ^= xor_words(base2[idx.long()])
    assert sink_xor(sink) == want


@pytest.mark.parametrize("ranges,groups", [(3, 2), (4, 1)])
def test_tile_read_stores_its_fold(ranges, groups):
    g = torch.Generator(device="cuda").manual_seed(ranges * 10 + groups)
    slots, B, pages = 20, 2, 8
    pool = torch.randn((slots, 64, 576), generator=g, device="cuda").to(torch.bfloat16)
    table = torch.randperm(slots, generator=g, device="cuda")[:B * pages].to(torch.int32)
    table = table.reshape(B, pages).contiguous()
    q = torch.randn((B, 64 * groups, 576), generator=g, device="cuda").to(torch.bfloat16)
    grid = B * ranges * groups
    rows = torch.empty(grid * 64 * 512, dtype=torch.float16, device="cuda")
    sink = torch.zeros(grid, dtype=torch.int32, device="cuda")
    calibrate.tile_read(pool, table, 64 * pages - 5, ranges, groups, rows, sink, q=q)
    torch.cuda.synchronize()
    # wavefront w stores its own fold into rows 16 w .. 16 w + 15 of the
    # workgroup; the sink holds wavefront 0's
    got = rows.view(torch.int32).reshape(grid, 4, -1)
    assert torch.equal(got, got[:, :, :1].expand_as(got))
    assert torch.equal(got[:, 0, 0], sink)
