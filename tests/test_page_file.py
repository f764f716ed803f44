"""Page files of the disk spill tier (voom_amd/page_file.py): vpack framing
(formats/packed.py:8-11, 57-59) -- header length, JSON header, then per tensor
the high plane (raw or zstd) and the raw low plane -- round-trips exactly."""
import json
import struct

import numpy as np
import pytest

from oracle import byteplane as ob
from voom_amd import page_file
from voom_amd import zstd as vz


def planes(words):
    lo, hi = ob.split(words)
    return lo, hi


@pytest.mark.parametrize("compressed", [False, True])
def test_round_trip_and_header(tmp_path, compressed):
    if compressed and not vz.available():
        pytest.skip("libzstd not present")
    rng = np.random.default_rng(0)
    k = rng.integers(0, 1 << 16, size=2 * 4 * 8, dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=2 * 8 * 4, dtype=np.uint16)
    (klo, khi), (vlo, vhi) = planes(k), planes(v)
    his = [vz.compress(khi, 1), vz.compress(vhi, 1)] if compressed else [khi, vhi]
    meta = [{"name": "k", "dtype": "BF16", "shape": [1, 2, 4, 8]},
            {"name": "v", "dtype": "BF16", "shape": [1, 2, 1, 8, 4]}]
    path = page_file.page_path(tmp_path, 3, 7)
    assert path.name == "kv_l3_p7.vt"
    n = page_file.write(path, 3, 7, meta, [klo, vlo], his, [compressed] * 2)
    assert path.stat().st_size == n
    raw = path.read_bytes()
    (hlen,) = struct.unpack("<Q", raw[:8])
    head = json.loads(raw[8:8 + hlen])
    assert head["format"] == "voom-kv-page" and head["layer"] == 3 and head["page"] == 7
    assert head["version"] == page_file.VERSION
    assert [t["shape"] for t in head["tensors"]] == [[1, 2, 4, 8], [1, 2, 1, 8, 4]]
    assert (head["tensors"][0]["hi_z"] is not None) == compressed
    # payload order per tensor: high plane, then low plane
    body = raw[8 + hlen:]
    assert body[:len(his[0])] == bytes(np.asarray(his[0]))
    lo = [np.empty_like(klo), np.empty_like(vlo)]
    hi = [np.empty_like(khi), np.empty_like(vhi)]
    page_file.read(path, lo, hi)
    assert np.array_equal(ob.merge(lo[0], hi[0]), k)
    assert np.array_equal(ob.merge(lo[1], hi[1]), v)


def test_rejects_malformed_files(tmp_path):
    path = tmp_path / "bad.vt"
    path.write_bytes(b"\x03\x00")
    with pytest.raises(ValueError):
        page_file.read(path, [np.empty(4, np.uint8)], [np.empty(4, np.uint8)])
    meta = [{"name": "latent", "dtype": "BF16", "shape": [1, 2, 2]}]
    good = tmp_path / "kv_l0_p0.vt"
    page_file.write(good, 0, 0, meta, [np.zeros(4, np.uint8)], [np.ones(4, np.uint8)], [False])
    with pytest.raises(ValueError):  # plane size differs from the page geometry
        page_file.read(good, [np.empty(8, np.uint8)], [np.empty(8, np.uint8)])
    trunc = tmp_path / "kv_l0_p1.vt"
    trunc.write_bytes(good.read_bytes()[:-2])
    with pytest.raises(ValueError):
        page_file.read(trunc, [np.empty(4, np.uint8)], [np.empty(4, np.uint8)])


def test_checksums_ride_in_the_header_and_damage_is_rejected(tmp_path):
    meta = [{"name": "latent", "dtype": "BF16", "shape": [2, 2, 2]}]
    lo, hi = np.arange(8, dtype=np.uint8), np.arange(8, 16, dtype=np.uint8)
    good = tmp_path / "kv_l0_p0.vt"
    page_file.write(good, 0, 0, meta, [lo], [hi], [False], sums=[[-5, 123456789]])
    out_lo, out_hi = np.empty(8, np.uint8), np.empty(8, np.uint8)
    head = page_file.read(good, [out_lo], [out_hi])
    assert head["sums"] == [[-5, 123456789]]
    assert np.array_equal(out_lo, lo) and np.array_equal(out_hi, hi)
    with pytest.raises(ValueError):
        page_file.write(tmp_path / "x.vt", 0, 0, meta, [lo], [hi], [False], sums=[[1], [2]])
    longer = tmp_path / "kv_l0_p1.vt"
    longer.write_bytes(good.read_bytes() + b"\x00")
    with pytest.raises(ValueError, match="trailing"):
        page_file.read(longer, [out_lo], [out_hi])
    broken = tmp_path / "kv_l0_p2.vt"
    raw = bytearray(good.read_bytes())
    raw[10] = ord("#")  # inside the JSON header
    broken.write_bytes(bytes(raw))
    with pytest.raises(ValueError):
        page_file.read(broken, [out_lo], [out_hi])


def test_truncated_zstd_frame_is_rejected(tmp_path):
    if not vz.available():
        pytest.skip("libzstd not present")
    rng = np.random.default_rng(5)
    lo = rng.integers(0, 256, size=4096, dtype=np.uint8)
    hi = np.repeat(np.arange(16, dtype=np.uint8), 256)
    frame = vz.compress(hi, 1)
    meta = [{"name": "latent", "dtype": "BF16", "shape": [1, 4, 1024]}]
    path = tmp_path / "kv_l0_p0.vt"
    page_file.write(path, 0, 0, meta, [lo], [frame[:-3]], [True])
    with pytest.raises(ValueError):
        page_file.read(path, [np.empty(4096, np.uint8)], [np.empty(4096, np.uint8)])
