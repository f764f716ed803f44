"""The C-ABI library loads and exports every symbol include/voom_hip.h declares.

CPU-only: nothing here launches a kernel.  Validation failures are checked
with null/invalid arguments, which the library rejects on the host before any
HIP call.
"""
import ctypes
import re
from pathlib import Path

import pytest

from voom_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "voom_hip.h"
CALIB_HEADER = ROOT / "include" / "voom_calibrate.h"


def declared_symbols(header=HEADER):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(voom_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_symbols()
    for required in ("voom_paged_gqa_decode", "voom_byteplane_split", "voom_byteplane_merge",
                     "voom_byteplane_split_slots", "voom_byteplane_merge_slots",
                     "voom_append_kv", "voom_gather_kv", "voom_merge_attn_states",
                     "voom_paged_gqa_partials", "voom_paged_gqa_combine",
                     "voom_mla_absorbed_decode", "voom_append_rows", "voom_gather_rows"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_every_declared_symbol():
    assert set(declared_symbols()) <= set(_lib.SIGNATURES)


def test_calibration_probes_live_in_their_own_library():
    """The bench's probe kernels are declared in voom_calibrate.h, exported by
    libvoom_calibrate.so and bound by voom_amd.calibrate -- not by the
    paged-KV library or its header."""
    from voom_amd import calibrate
    from voom_amd._build import CALIB_LIB_PATH

    probes = declared_symbols(CALIB_HEADER)
    assert set(probes) == {"voom_stream_read", "voom_gather_read", "voom_tile_read"}
    assert not set(probes) & set(declared_symbols())
    _lib.lib()  # the probe library links against the paged-KV library
    cal = ctypes.CDLL(str(CALIB_LIB_PATH))
    assert all(hasattr(cal, n) for n in probes)
    product = ctypes.CDLL(str(_lib.LIB_PATH))
    assert not any(hasattr(product, n) for n in probes)
    assert set(probes) == set(calibrate.SIGNATURES)


def test_abi_version_and_workspace_query():
    lib = _lib.lib()
    assert lib.voom_abi_version() == 6
    assert lib.voom_paged_gqa_workspace_bytes(16, 32, 8, 128, 2048) > 0
    assert lib.voom_paged_gqa_workspace_bytes(0, 32, 8, 128, 2048) == 0


def test_validation_errors_raise_value_error():
    lib = _lib.lib()
    rc = lib.voom_paged_gqa_decode(None, None, None, None, None, None, None, None, 0,
                                   1, 4, 2, 128, 64, 1, 1, 1.0, 1, None)
    assert rc == _lib.VOOM_EINVAL
    assert "null pointer" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(rc, "paged_gqa_decode")
    fake = ctypes.c_void_p(256)
    rc = lib.voom_paged_gqa_decode(fake, fake, fake, fake, fake, fake, None, fake, 1 << 30,
                                   1, 4, 2, 96, 64, 1, 1, 1.0, 1, None)
    assert rc == _lib.VOOM_EINVAL and "head_dim" in _lib.last_error()
    rc = lib.voom_paged_gqa_decode(fake, fake, fake, fake, fake, fake, None, fake, 1 << 30,
                                   1, 48, 2, 128, 64, 1, 1, 1.0, 1, None)
    assert rc == _lib.VOOM_EINVAL and "GQA group" in _lib.last_error()
    rc = lib.voom_paged_gqa_decode(fake, fake, fake, fake, fake, fake, None, fake, 1 << 30,
                                   1, 4, 2, 128, 48, 1, 1, 1.0, 1, None)
    assert rc == _lib.VOOM_EINVAL and "page_tokens" in _lib.last_error()
    rc = lib.voom_paged_gqa_decode(fake, fake, fake, fake, fake, fake, None, fake, 16,
                                   1, 4, 2, 128, 64, 1, 1, 1.0, 64, None)
    assert rc == _lib.VOOM_EINVAL and "workspace" in _lib.last_error()
    rc = lib.voom_paged_gqa_partials(fake, fake, fake, fake, None, fake, 1 << 30,
                                     1, 4, 2, 128, 64, 1, 1, 1.0, 1, None)
    assert rc == _lib.VOOM_EINVAL and "null pointer" in _lib.last_error()
    rc = lib.voom_paged_gqa_combine(fake, fake, None, fake, 16, 1, 4, 2, 128, 64, 1, 64, None)
    assert rc == _lib.VOOM_EINVAL and "workspace" in _lib.last_error()
    rc = lib.voom_byteplane_split_slots(fake, fake, 1, 100, 1, fake, fake, None, None)
    assert rc == _lib.VOOM_EINVAL and "multiple of 64" in _lib.last_error()
    rc = lib.voom_page_sums_verify(fake, fake, 4, 0, fake, None)
    assert rc == _lib.VOOM_EINVAL and "tag" in _lib.last_error()
    rc = lib.voom_copy_rows(None, 64, fake, 64, 64, 3, None)
    assert rc == _lib.VOOM_EINVAL and "null pointer" in _lib.last_error()
    rc = lib.voom_copy_rows(fake, 64, fake, 32, 64, 3, None)  # rows would overlap
    assert rc == _lib.VOOM_EINVAL and "exceeds a pitch" in _lib.last_error()
    assert lib.voom_copy_rows(None, 0, None, 0, 0, 5, None) == 0  # nothing to copy
    assert lib.voom_copy_rows(None, 0, None, 0, 64, 0, None) == 0


def test_runtime_error_mapping():
    with pytest.raises(RuntimeError):
        _lib.check(2, "x")
