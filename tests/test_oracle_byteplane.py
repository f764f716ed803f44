"""Pins the byte-plane oracle: exhaustive closed form over every 16-bit pattern."""
import numpy as np

from oracle import byteplane as ob


def all_patterns():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_split_matches_closed_form_for_every_pattern():
    e = all_patterns()
    lo, hi = ob.split(e)
    assert np.array_equal(lo, (e & 0xFF).astype(np.uint8))
    assert np.array_equal(hi, (e >> 8).astype(np.uint8))


def test_merge_inverts_split_bit_exactly():
    e = all_patterns()
    rng = np.random.default_rng(0)
    e = e[rng.permutation(e.size)]
    lo, hi = ob.split(e)
    assert np.array_equal(ob.merge(lo, hi), e)


def test_bf16_special_values_survive():
    # +-0, subnormals, +-inf and NaN payloads are just bytes to the codec.
    specials = np.array([0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC0, 0x7F81,
                         0xFFFF], dtype=np.uint16)
    lo, hi = ob.split(specials)
    assert np.array_equal(ob.merge(lo, hi), specials)


def test_c_restatement_agrees_with_numpy():
    lib = ob.load_c()
    assert lib is not None, "oracle C library not built (run __graft_entry__.build())"
    e = all_patterns()
    lo_c, hi_c = ob.split_c(lib, e)
    lo, hi = ob.split(e)
    assert np.array_equal(lo_c, lo) and np.array_equal(hi_c, hi)
    assert np.array_equal(ob.merge_c(lib, lo, hi), e)
    assert ob.split_c(lib, np.zeros(0, dtype=np.uint16))[0].size == 0
