"""Pins the spilled-page checksum restatement (oracle/page_sums.py).

fmix32 must be a bijection (so any single changed word changes the sum) and
the word key must make positions matter (so moved words are caught); the
sum must be the plain mod-2^32 sum of per-word terms (so it can be reduced in
any order on the GPU).  A dropped key, a wrong shift or a non-bijective mix
fails one of these."""
import numpy as np

from oracle import page_sums as ops_


def test_fmix32_is_a_bijection_on_a_large_sample():
    rng = np.random.default_rng(0)
    x = np.unique(rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32))
    y = ops_.fmix32(x)
    assert np.unique(y).size == x.size
    assert int(ops_.fmix32(np.array([0], np.uint32))[0]) == 0  # zero is its fixed point


def test_fmix32_avalanches():
    # flipping one input bit flips about half the output bits
    rng = np.random.default_rng(1)
    x = rng.integers(0, 1 << 32, size=4096, dtype=np.uint64).astype(np.uint32)
    flips = []
    for bit in range(32):
        d = ops_.fmix32(x) ^ ops_.fmix32(x ^ np.uint32(1 << bit))
        flips.append(np.unpackbits(d.view(np.uint8)).mean() * 32)
    assert 14 < min(flips) and max(flips) < 18


def test_every_single_word_change_changes_the_sum():
    rng = np.random.default_rng(2)
    page = rng.integers(0, 1 << 16, size=4096, dtype=np.uint64).astype(np.uint16)
    base = ops_.slot_sum(page)
    for _ in range(2000):
        bad = page.copy()
        i = rng.integers(page.size)
        bad[i] ^= np.uint16(1 << int(rng.integers(16)))
        assert ops_.slot_sum(bad) != base


def test_moved_words_change_the_sum():
    rng = np.random.default_rng(3)
    w = rng.integers(0, 1 << 32, size=512, dtype=np.uint64).astype(np.uint32)
    base = ops_.slot_sum(w)
    for _ in range(500):
        i, j = rng.choice(w.size, size=2, replace=False)
        if w[i] == w[j]:
            continue
        sw = w.copy()
        sw[[i, j]] = sw[[j, i]]
        assert ops_.slot_sum(sw) != base


def test_sum_is_the_modular_sum_of_keyed_terms():
    rng = np.random.default_rng(4)
    w = rng.integers(0, 1 << 32, size=300, dtype=np.uint64).astype(np.uint32)
    total = 0
    for j, word in enumerate(w.tolist()):
        total += int(ops_.fmix32(np.array([(word + j * ops_.KEY) & 0xFFFFFFFF], np.uint32))[0])
    assert ops_.slot_sum(w) == total % (1 << 32)
    zeros = np.zeros(64, np.uint32)
    keyed = [int(ops_.fmix32(np.array([(j * ops_.KEY) & 0xFFFFFFFF], np.uint32))[0])
             for j in range(64)]
    assert ops_.slot_sum(zeros) == sum(keyed) % (1 << 32)
