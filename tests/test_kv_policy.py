"""PagedKVCache budget policy on the CPU: the product planner against the
oracle restatement of runtime/kv_paged.py, plus hand-computed orders."""
import numpy as np
import pytest

from oracle.kv_policy import PagedKVPolicy
from voom_amd.kv_paged import budget_victims


class Meta:
    def __init__(self, nbytes):
        self.resident = True
        self.nbytes = nbytes


def drive_product(num_layers, max_bytes, PT, resident_pages, token_bytes, steps):
    """Bookkeeping with the product's planner (no device needed)."""
    pages = [[] for _ in range(num_layers)]
    lens = [0] * num_layers
    log = []
    for layer, n in steps:
        lens[layer] += n
        while (len(pages[layer]) + 1) * PT <= lens[layer]:
            pages[layer].append(Meta(PT * token_bytes))
        if layer == num_layers - 1:
            cur = sum(sum(p.nbytes for p in ps if p.resident) + (l - len(ps) * PT) * token_bytes
                      for ps, l in zip(pages, lens))
            for l, i in budget_victims(pages, resident_pages, cur, max_bytes):
                pages[l][i].resident = False
                log.append((l, i))
    return log


def drive_oracle(num_layers, max_bytes, PT, resident_pages, token_bytes, steps):
    pol = PagedKVPolicy(num_layers, max_bytes, PT, resident_pages, token_bytes)
    for layer, n in steps:
        pol.update(layer, n)
    return pol.spill_log


def test_reference_unit_test_geometry():
    # tests/test_kv_spill_compress.py:22-60: 2 layers, max_bytes=1, page 4,
    # resident_pages=0; 4 tokens per layer, then 1 more -> both layers' page 0 spill.
    token_bytes = 1 * 2 * 8 * 2 * 2   # B=1, NKV=2, D=8, bf16, K+V
    steps = [(0, 4), (1, 4), (0, 1), (1, 1)]
    log = drive_oracle(2, 1, 4, 0, token_bytes, steps)
    assert log == [(0, 0), (1, 0)]
    assert drive_product(2, 1, 4, 0, token_bytes, steps) == log


def test_hand_computed_round_robin_keeps_newest_page():
    # 3 layers, page 2 tokens, 1 byte per token; budget 9 bytes; resident_pages=1.
    # After 8 decode steps every layer has 4 closed pages (24 B > 9).
    steps = [(l, 1) for _ in range(8) for l in range(3)]
    log = drive_oracle(3, 9, 2, 1, 1, steps)
    # Budget is checked after each step's last layer.  Step 4: 12 B > 9 with two
    # closed pages per layer; page 0 of layers 0 and 1 spill (12 -> 10 -> 8).
    # Step 5: 8 + 3 = 11 B > 9, page 0 of layer 2 spills (-> 9).
    assert log[:3] == [(0, 0), (1, 0), (2, 0)]
    assert all(i < 3 for _, i in log)          # page 3 (the newest) never spills
    assert drive_product(3, 9, 2, 1, 1, steps) == log


@pytest.mark.parametrize("seed", range(20))
def test_random_schedules_agree(seed):
    rng = np.random.default_rng(seed)
    L = int(rng.integers(1, 5))
    PT = int(rng.choice([1, 2, 4, 8]))
    rp = int(rng.integers(0, 3))
    tb = int(rng.integers(1, 5))
    max_bytes = int(rng.integers(0, 200))
    steps = []
    for _ in range(int(rng.integers(1, 30))):
        n = int(rng.integers(1, 6))
        steps += [(l, n) for l in range(L)]
    assert drive_product(L, max_bytes, PT, rp, tb, steps) == \
        drive_oracle(L, max_bytes, PT, rp, tb, steps)


def test_within_budget_spills_nothing():
    assert budget_victims([[Meta(10)]], 0, 10, 10) == []


def test_vectorised_victims_match_the_reference_order():
    """budget_victims_fast (the cache's path for pages of one size) picks the
    same pages in the same order as the reference-order loop."""
    import numpy as np

    from voom_amd.kv_paged import budget_victims_fast

    class Page:
        def __init__(self, resident):
            self.resident = resident
            self.nbytes = 100

    rng = np.random.default_rng(0)
    for trial in range(300):
        L = int(rng.integers(1, 6))
        lengths = rng.integers(0, 12, size=L)
        cap = int(lengths.max()) + int(rng.integers(0, 3))
        resident = rng.random((L, max(cap, 1))) < 0.7
        keep = int(rng.integers(0, 3))
        pages = [[Page(bool(resident[l, i])) for i in range(lengths[l])] for l in range(L)]
        current = int(rng.integers(0, 4000))
        max_bytes = int(rng.integers(0, 4000))
        want = budget_victims(pages, keep, current, max_bytes)
        layers, idx = budget_victims_fast(resident, lengths, keep, 100, current, max_bytes)
        assert list(zip(layers.tolist(), idx.tolist())) == want, trial
