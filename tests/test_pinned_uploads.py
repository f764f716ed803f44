"""The pinned index-list ring of PagedKVCache (_PinnedUploads) on the CPU, with
fake events: a region is rewritten only after every pending reader that
overlaps it has finished, wherever that reader sits in the queue."""
import numpy as np
import pytest
import torch

from voom_amd.kv_paged import _PinnedUploads


class FakeEvent:
    def __init__(self, name, log, done=False):
        self.name, self.log, self.done = name, log, done

    def query(self):
        return self.done

    def synchronize(self):
        self.log.append(self.name)
        self.done = True


def stage(ring, n, name, log):
    ring.stage(np.arange(n, dtype=np.int32))
    ring.settle(FakeEvent(name, log))


def test_a_region_pending_from_two_laps_back_does_not_hide_an_overlap():
    log = []
    ring = _PinnedUploads(torch.device("cpu"), pin=False, words=200)
    stage(ring, 90, "a", log)      # [0, 90)
    stage(ring, 90, "b", log)      # [90, 180)
    stage(ring, 20, "x", log)      # [180, 200): stays pending, overlaps nothing below
    stage(ring, 90, "y", log)      # wraps: [0, 90) waits for a only
    assert log == ["a"]
    stage(ring, 90, "z", log)      # [90, 180) waits for b only
    assert log == ["a", "b"]
    stage(ring, 30, "w", log)      # wraps again: [0, 30) overlaps y, queued behind pending x
    assert log == ["a", "b", "y"]


def test_finished_readers_are_dropped_and_unsettled_overlaps_raise():
    log = []
    ring = _PinnedUploads(torch.device("cpu"), pin=False, words=128)
    ring.stage(np.arange(40, dtype=np.int32))   # [0, 40), staged, never settled
    ring.stage(np.arange(40, dtype=np.int32))   # [40, 80)
    ring.stage(np.arange(40, dtype=np.int32))   # [80, 120)
    with pytest.raises(RuntimeError, match="never settled"):
        ring.stage(np.arange(40, dtype=np.int32))
    ring = _PinnedUploads(torch.device("cpu"), pin=False, words=128)
    ring.stage(np.arange(60, dtype=np.int32))   # [0, 60)
    ring.settle(FakeEvent("done", log, done=True))
    ring.stage(np.arange(60, dtype=np.int32))   # [60, 120)
    ring.settle(FakeEvent("p", log))
    ring.stage(np.arange(60, dtype=np.int32))   # wraps to [0, 60): only the finished reader
    assert log == [] and len(ring.inflight) == 2
