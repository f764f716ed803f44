"""Host logic of the spill ready events (no GPU): a reload or upload that
needs many spill blocks waits on one event per recording stream -- the newest,
since the events of one stream complete in the order they were recorded --
and a host wait is skipped for events a later wait of their stream already
covered."""
from types import SimpleNamespace

from voom_amd.kv_paged import PagedKVCache


class FakeEvent:
    def __init__(self, name):
        self.name = name
        self.syncs = 0

    def synchronize(self):
        self.syncs += 1


class FakeStream:
    def __init__(self, handle):
        self.cuda_stream = handle
        self.waited = []

    def wait_event(self, ev):
        self.waited.append(ev.name)


def cache_stub():
    kv = object.__new__(PagedKVCache)
    kv._ready_seq = 0
    kv._ready_done = {}
    return kv


def spilled_block(kv, stream, name):
    sb = SimpleNamespace(rec_ready={}, ready=None, ready_at=None)
    kv._set_ready(sb, 0, FakeEvent(name), stream)
    return sb


def test_one_wait_per_recording_stream_on_its_newest_event():
    kv = cache_stub()
    main, side = FakeStream(11), FakeStream(22)
    blocks = [spilled_block(kv, main, f"m{i}") for i in range(5)]
    blocks += [spilled_block(kv, side, f"s{i}") for i in range(3)]
    blocks.append(spilled_block(kv, main, "m5"))
    blocks.append(SimpleNamespace(ready=None, ready_at=None))  # nothing recorded yet
    waiter = FakeStream(33)
    kv._wait_ready(waiter, reversed(blocks))  # any order, any iterable
    assert sorted(waiter.waited) == ["m5", "s2"]


def test_host_waits_skip_events_a_later_wait_covered():
    kv = cache_stub()
    main = FakeStream(11)
    old = [spilled_block(kv, main, f"m{i}") for i in range(4)]
    kv._sync_ready(old)
    assert [sb.ready.syncs for sb in old] == [0, 0, 0, 1]
    for sb in old:  # releasing them one by one waits for nothing more
        kv._sync_ready([sb])
    assert [sb.ready.syncs for sb in old] == [0, 0, 0, 1]
    new = spilled_block(kv, main, "m4")  # recorded after the wait: not covered
    kv._sync_ready([new])
    assert new.ready.syncs == 1
    side = spilled_block(kv, FakeStream(22), "s0")  # another stream: its own watermark
    kv._sync_ready([side])
    assert side.ready.syncs == 1
