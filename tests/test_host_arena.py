"""Host arena allocator (CPU, unpinned): first fit, coalescing, reuse."""
from voom_amd.host_arena import HostArena


def test_alloc_free_coalesce_and_reuse():
    a = HostArena(slab_bytes=4096, pin=False)
    b1 = a.alloc(1000)
    b2 = a.alloc(1000)
    b3 = a.alloc(1000)
    assert a.capacity == 4096 and b1.view.numel() == 1000
    assert (b1.offset, b2.offset, b3.offset) == (0, 1024, 2048)
    a.free(b2)
    a.free(b1)
    b4 = a.alloc(2000)              # fits in the coalesced hole at 0
    assert b4.offset == 0 and b4.slab == 0
    b5 = a.alloc(5000)              # larger than a slab: a dedicated slab
    assert b5.slab == 1 and b5.view.numel() == 5000
    b4.view.fill_(7)
    b3.view.fill_(9)
    assert int(b4.view.sum()) == 7 * 2000 and int(b3.view[0]) == 9
    a.free(b3); a.free(b4); a.free(b5)
    assert a.used_bytes == 0


def test_reserve_grows_capacity():
    a = HostArena(slab_bytes=1 << 16, pin=False)
    a.reserve(300000)
    assert a.capacity >= 300000
    a.close()
    assert a.capacity == 0
