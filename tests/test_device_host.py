"""The device block cache's bookkeeping (no device calls: blocks are handed in and out by address)."""
import threading

from seedpack_amd.device import _Cache


def test_cache_takes_least_block_up_to_twice_the_request():
    c = _Cache(limit=1 << 40)
    mine = c.mine()
    for n, p in ((8 << 20, 1), (12 << 20, 2), (40 << 20, 3), (12 << 20, 4)):
        assert c.give(mine, 0, p, n)
    assert c.take(0, 10 << 20) == (12 << 20, 4)          # the least class >= 10 MB, last freed first
    assert c.take(0, 10 << 20) == (12 << 20, 2)
    assert c.take(0, 10 << 20) is None                   # 40 MB is more than twice 10 MB
    assert c.take(1, 8 << 20) is None                    # another device
    assert c.take(0, 30 << 20) == (40 << 20, 3)
    assert c.take(0, 8 << 20) == (8 << 20, 1)
    assert c.bytes == 0 and c.take(0, 4096) is None


def test_cache_blocks_stay_with_their_thread_and_limit_holds():
    c = _Cache(limit=16 << 20)
    mine = c.mine()
    assert c.give(mine, 0, 7, 8 << 20) and c.give(mine, 0, 8, 8 << 20)
    assert not c.give(mine, 0, 9, 4096)                  # beyond the limit: the caller frees it
    other = []
    t = threading.Thread(target=lambda: other.append(c.take(0, 8 << 20)))
    t.start()
    t.join()
    assert other == [None]                               # another thread's blocks are not reused
    assert c.take(0, 8 << 20) in ((8 << 20, 7), (8 << 20, 8))
