"""Allocator mirror against the reference's own allocator tests
(tests/test_kv_cache_manager.py:5-119 of the reference, same cases and
expected values)."""
import pytest

from auto_infer_amd.kv_cache_manager import KVCacheManager


def test_blocks_needed():
    m = KVCacheManager(num_blocks=10, block_size=4)
    assert [m.blocks_needed(n) for n in (0, 1, 4, 5)] == [0, 1, 1, 2]


def test_allocate_and_free():
    m = KVCacheManager(10, 4)
    blocks = m.allocate(6)
    assert len(blocks) == 2 and m.num_free_blocks() == 8
    m.free(blocks)
    assert m.num_free_blocks() == 10


def test_lifo_block_order():
    """The free list pops from its tail: the first allocation gets N-1, N-2."""
    m = KVCacheManager(10, 4)
    assert m.allocate(8) == [9, 8]
    a = m.allocate(4)
    m.free(a)
    assert m.allocate(4) == a


def test_append_slots_only_when_last_block_full():
    m = KVCacheManager(10, 4)
    blocks = m.allocate(4)
    assert m.num_free_blocks() == 9
    assert len(m.append_slots(blocks, cur_num_tokens=4, num_new_tokens=1)) == 1
    assert m.num_free_blocks() == 8
    assert m.append_slots(blocks, cur_num_tokens=5, num_new_tokens=2) == []


def test_allocate_oom():
    m = KVCacheManager(1, 4)
    with pytest.raises(MemoryError):
        m.allocate(100)


def test_can_allocate():
    m = KVCacheManager(2, 4)
    assert m.can_allocate(8) is True and m.can_allocate(9) is False


def test_prefix_caching_share_and_release():
    m = KVCacheManager(10, 4)
    toks = [1, 2, 3, 4, 5, 6, 7, 8]
    blk = m.allocate(8)
    m.register_prefix(toks, blk)
    free_after_first = m.num_free_blocks()
    shared = m.match_prefix(toks)
    assert shared == blk and m.num_free_blocks() == free_after_first
    m.free(shared)
    assert m.num_free_blocks() == free_after_first
    m.free(blk)
    assert m.num_free_blocks() == 10
    assert m.match_prefix(toks) == blk


def test_prefix_partial_match():
    m = KVCacheManager(10, 4)
    blk = m.allocate(8)
    m.register_prefix([1, 2, 3, 4, 5, 6, 7, 8], blk)
    assert m.match_prefix([1, 2, 3, 4, 9, 9, 9, 9]) == [blk[0]]


def test_free_retains_registered_block_for_reuse():
    m = KVCacheManager(10, 4)
    toks = [1, 2, 3, 4, 5, 6, 7, 8]
    blk = m.allocate(8)
    m.register_prefix(toks, blk)
    m.free(blk)
    assert m.num_free_blocks() == 10
    assert m.match_prefix(toks) == blk
    assert m.num_free_blocks() == 8


def test_lru_eviction_unregisters_oldest():
    m = KVCacheManager(2, 4)
    a = m.allocate(4)
    m.register_prefix([1, 2, 3, 4], a)
    m.free(a)
    assert len(m.allocate(8)) == 2 and m.num_free_blocks() == 0
    assert m.match_prefix([1, 2, 3, 4]) == []


def test_lru_eviction_order_two_blocks():
    m = KVCacheManager(3, 4)
    a = m.allocate(4)
    m.register_prefix([1, 2, 3, 4], a)
    m.free(a)
    b = m.allocate(4)
    m.register_prefix([5, 6, 7, 8], b)
    m.free(b)
    assert m.num_free_blocks() == 3
    assert len(m.allocate(8)) == 2
    assert m.match_prefix([1, 2, 3, 4]) == []
    assert m.match_prefix([5, 6, 7, 8]) == b
