"""Paged KV pool growth and the page allocator (host logic, CPU tensors).

Growth follows the reference's dense cache (paged_kv_store.py:304-330,
543-579): max(16, 2 x capacity, required) pages, or exactly max_pages when
capped, the old pages copied in place; page ids never change.
"""

import pytest
import torch

from pagelora_amd.kv_pool import PageAllocator, PagedKVPool, Request


def _pool(cap, max_pages=0):
    return PagedKVPool(num_layers=2, capacity_pages=cap, page_size=4, num_kv_heads=1, head_dim=8,
                       dtype=torch.float32, device="cpu", max_pages=max_pages)


def test_growth_doubles_and_keeps_pages():
    pool = _pool(4)
    r = Request()
    pool.reserve(r, 12)  # pages 1..3 fill the initial pool
    assert r.own_pages == [1, 2, 3] and pool.grow_count == 0
    pool.cache.copy_(torch.arange(pool.cache.numel(), dtype=torch.float32).reshape(pool.cache.shape))
    before = pool.cache.clone()
    ptr = pool.cache.data_ptr()
    pool.reserve(r, 5)  # two more pages: the pool grows to max(16, 8, 6) = 16
    assert pool.grow_count == 1 and pool.version == 1
    assert pool.capacity_pages == 16 and pool.cache.data_ptr() != ptr
    assert r.own_pages == [1, 2, 3, 4, 5]
    assert torch.equal(pool.cache[:, :4], before)
    assert pool.allocator.free_pages == 16 - 6


def test_growth_to_the_required_size():
    pool = _pool(16)
    r = Request()
    pool.reserve(r, 4 * 70)  # 70 pages > 2 x 16
    assert pool.capacity_pages == 71 and r.own_pages == list(range(1, 71))


def test_capped_growth_goes_straight_to_max_pages_then_fails():
    pool = _pool(4, max_pages=10)
    r = Request()
    pool.reserve(r, 4 * 4)
    assert pool.capacity_pages == 10 and r.own_pages == [1, 2, 3, 4]
    pool.reserve(r, 4 * 5)
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        pool.reserve(r, 4)
    # a failed allocation takes nothing
    assert r.own_pages == list(range(1, 10)) and pool.allocator.free_pages == 0


def test_fixed_pool_raises_when_exhausted():
    pool = _pool(4, max_pages=None)
    r = Request()
    pool.reserve(r, 12)
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.reserve(r, 1)
    assert pool.grow_count == 0


def test_max_pages_below_capacity_is_rejected():
    with pytest.raises(ValueError):
        _pool(8, max_pages=4)


def test_allocator_hands_out_freed_pages_before_new_ones():
    grown = []

    def grow(required):
        grown.append(required)
        return 8

    a = PageAllocator(4, grow=grow)
    first = a.allocate(3)
    a.free([2])
    assert a.allocate(2) == [2, 4] and grown == [5] and a.capacity == 8
