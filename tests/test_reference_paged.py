"""The reference's page allocator and block table test cases (reference tests/test_paged.py), one
for one, on this package's host-side PageAllocator / BlockTable (CPU: pure bookkeeping)."""

from __future__ import annotations

import random

import pytest

from plastic_infer.kv.paged import DEFAULT_CHUNK_PAGES, DEFAULT_PAGE_SIZE, BlockTable, PageAllocator


def test_defaults():
    assert DEFAULT_PAGE_SIZE == 16 and DEFAULT_CHUNK_PAGES == 16


# ---- TestPageAllocator (reference :19-107) ------------------------------------------------------

def test_initial_state():
    a = PageAllocator(100)
    assert (a.total_pages, a.free_pages, a.used_pages) == (100, 100, 0)


def test_alloc_and_free():
    a = PageAllocator(10)
    p = a.alloc()
    assert 0 <= p < 10 and a.is_used(p)
    assert (a.free_pages, a.used_pages) == (9, 1)
    a.free(p)
    assert a.free_pages == 10 and not a.is_used(p)


def test_alloc_unique():
    a = PageAllocator(50)
    assert len({a.alloc() for _ in range(50)}) == 50
    assert a.free_pages == 0


def test_alloc_full_raises():
    a = PageAllocator(3)
    for _ in range(3):
        a.alloc()
    with pytest.raises(IndexError):
        a.alloc()


def test_alloc_many():
    a = PageAllocator(20)
    ids = a.alloc_many(5)
    assert len(ids) == len(set(ids)) == 5 and a.free_pages == 15


def test_alloc_many_overflow():
    with pytest.raises(IndexError):
        PageAllocator(5).alloc_many(10)


def test_free_reuse_is_lifo():
    a = PageAllocator(10)
    p1, p2 = a.alloc(), a.alloc()
    a.free(p2)
    a.free(p1)
    assert a.alloc() == p1   # freed last, handed out first
    assert a.alloc() == p2


def test_free_many():
    a = PageAllocator(20)
    ids = a.alloc_many(10)
    a.free_many(ids[:5])
    assert a.free_pages == 15
    for pid in ids[5:]:
        a.free(pid)
    assert a.free_pages == 20


def test_free_unused_raises():
    with pytest.raises(AssertionError):
        PageAllocator(10).free(42)


def test_no_leak_through_random_allocation():
    rng = random.Random(12345)
    a = PageAllocator(100)
    held: list[int] = []
    for _ in range(1000):
        if held and rng.random() < 0.5:
            a.free(held.pop(rng.randrange(len(held))))
        elif a.free_pages > 0:
            held.append(a.alloc())
    for pid in held:
        a.free(pid)
    assert (a.free_pages, a.used_pages) == (100, 0)


# ---- TestBlockTable (reference :114-189) --------------------------------------------------------

def test_empty_table():
    bt = BlockTable(n_layers=4, page_size=16)
    assert all(bt.num_logical_pages(l) == 0 and bt.num_tokens(l) == 0 for l in range(4))


def test_append_and_get():
    bt = BlockTable(n_layers=2, page_size=16)
    bt.append_page(0, 10)
    bt.append_page(0, 20)
    bt.append_page(1, 30)
    assert (bt.num_logical_pages(0), bt.num_logical_pages(1), bt.num_tokens(0)) == (2, 1, 32)
    assert (bt.get_page(0, 0), bt.get_page(0, 1), bt.get_page(1, 0)) == (10, 20, 30)


def test_get_page_for_token():
    bt = BlockTable(n_layers=1, page_size=16)
    bt.append_page(0, 100)
    bt.append_page(0, 200)
    assert [bt.get_page_for_token(0, t) for t in (0, 15, 16, 31)] == [100, 100, 200, 200]


def test_all_page_ids():
    bt = BlockTable(n_layers=3, page_size=16)
    for layer, pid in ((0, 1), (0, 2), (1, 3), (2, 2)):
        bt.append_page(layer, pid)
    assert bt.all_page_ids() == {1, 2, 3}


def test_chunk_page_ids():
    bt = BlockTable(n_layers=2, page_size=16)
    for l in range(2):
        for i in range(32):
            bt.append_page(l, l * 100 + i)
    c0, c1 = bt.chunk_page_ids(0, pages_per_chunk=16), bt.chunk_page_ids(1, pages_per_chunk=16)
    assert len(c0) == 32 and {0, 100, 15, 115} <= set(c0)
    assert len(c1) == 32 and {16, 116} <= set(c1)


def test_is_chunk_complete():
    bt = BlockTable(n_layers=2, page_size=16)
    for l in range(2):
        for i in range(20):
            bt.append_page(l, l * 100 + i)
    assert bt.is_chunk_complete(0, pages_per_chunk=16)
    assert not bt.is_chunk_complete(1, pages_per_chunk=16)
    assert not bt.is_chunk_complete(2, pages_per_chunk=16)


def test_chunk_partial():
    bt = BlockTable(n_layers=2, page_size=16)
    for l in range(2):
        for i in range(10):
            bt.append_page(l, l * 10 + i)
    assert len(bt.chunk_page_ids(0, pages_per_chunk=16)) == 20


# ---- TestAllocatorBlockTableIntegration (reference :196-260) ------------------------------------

def test_append_allocates():
    alloc, bt = PageAllocator(100), BlockTable(n_layers=4, page_size=16)
    for tok in range(100):
        for l in range(4):
            if bt.num_logical_pages(l) <= tok // 16:
                bt.append_page(l, alloc.alloc())
    assert bt.num_logical_pages(0) == 7
    assert (alloc.used_pages, alloc.free_pages) == (28, 72)


def test_evict_chunk_frees_pages():
    alloc, bt = PageAllocator(100), BlockTable(n_layers=2, page_size=16)
    for l in range(2):
        for _ in range(48):
            bt.append_page(l, alloc.alloc())
    assert alloc.used_pages == 96
    chunk0 = bt.chunk_page_ids(0, pages_per_chunk=16)
    assert len(chunk0) == 32
    alloc.free_many(chunk0)
    assert alloc.free_pages == 36


def test_cross_request_reuse():
    alloc = PageAllocator(50)
    bt1 = BlockTable(n_layers=2, page_size=16)
    for l in range(2):
        for _ in range(15):
            bt1.append_page(l, alloc.alloc())
    assert alloc.used_pages == 30
    alloc.free_many(list(bt1.all_page_ids()))
    assert (alloc.free_pages, alloc.used_pages) == (50, 0)
    bt2 = BlockTable(n_layers=4, page_size=16)
    for l in range(4):
        for _ in range(10):
            bt2.append_page(l, alloc.alloc())
    assert alloc.used_pages == 40
