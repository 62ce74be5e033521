"""Host-side bookkeeping of the drop-in package (CPU, no GPU): page allocator, block tables,
chunk keys, the LRU residency pool, and the expert slot-pool policy oracle. Expectations follow
the reference's tests (reference tests/test_paged.py, tests/test_resident.py,
tests/test_experts.py, tests/test_chunk.py)."""

from __future__ import annotations

import hashlib
import random

import numpy as np
import pytest

import oracle.expert_copy as OC
from plastic_infer.kv.chunk import (
    compute_prefix_hashes,
    compute_prefix_hashes_and_final,
    longest_prefix_hits,
)
from plastic_infer.kv.paged import BlockTable, PageAllocator
from plastic_infer.store.resident import LruPool
from plastic_infer.store.tiers import Tier


class TestPageAllocator:
    def test_fresh_order_and_counts(self):
        a = PageAllocator(10)
        assert (a.total_pages, a.free_pages, a.used_pages) == (10, 10, 0)
        assert [a.alloc() for _ in range(3)] == [0, 1, 2]
        assert a.used_pages == 3 and a.is_used(1) and not a.is_used(5)

    def test_lifo_reuse(self):
        a = PageAllocator(10)
        p1, p2 = a.alloc(), a.alloc()
        a.free(p2)
        a.free(p1)
        assert a.alloc() == p1 and a.alloc() == p2

    def test_alloc_many_matches_repeated_alloc(self):
        a, b = PageAllocator(20), PageAllocator(20)
        b.free_many([])
        assert a.alloc_many(5) == [b.alloc() for _ in range(5)]

    def test_errors(self):
        a = PageAllocator(3)
        a.alloc_many(3)
        with pytest.raises(IndexError):
            a.alloc()
        with pytest.raises(IndexError):
            PageAllocator(5).alloc_many(10)
        with pytest.raises(AssertionError):
            PageAllocator(10).free(4)
        with pytest.raises(AssertionError):
            PageAllocator(0)

    def test_random_churn_no_leak(self):
        rng = random.Random(12345)
        a = PageAllocator(100)
        used: list[int] = []
        for _ in range(2000):
            if used and rng.random() < 0.5:
                a.free(used.pop(rng.randrange(len(used))))
            elif a.free_pages:
                used.append(a.alloc())
        assert len(set(used)) == len(used)
        a.free_many(used)
        assert a.free_pages == 100 and a.used_pages == 0


class TestBlockTable:
    def test_mapping(self):
        bt = BlockTable(n_layers=2, page_size=16)
        bt.append_page(0, 100)
        bt.append_page(0, 200)
        bt.append_page(1, 30)
        assert bt.num_logical_pages(0) == 2 and bt.num_tokens(0) == 32
        assert bt.get_page_for_token(0, 15) == 100 and bt.get_page_for_token(0, 16) == 200
        assert bt.all_page_ids() == {100, 200, 30}

    def test_chunks(self):
        bt = BlockTable(n_layers=2, page_size=16)
        for l in range(2):
            for i in range(20):
                bt.append_page(l, l * 100 + i)
        c0 = bt.chunk_page_ids(0, 16)
        assert len(c0) == 32 and c0[:2] == [0, 1] and c0[16] == 100
        assert len(bt.chunk_page_ids(1, 16)) == 8
        assert bt.is_chunk_complete(0, 16) and not bt.is_chunk_complete(1, 16)


class TestChunkKeys:
    def test_hash_chain_format(self):
        toks = list(range(8)) + [2**32 - 1] * 8
        keys, final = compute_prefix_hashes_and_final(toks, chunk_size=8)
        h = hashlib.sha256(b"plastic-infer-kv-v1").digest()
        for i in range(2):
            c = hashlib.sha256(b"".join(t.to_bytes(4, "little") for t in toks[8 * i:8 * i + 8]))
            nxt = hashlib.sha256(h + c.digest()).digest()
            assert keys[i].prefix_key == h and keys[i].cumulative_key == nxt
            h = nxt
        assert final == h

    def test_alignment_and_prefix_hits(self):
        with pytest.raises(ValueError):
            compute_prefix_hashes([1, 2, 3], chunk_size=2)
        keys = compute_prefix_hashes(list(range(12)), chunk_size=4)
        index = {keys[0].full_key: keys[0], keys[1].full_key: keys[1]}
        matched, tail = longest_prefix_hits(index, list(range(14)), chunk_size=4)
        assert matched == keys[:2] and tail == 8
        matched, tail = longest_prefix_hits(index, [9] + list(range(1, 12)), chunk_size=4)
        assert matched == [] and tail == 0


@pytest.fixture
def pool() -> LruPool:
    p: LruPool = LruPool(1000)
    for i in range(5):
        p.add(f"p{i}", 100, Tier.GPU)
    return p


class TestLruPool:
    def test_accounting_and_pins(self, pool):
        assert pool.used_bytes == 500 and pool.can_fit(500) and not pool.can_fit(501)
        pool.pin("p0")
        with pytest.raises(AssertionError):
            pool.remove("p0")
        pool.unpin("p0")
        with pytest.raises(AssertionError):
            pool.unpin("p0")

    def test_lru_order_and_pins(self, pool):
        pool.pin("p0")
        pool.unpin("p0")                      # p0 becomes newest
        assert [p.key for p in pool.evict_lru(100)] == ["p1"]
        pool.pin("p2")
        assert "p2" not in {p.key for p in pool.evict_lru(300)}

    def test_evict_to_fit_and_tiers(self, pool):
        assert pool.evict_to_fit(100) == []
        assert len(pool.evict_to_fit(800)) == 3 and pool.free_bytes >= 800
        p2: LruPool = LruPool(1000)
        for i in range(5):
            p2.add(f"p{i}", 100)
        p2.set_tier("p0", Tier.HOST)
        p2.set_tier("p1", Tier.DISK)
        assert p2.used_bytes == 300
        assert {p.key for p in p2.evict_lru(500)} == {"p2", "p3", "p4"}
        p2.set_tier("p0", Tier.GPU)
        assert p2.used_bytes == 100 and len(p2) == 2


class _ListModel:
    """Executable statement of the LruPool contract on a plain recency list (oldest first):
    the model the tracker must agree with on every observable after every operation."""

    def __init__(self, budget):
        self.budget, self.order, self.pages = budget, [], {}

    def _use(self, k):
        if k in self.order:
            self.order.remove(k)
        self.order.append(k)

    def used(self):
        return sum(b for b, t, _ in self.pages.values() if t == Tier.GPU)

    def add(self, k, b, t):
        self.pages[k] = [b, t, 0]
        self._use(k)

    def pin(self, k):
        self.pages[k][2] += 1
        self._use(k)

    def unpin(self, k):
        self.pages[k][2] -= 1
        self._use(k)

    def set_tier(self, k, t):
        self.pages[k][1] = t
        self._use(k)

    def remove(self, k):
        del self.pages[k]
        self.order.remove(k)

    def evict(self, need):
        out, freed = [], 0
        for k in list(self.order):
            if freed >= need:
                break
            b, t, pins = self.pages[k]
            if pins or t != Tier.GPU:
                continue
            self.remove(k)
            out.append(k)
            freed += b
        return out


@pytest.mark.parametrize("seed", range(8))
def test_lru_pool_matches_recency_list_model(seed):
    """3000 random operations (adds, pins, unpins, tier moves, removes, evictions with zero,
    small and huge requests) on the tracker and on the list model: same evicted keys in the
    same order, same byte accounting, same recency order, same errors."""
    import random

    rng = random.Random(seed)
    pool: LruPool = LruPool(5000)
    model = _ListModel(5000)
    tiers = [Tier.GPU, Tier.GPU, Tier.GPU, Tier.HOST, Tier.DISK]
    next_key = 0
    for _ in range(3000):
        keys = list(model.pages)
        op = rng.randrange(7)
        if op == 0 or not keys:
            k, b, t = next_key, rng.randrange(0, 400), rng.choice(tiers)
            next_key += 1
            pool.add(k, b, t)
            model.add(k, b, t)
        elif op == 1:
            k = rng.choice(keys)
            pool.pin(k)
            model.pin(k)
        elif op == 2:
            k = rng.choice(keys)
            if model.pages[k][2] == 0:
                with pytest.raises(AssertionError):
                    pool.unpin(k)
            else:
                pool.unpin(k)
                model.unpin(k)
        elif op == 3:
            k, t = rng.choice(keys), rng.choice(tiers)
            pool.set_tier(k, t)
            model.set_tier(k, t)
        elif op == 4:
            k = rng.choice(keys)
            if model.pages[k][2]:
                with pytest.raises(AssertionError):
                    pool.remove(k)
            else:
                assert pool.remove(k).key == k
                model.remove(k)
        elif op == 5:
            need = rng.choice([0, 1, rng.randrange(0, 1500), 10 ** 9])
            assert [p.key for p in pool.evict_lru(need)] == model.evict(need)
        else:
            want = rng.randrange(0, 6000)
            fits = model.used() + want <= model.budget
            got = [p.key for p in pool.evict_to_fit(want)]
            assert got == ([] if fits else model.evict(want - (model.budget - model.used())))
        assert pool.used_bytes == model.used() and len(pool) == len(model.pages)
        assert pool.lru_keys() == model.order
        assert pool.all_pinned() == (not any(p == 0 and t == Tier.GPU
                                             for _, t, p in model.pages.values()))
    with pytest.raises(AssertionError):
        pool.add(next(iter(model.pages)), 1) if model.pages else pool.add(-1, 1) or pool.add(-1, 1)


class TestSlotPoolPolicyOracle:
    """The oracle's residency decisions on the reference's ExpertSlotPool scenarios
    (reference tests/test_experts.py:71-131)."""

    def _policy(self, slots):
        return OC.SlotPoolPolicy({(l, e): 1 for l in range(2) for e in range(4)}, slots)

    def test_lru_order(self):
        p = self._policy(3)
        p.ensure(0, [0, 1]); p.release(0, [0, 1])
        p.ensure(0, [0]); p.release(0, [0])
        p.ensure(0, [2, 3]); p.release(0, [2, 3])
        assert p.resident() == {(0, 0), (0, 2), (0, 3)}

    def test_pinned_survives(self):
        p = self._policy(3)
        p.ensure(0, [0, 1]); p.release(0, [0])
        p.ensure(0, [2, 3]); p.release(0, [2, 3])
        assert p.resident() == {(0, 1), (0, 2), (0, 3)}

    def test_hit_miss_counts(self):
        p = self._policy(4)
        for ids in ([0, 1], [0, 1], [2, 3]):
            p.ensure(0, ids); p.release(0, ids)
        assert (p.hits, p.misses) == (2, 4)


@pytest.mark.parametrize("seed,n_slots,universe,calls", [(0, 16, 64, 200), (1, 64, 6144, 100),
                                                          (2, 5, 12, 300)])
def test_staging_lru_follows_the_admission_rule(seed, n_slots, universe, calls):
    """The host staging LRU of the "static" expert policy makes the decisions of the device
    admission kernel, as the slot-cache oracle restates it: same slot for every id, same ids
    copied into the same slots, call after call."""
    import oracle.slot_cache as SC
    from plastic_infer.moe.offload_cache import _StagingLru

    rng = np.random.default_rng(seed)
    lru = _StagingLru(n_slots)
    st = SC.new_state(universe, n_slots)
    for _ in range(calls):
        n = int(rng.integers(1, n_slots + 1))
        ids = rng.choice(universe, size=n, replace=False).astype(np.int64)
        slots, new_ids, victims = lru.place(ids)
        out, src, dst, num, _ = SC.lru_ensure(st, ids)
        assert np.array_equal(slots, out.astype(np.int64))
        assert np.array_equal(new_ids, src.astype(np.int64))
        assert np.array_equal(victims, dst.astype(np.int64))
    lru.forget_range(0, n_slots)
    assert (lru.owner == -1).all() and not lru.slot_of
