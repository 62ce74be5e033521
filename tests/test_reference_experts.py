"""The reference's expert bank / slot pool test cases (reference tests/test_experts.py), one for
one. The bank is host-side (CPU tests); the slot pool keeps its resident experts in HBM and loads
them through the HIP row copies on a side stream (GPU tests). Same shapes, seeds, budgets and
expectations; data comparisons are exact."""

from __future__ import annotations

import pytest
import torch

from plastic_infer.store.experts import ExpertBank, ExpertSlotPool, ExpertWeights


def _expert(seed: int, H: int = 8, I: int = 16) -> ExpertWeights:
    """reference :15-21: w1, w3 [I, H], w2 [H, I], fp32, seeded."""
    g = torch.Generator().manual_seed(seed)
    return ExpertWeights(w1=torch.randn(I, H, generator=g), w2=torch.randn(H, I, generator=g),
                         w3=torch.randn(I, H, generator=g))


EXPERT_BYTES = _expert(0).bytes()  # 3 x 128 fp32 = 1536


@pytest.fixture
def bank() -> ExpertBank:
    b = ExpertBank()
    for l in range(2):
        for e in range(4):
            b.add(l, e, _expert(l * 100 + e))
    return b


def _pool(bank: ExpertBank, n_slots: int) -> ExpertSlotPool:
    return ExpertSlotPool(bank, budget_bytes=n_slots * EXPERT_BYTES)


# ---- TestExpertBank (reference :43-60), host ----------------------------------------------------

def test_add_get_roundtrip(bank):
    assert (0, 2) in bank and bank[(0, 2)].w1.shape == (16, 8) and len(bank) == 8


def test_bytes_accounting(bank):
    assert EXPERT_BYTES == 1536
    assert bank.bytes((0, 0)) == EXPERT_BYTES
    assert bank.total_bytes == len(bank) * EXPERT_BYTES


def test_duplicate_add_raises(bank):
    with pytest.raises(AssertionError):
        bank.add(0, 0, _expert(1))


def test_unknown_key_missing(bank):
    assert (9, 9) not in bank


# ---- TestSlotPoolBudget (reference :63-127), HBM pool -------------------------------------------

@pytest.mark.gpu
def test_budget_holds_subset(dev, bank):
    pool = _pool(bank, 2)
    pool.ensure(0, [0, 1])
    pool.release(0, [0, 1])
    assert pool.pool.used_bytes == 2 * EXPERT_BYTES and pool.pool.free_bytes == 0


@pytest.mark.gpu
def test_evicts_lru_when_over_budget(dev, bank):
    pool = _pool(bank, 2)
    for ids in ([0, 1], [2, 3]):
        pool.ensure(0, ids)
        pool.release(0, ids)
    assert (0, 0) not in pool.pool and (0, 1) not in pool.pool
    assert (0, 2) in pool.pool and (0, 3) in pool.pool
    assert pool.pool.used_bytes == 2 * EXPERT_BYTES


@pytest.mark.gpu
def test_lru_order_respected(dev, bank):
    pool = _pool(bank, 3)
    for ids in ([0, 1], [0], [2, 3]):   # re-touching 0 leaves 1 least recently used
        pool.ensure(0, ids)
        pool.release(0, ids)
    assert (0, 1) not in pool.pool
    assert all((0, e) in pool.pool for e in (0, 2, 3))


@pytest.mark.gpu
def test_d7_pinned_survives_eviction(dev, bank):
    pool = _pool(bank, 3)
    pool.ensure(0, [0, 1])
    pool.release(0, [0])     # expert 1 stays pinned
    pool.ensure(0, [2, 3])   # two slots needed, one free: only the unpinned 0 may go
    pool.release(0, [2, 3])
    assert (0, 1) in pool.pool and (0, 0) not in pool.pool
    assert (0, 2) in pool.pool and (0, 3) in pool.pool


@pytest.mark.gpu
def test_all_pinned_blocks_eviction(dev, bank):
    pool = _pool(bank, 2)
    pool.ensure(0, [0, 1])
    assert pool.pool.evict_to_fit(EXPERT_BYTES) == []
    assert (0, 0) in pool.pool and (0, 1) in pool.pool
    pool.release(0, [0, 1])


@pytest.mark.gpu
def test_budget_below_one_expert_rejected(dev, bank):
    with pytest.raises(AssertionError):
        ExpertSlotPool(bank, budget_bytes=EXPERT_BYTES - 1)


# ---- TestEnsure (reference :130-200), HBM pool --------------------------------------------------

@pytest.mark.gpu
def test_miss_loads_then_hit_reuses(dev, bank):
    pool = _pool(bank, 4)
    r1 = pool.ensure(0, [0, 1])
    pool.release(0, [0, 1])
    assert (pool.misses, pool.hits) == (2, 0)
    r2 = pool.ensure(0, [0, 1])
    pool.release(0, [0, 1])
    assert (pool.misses, pool.hits) == (2, 2)
    assert r2[0] is r1[0] and r2[1] is r1[1]   # the same resident tensors on a hit


@pytest.mark.gpu
def test_hit_rate(dev, bank):
    pool = _pool(bank, 4)
    for ids in ([0, 1], [0, 1], [2, 3]):
        pool.ensure(0, ids)
        pool.release(0, ids)
    assert (pool.misses, pool.hits) == (4, 2)
    assert pool.hit_rate == pytest.approx(2 / 6)


@pytest.mark.gpu
def test_data_matches_bank(dev, bank):
    pool = _pool(bank, 4)
    got = pool.ensure(0, [1, 3])
    pool.release(0, [1, 3])
    for e, w in got.items():
        ref = bank[(0, e)]
        assert w.w1.device.type == "cuda"
        assert torch.equal(w.w1.cpu(), ref.w1) and torch.equal(w.w2.cpu(), ref.w2)
        assert torch.equal(w.w3.cpu(), ref.w3)


@pytest.mark.gpu
def test_double_release_raises(dev, bank):
    pool = _pool(bank, 4)
    pool.ensure(0, [0])
    pool.release(0, [0])
    with pytest.raises(AssertionError):
        pool.release(0, [0])


@pytest.mark.gpu
def test_correct_with_single_slot(dev, bank):
    pool = _pool(bank, 1)
    for l in range(2):
        for e in range(4):
            got = pool.ensure(l, [e])
            pool.release(l, [e])
            assert torch.equal(got[e].w1.cpu(), bank[(l, e)].w1)
    assert pool.pool.used_bytes <= EXPERT_BYTES
