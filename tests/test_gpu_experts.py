"""GPU parity of the expert-weight movement: row index-copy kernels, host-planned DMA row
copies, and the HBM expert slot pool (reference tests/test_experts.py scenarios) — bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.expert_copy as OC
from plastic_infer.kernel import copy_rows_async, fast_index_copy, fast_index_copy_multi
from plastic_infer.kernel.index_copy import device_ptr
from plastic_infer.store.experts import ExpertBank, ExpertSlotPool, ExpertWeights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("src_on_host", [False, True])
def test_fast_index_copy(dev, idx_dtype, src_on_host):
    g = torch.Generator().manual_seed(1)
    src = torch.randn(12, 3, 256, generator=g).to(torch.bfloat16)
    dst = torch.randn(8, 3, 256, generator=g).to(torch.bfloat16)
    di = [5, 0, -1, 7, 2]
    si = [11, 3, 4, 0, 9]
    ref_np = dst.clone().view(torch.int16).numpy()
    OC.index_copy_rows(ref_np, di, src.view(torch.int16).numpy(), si, n=4)
    gsrc = src.pin_memory() if src_on_host else src.to(dev)
    gdst = dst.to(dev)
    fast_index_copy(gdst, torch.tensor(di, dtype=idx_dtype, device=dev), gsrc,
                    torch.tensor(si, dtype=idx_dtype, device=dev),
                    num_indices=torch.tensor([4], dtype=torch.int64, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(gdst.cpu().view(torch.int16), torch.from_numpy(ref_np))


def test_fast_index_copy_odd_row_bytes(dev):
    src = torch.arange(7 * 5, dtype=torch.uint8).view(7, 5)
    dst = torch.zeros(4, 5, dtype=torch.uint8)
    ref = dst.clone().numpy()
    OC.index_copy_rows(ref, [3, 1], src.numpy(), [6, 2])
    gdst = dst.to(dev)
    fast_index_copy(gdst, torch.tensor([3, 1], device=dev), src.to(dev), torch.tensor([6, 2], device=dev))
    assert np.array_equal(gdst.cpu().numpy(), ref)


def test_fast_index_copy_multi(dev):
    g = torch.Generator().manual_seed(2)
    banks_src = [torch.randn(6, 64, generator=g), torch.randn(6, 16, generator=g)]
    banks_dst = [torch.zeros(4, 64, device=dev), torch.zeros(4, 16, device=dev)]
    srcs = [b.pin_memory() for b in banks_src]
    dst_ptrs = torch.tensor([device_ptr(d) for d in banks_dst], dtype=torch.int64, device=dev)
    src_ptrs = torch.tensor([device_ptr(s) for s in srcs], dtype=torch.int64, device=dev)
    feat = torch.tensor([64 * 4, 16 * 4], dtype=torch.int64, device=dev)
    fast_index_copy_multi(dst_ptrs, src_ptrs, feat, torch.tensor([2, 0, 3], device=dev),
                          torch.tensor([5, 1, 4], device=dev))
    torch.cuda.synchronize()
    for s, d in zip(banks_src, banks_dst):
        ref = torch.zeros(4, s.shape[1])
        ref[[2, 0, 3]] = s[[5, 1, 4]]
        assert torch.equal(d.cpu(), ref)


def test_copy_rows_async_merges_runs(dev):
    g = torch.Generator().manual_seed(3)
    src = torch.randn(10, 1000, generator=g).pin_memory()
    dst = torch.zeros(10, 1000, device=dev)
    stream = torch.cuda.Stream(device=dev)
    n = copy_rows_async(dst, [0, 1, 2, 7, 5, 6], src, [3, 4, 5, 0, 8, 9], stream=stream)
    assert n == 3          # runs (0-2 <- 3-5), (7 <- 0), (5-6 <- 8-9)
    stream.synchronize()
    ref = torch.zeros(10, 1000)
    ref[[0, 1, 2, 7, 5, 6]] = src[[3, 4, 5, 0, 8, 9]]
    assert torch.equal(dst.cpu(), ref)
    back = torch.zeros(3, 1000).pin_memory()
    copy_rows_async(back, [0, 1, 2], dst, [7, 0, 6])       # device -> pinned host
    torch.cuda.synchronize()
    assert torch.equal(back, ref[[7, 0, 6]])


# ---- expert slot pool (reference tests/test_experts.py scenarios) -----------------------------

def _expert(seed, H=8, I=16):
    g = torch.Generator().manual_seed(seed)
    return ExpertWeights(torch.randn(I, H, generator=g), torch.randn(H, I, generator=g),
                         torch.randn(I, H, generator=g))


EXPERT_BYTES = _expert(0).bytes()


@pytest.fixture
def bank():
    b = ExpertBank()
    for l in range(2):
        for e in range(4):
            b.add(l, e, _expert(l * 100 + e))
    return b


def _pool(bank, n, dev):
    return ExpertSlotPool(bank, budget_bytes=n * EXPERT_BYTES, device=dev)


def test_pool_lru_and_pins(dev, bank):
    p = _pool(bank, 3, dev)
    p.ensure(0, [0, 1]); p.release(0, [0, 1])
    p.ensure(0, [0]); p.release(0, [0])
    p.ensure(0, [2, 3]); p.release(0, [2, 3])
    assert (0, 1) not in p.pool and {(0, 0), (0, 2), (0, 3)} <= set(p.pool._pages)
    q = _pool(bank, 3, dev)
    q.ensure(0, [0, 1]); q.release(0, [0])
    q.ensure(0, [2, 3]); q.release(0, [2, 3])
    assert (0, 1) in q.pool and (0, 0) not in q.pool
    r = _pool(bank, 2, dev)
    r.ensure(0, [0, 1])
    assert r.pool.evict_to_fit(EXPERT_BYTES) == []
    with pytest.raises(AssertionError):
        _pool(bank, 0, dev)


def test_pool_hits_identity_and_data(dev, bank):
    p = _pool(bank, 4, dev)
    r1 = p.ensure(0, [1, 3]); p.release(0, [1, 3])
    r2 = p.ensure(0, [1, 3]); p.release(0, [1, 3])
    assert (p.hits, p.misses) == (2, 2) and r2[1] is r1[1] and r2[3] is r1[3]
    for e, w in r1.items():
        ref = bank[(0, e)]
        for a, b in zip((w.w1, w.w2, w.w3), (ref.w1, ref.w2, ref.w3)):
            assert a.device.type == "cuda" and torch.equal(a.cpu(), b)
    with pytest.raises(AssertionError):
        p.release(0, [1, 1, 1])


def test_pool_single_slot_serves_everything(dev, bank):
    p = _pool(bank, 1, dev)
    for l in range(2):
        for e in range(4):
            got = p.ensure(l, [e])
            assert torch.equal(got[e].w2.cpu(), bank[(l, e)].w2)
            p.release(l, [e])
    assert p.pool.used_bytes <= EXPERT_BYTES


def test_pool_policy_matches_oracle_on_random_traffic(dev, bank):
    rng = np.random.default_rng(9)
    p = _pool(bank, 3, dev)
    o = OC.SlotPoolPolicy({k: EXPERT_BYTES for k in bank.keys()}, 3 * EXPERT_BYTES)
    for _ in range(40):
        layer = int(rng.integers(0, 2))
        ids = rng.choice(4, size=int(rng.integers(1, 3)), replace=False).tolist()
        got = p.ensure(layer, ids)
        o.ensure(layer, ids)
        for e in ids:
            assert torch.equal(got[e].w1.cpu(), bank[(layer, e)].w1)
        p.release(layer, ids)
        o.release(layer, ids)
        assert set(p.pool._pages) == o.resident()
    assert (p.hits, p.misses) == (o.hits, o.misses)


def test_alloc_pinned_exact(dev):
    """Exact-size page-locked host tensors: pinned, contiguous, of the asked shape and dtype;
    rows move to and from the device bit for bit, also through the multi-bank index copy that
    reads them through their device mapping; a tensor of 0 elements has its shape."""
    from plastic_infer.kernel.pinned import alloc_pinned_exact

    g = torch.Generator().manual_seed(61)
    for dtype, shape in ((torch.bfloat16, (5, 3, 256)), (torch.float32, (7, 100)),
                         (torch.float16, (1, 8))):
        t = alloc_pinned_exact(shape, dtype)
        assert t.shape == shape and t.dtype == dtype and t.is_contiguous() and t.is_pinned()
        src = torch.randn(shape, generator=g).to(dtype)
        t.copy_(src)
        d = t.to(dev, non_blocking=True)
        torch.cuda.synchronize(dev)
        assert torch.equal(d.cpu(), src)
        back = alloc_pinned_exact(shape, dtype)
        back.copy_(d, non_blocking=True)
        torch.cuda.synchronize(dev)
        assert torch.equal(back, src)
    bank = alloc_pinned_exact((6, 512), torch.bfloat16)
    bank.copy_(torch.randn(6, 512, generator=g).to(torch.bfloat16))
    dst = torch.zeros(4, 512, dtype=torch.bfloat16, device=dev)
    dp = torch.tensor([dst.data_ptr()], dtype=torch.int64, device=dev)
    sp = torch.tensor([device_ptr(bank)], dtype=torch.int64, device=dev)
    fb = torch.tensor([1024], dtype=torch.int64, device=dev)
    fast_index_copy_multi(dp, sp, fb, torch.tensor([3, 0], dtype=torch.int32, device=dev),
                          torch.tensor([5, 2], dtype=torch.int32, device=dev))
    exp = torch.zeros(4, 512, dtype=torch.bfloat16)
    exp[3], exp[0] = bank[5], bank[2]
    assert torch.equal(dst.cpu(), exp)
    z = alloc_pinned_exact((0, 4), torch.bfloat16)
    assert z.shape == (0, 4) and z.dtype == torch.bfloat16
