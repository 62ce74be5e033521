"""GPU parity of the device slot cache (LRU admission, bookkeeping kernels) and of
OffloadMoeCache's decode / prefill expert movement. Every check is bit-exact: maps, usage,
clock, plan, stats against the oracle; slot-cache rows against the pinned host banks."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.slot_cache as SC
from plastic_infer.kernel.fast_index_copy import fast_index_copy_jit, fast_index_copy_multi_jit
from plastic_infer.kernel.lru_ensure import N_STATS, lru_ensure
from plastic_infer.moe.offload_cache import OffloadMoeCache

pytestmark = pytest.mark.gpu


class DevState:
    def __init__(self, dev, num_total: int, num_cached: int):
        self.slot_of_id = torch.full((num_total,), -1, dtype=torch.int32, device=dev)
        self.id_of_slot = torch.full((num_cached,), -1, dtype=torch.int32, device=dev)
        self.usage = torch.zeros(num_cached, dtype=torch.int64, device=dev)
        self.step = torch.zeros((), dtype=torch.int64, device=dev)
        plan = num_cached
        self.src = torch.full((plan,), -7, dtype=torch.int32, device=dev)
        self.dst = torch.full((plan,), -7, dtype=torch.int32, device=dev)
        self.num = torch.zeros(1, dtype=torch.int64, device=dev)
        self.stats = torch.zeros(N_STATS, dtype=torch.int64, device=dev)

    def ensure(self, query: np.ndarray, id_base: int):
        q = torch.tensor(query, dtype=torch.int32, device=self.slot_of_id.device)
        lru_ensure(q, self.slot_of_id, self.id_of_slot, self.usage, self.step, q, self.src,
                   self.dst, self.num, stats=self.stats, id_base=id_base)
        return q.cpu().numpy()

    def assert_equal(self, st: dict):
        assert np.array_equal(self.slot_of_id.cpu().numpy(), st["slot_of_id"])
        assert np.array_equal(self.id_of_slot.cpu().numpy(), st["id_of_slot"])
        assert np.array_equal(self.usage.cpu().numpy(), st["usage"])
        assert int(self.step) == st["step"]


@pytest.mark.parametrize("seed,layers,experts,cached,k,calls", [
    (0, 4, 16, 20, 12, 40),       # small cache, constant cross-layer eviction
    (1, 48, 128, 3072, 512, 12),  # Qwen3-30B-A3B decode shape: B=64 x top-8 over 50% slots
    (2, 2, 8, 8, 64, 30),         # many duplicates, cache exactly one layer
    (3, 1, 2048, 2048, 2048, 4),  # the largest query held in LDS
    (4, 3, 1, 1, 3, 10),          # one slot
    (5, 48, 128, 3072, 4096, 10), # 512 rows x top-8: the wide-query kernel
    (6, 2, 6000, 5000, 6000, 5),  # up to 5000 misses a call: several batches of 2048
    (7, 3, 40, 50, 2500, 12),     # long queries of few distinct ids, many duplicates
])
def test_lru_ensure_matches_oracle(dev, seed, layers, experts, cached, k, calls):
    rng = np.random.default_rng(seed)
    total = layers * experts
    st, ds = SC.new_state(total, cached), DevState(dev, total, cached)
    stats = np.zeros(3, np.int64)
    for c in range(calls):
        layer = int(rng.integers(0, layers))
        distinct = int(rng.integers(1, min(experts, cached, k) + 1))
        ids = rng.choice(experts, size=distinct, replace=False)
        query = rng.choice(ids, size=k) if c % 3 else ids
        print(f"call {c}: layer {layer}, {query.size} ids, {distinct} distinct", flush=True)
        out, src, dst, n, dstats = SC.lru_ensure(st, query, id_base=layer * experts)
        got = ds.ensure(query, layer * experts)
        stats += np.asarray(dstats)
        assert np.array_equal(got, out), c
        assert int(ds.num) == n
        assert np.array_equal(ds.src[:n].cpu().numpy(), src)
        assert np.array_equal(ds.dst[:n].cpu().numpy(), dst)
        ds.assert_equal(st)
    assert np.array_equal(ds.stats.cpu().numpy(), stats)


def test_lru_ensure_largest_cache_and_inert_ids(dev):
    total, cached = 40000, 16384
    st, ds = SC.new_state(total, cached), DevState(dev, total, cached)
    rng = np.random.default_rng(7)
    for c in range(6):
        query = rng.choice(total, size=2048, replace=False)
        out, src, dst, n, _ = SC.lru_ensure(st, query)
        assert np.array_equal(ds.ensure(query, 0), out)
        ds.assert_equal(st)
    # ids outside [0, num_total) are inert: out -1, nothing admitted for them
    q = np.array([5, -3, total + 10, 5], np.int64)
    out, _, _, n, _ = SC.lru_ensure(st, q[[0, 3]])
    got = ds.ensure(q, 0)
    assert got.tolist() == [out[0], -1, -1, out[1]]
    ds.assert_equal(st)


def test_lru_ensure_fragmented_usage_rounds_and_sorted_path(dev):
    """Victims come in rounds of equal usage; a call needing more than 8 rounds takes the
    sorted path. Single-id calls give every slot its own usage value, so a call with m misses
    needs m rounds: 8 stays on the rounds, 9 and 40 take the sorted path."""
    total, cached = 1000, 64
    st, ds = SC.new_state(total, cached), DevState(dev, total, cached)
    nxt = 0

    def call(query):
        out, src, dst, n, _ = SC.lru_ensure(st, np.asarray(query, np.int64))
        got = ds.ensure(np.asarray(query, np.int64), 0)
        assert np.array_equal(got, out)
        assert int(ds.num) == n
        assert np.array_equal(ds.src[:n].cpu().numpy(), src)
        assert np.array_equal(ds.dst[:n].cpu().numpy(), dst)
        ds.assert_equal(st)

    for _ in range(cached):                 # one new id per call: 64 distinct usage values
        call([nxt])
        nxt += 1
    for m in (40, 8, 9, 3, 1, 16):
        call(list(range(nxt, nxt + m))[::-1])
        nxt += m
        for _ in range(5):                  # re-fragment a few slots
            call([nxt])
            nxt += 1


def test_lru_ensure_more_misses_than_slots_admits_what_fits(dev):
    ds = DevState(dev, 100, 4)
    ds.ensure(np.array([1, 2]), 0)
    got = ds.ensure(np.array([2, 9, 8, 7, 6]), 0)   # 2 hits; 4 misses, 3 evictable slots
    assert got[0] == ds.slot_of_id[2].item() and int(ds.num) == 3
    assert sorted(got[1:].tolist()) == [-1] + sorted(set(range(4)) - {got[0]})
    assert got[1] == -1                               # the largest missing id is left out


def test_materialize_reset_invalidate_compact_match_oracle(dev):
    from plastic_infer import _native as N

    L, E, C = 3, 8, 20
    st, ds = SC.new_state(L * E, C), DevState(dev, L * E, C)
    rng = np.random.default_rng(11)
    for c in range(8):
        layer = c % L
        q = rng.choice(E, size=5, replace=False)
        SC.lru_ensure(st, q, id_base=layer * E)
        ds.ensure(q, layer * E)
    s = torch.cuda.current_stream(dev).cuda_stream
    ev = torch.full((C,), -1, dtype=torch.int32, device=dev)
    srci = torch.full((C,), -1, dtype=torch.int32, device=dev)
    num = torch.zeros(1, dtype=torch.int64, device=dev)
    ref_ev, ref_src, ref_n = SC.materialize(st, 1, E)
    N.call("pia_slot_cache_materialize", ds.slot_of_id.data_ptr(), L * E, ds.id_of_slot.data_ptr(),
           ds.usage.data_ptr(), C, ds.step.data_ptr(), ev.data_ptr(), srci.data_ptr(),
           num.data_ptr(), 1, E, s)
    ds.assert_equal(st)
    assert ev[:E].cpu().tolist() == ref_ev.tolist() and srci[:E].cpu().tolist() == ref_src.tolist()
    assert int(num) == ref_n
    SC.invalidate(st, 2, 11)
    N.call("pia_slot_cache_invalidate", ds.slot_of_id.data_ptr(), L * E, ds.id_of_slot.data_ptr(),
           ds.usage.data_ptr(), C, 2, 11, s)
    ds.assert_equal(st)
    row = torch.tensor([3, -1, 25, 4, 19, 30, 0, 16], dtype=torch.int32, device=dev)
    hd = torch.full((8,), -1, dtype=torch.int32, device=dev)
    hs = torch.full((8,), -1, dtype=torch.int32, device=dev)
    N.call("pia_prefill_hit_compact", row.data_ptr(), hd.data_ptr(), hs.data_ptr(), num.data_ptr(),
           8, 16, 8, s)
    rd, rs, rn = SC.prefill_hit_compact(row.cpu().numpy(), 8, 16)
    assert int(num) == rn and hd[:rn].cpu().tolist() == rd.tolist()
    assert hs[:rn].cpu().tolist() == rs.tolist()
    SC.reset(st)
    N.call("pia_slot_cache_reset", ds.slot_of_id.data_ptr(), L * E, ds.id_of_slot.data_ptr(),
           ds.usage.data_ptr(), C, ds.step.data_ptr(), None, 0, num.data_ptr(), s)
    ds.assert_equal(st)
    assert int(num) == 0


@pytest.mark.parametrize("seed,total,cached,k,calls,spread", [
    (10, 60000, 40000, 2000, 26, False),    # warm-up, then evictions among clustered usages
    (11, 50000, 40000, 64, 3, False),       # a fresh cache: every usage 0, ties by slot
    (12, 70000, 48000, 1500, 6, True),      # usages spread over five bytes: multi-pass select
    (13, 200000, 131075, 700, 4, False),    # an odd cache size past 2^17
])
def test_lru_ensure_streamed_large_cache_matches_oracle(dev, seed, total, cached, k, calls,
                                                        spread):
    """Caches beyond the LDS-resident 16384 slots take the streaming admission kernel: the same
    maps, usage, clock, plan and stats as the oracle's sequential argmin rule, call by call."""
    rng = np.random.default_rng(seed)
    st, ds = SC.new_state(total, cached), DevState(dev, total, cached)
    if spread:   # usages of a long-running cache: distinct values over ~2^40
        u = rng.integers(0, 1 << 40, size=cached).astype(np.int64)
        st["usage"][:] = u
        ds.usage.copy_(torch.from_numpy(u))
        st["step"] = 1 << 41
        ds.step.fill_(1 << 41)
    stats = np.zeros(3, np.int64)
    for c in range(calls):
        ids = rng.choice(total, size=k, replace=False)
        query = np.concatenate([ids, ids[: k // 10]])[:k] if c % 2 else ids
        out, src, dst, n, dstats = SC.lru_ensure(st, query)
        stats += dstats
        got = ds.ensure(query, 0)
        assert np.array_equal(got, out), c
        assert int(ds.num) == n
        assert np.array_equal(ds.dst.cpu().numpy()[:n], dst)
        assert np.array_equal(ds.src.cpu().numpy()[:n], src)
    ds.assert_equal(st)
    assert np.array_equal(ds.stats.cpu().numpy(), stats)


# ---- OffloadMoeCache --------------------------------------------------------------------------

def _banks(L: int, E: int, H: int, I: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    gate_up = [torch.randn(E, 2 * I, H, generator=g).to(torch.bfloat16).pin_memory()
               for _ in range(L)]
    down = [torch.randn(E, H, I, generator=g).to(torch.bfloat16).pin_memory() for _ in range(L)]
    return {"gate_up": gate_up, "down": down}


def _check_resident(cache, banks, layer: int, experts, slots):
    gu, dn = cache.bank_caches["gate_up"], cache.bank_caches["down"]
    for e, s in zip(experts, slots):
        assert torch.equal(gu[s].cpu(), banks["gate_up"][layer][e]), (layer, e, s)
        assert torch.equal(dn[s].cpu(), banks["down"][layer][e]), (layer, e, s)


@pytest.mark.parametrize("fused", [True, False])
def test_offload_cache_decode_steps(dev, fused):
    L, E, H, I, B, K = 4, 16, 128, 64, 6, 4
    banks = _banks(L, E, H, I, 3)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=24, device=dev,
                            multi_bank_copy=fused)
    cache.collect_stats = True
    cache.set_bank_sources(banks)
    assert cache._banks.multi_ok == fused
    st = SC.new_state(L * E, 24)
    rng = np.random.default_rng(5)
    stats = np.zeros((L, 3), np.int64)
    for step in range(12):
        for layer in range(L):
            ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(B)])
            out, _, _, _, dstats = SC.lru_ensure(st, ids.reshape(-1), id_base=layer * E)
            stats[layer] += dstats
            t = torch.tensor(ids, dtype=torch.int32, device=dev)
            cache.ensure_experts(layer, t)
            cache.copy_missing()
            assert np.array_equal(t.cpu().numpy().reshape(-1), out)
            _check_resident(cache, banks, layer, ids.reshape(-1), out)
    assert np.array_equal(cache.slot_for_id.cpu().numpy().reshape(-1), st["slot_of_id"])
    assert np.array_equal(cache.lru_stats.cpu().numpy(), stats)
    m = cache.decode_miss_stats()
    assert m["layer_calls"] == 12 * L and 0 < m["miss_rate"] <= 1
    cache.materialize_layer(2)
    cache.copy_missing()
    _check_resident(cache, banks, 2, range(E), range(E))
    views = cache.bank_views(E)
    assert torch.equal(views[0].cpu(), banks["gate_up"][2])
    cache.reset()
    assert int((cache.slot_for_id >= 0).sum()) == 0 and int(cache.step) == 0


@pytest.mark.parametrize("hit_d2d", [False, True])
def test_offload_cache_prefill_double_buffer(dev, hit_d2d):
    L, E, H, I = 5, 8, 256, 256       # gate_up rows 256 KiB (gathered), down rows 128 KiB
    banks = _banks(L, E, H, I, 9)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=3 * E, device=dev,
                            prefill_overlap=True, prefill_hit_d2d=hit_d2d)
    cache.set_bank_sources(banks)
    # a decode step first: 4 experts x 5 layers fill slots 0..19, so the last layer's sit
    # above the 2E = 16 slots the buffers own and are gathered device-side
    for layer in range(L):
        ids = torch.tensor([[0, 3], [5, 6]], dtype=torch.int32, device=dev)
        cache.ensure_experts(layer, ids)
        cache.copy_missing()
    compute = torch.cuda.current_stream(dev)
    for rep in range(2):
        cache.begin_prefill()
        cache.prefetch_prefill_layer(0)
        for layer in range(L):
            cache.prefetch_prefill_layer(layer + 1)        # next layer crosses PCIe meanwhile
            gu, dn = cache.wait_prefill_layer(layer)
            scratch = torch.empty_like(gu)
            scratch.copy_(gu)                               # stand-in consumer on the compute stream
            assert torch.equal(gu.cpu(), banks["gate_up"][layer]), (rep, layer)
            assert torch.equal(dn.cpu(), banks["down"][layer]), (rep, layer)
            cache.release_prefill_layer(layer)
        compute.synchronize()
    if hit_d2d:
        assert cache.prefill_hit_rows == 2 * 4 and cache.prefill_total_rows == 2 * L * E
    # decode after prefill: the buffers' slots were invalidated, residency stays consistent
    ids = torch.tensor([[1, 2]], dtype=torch.int32, device=dev)
    cache.ensure_experts(3, ids)
    cache.copy_missing()
    _check_resident(cache, banks, 3, [1, 2], ids.cpu().reshape(-1).tolist())
    sid = cache.slot_for_id.cpu().numpy().reshape(-1)
    ios = cache.id_of_slot.cpu().numpy()
    res = np.nonzero(sid >= 0)[0]
    assert np.array_equal(ios[sid[res]], res)


def test_fast_index_copy_dropin_names(dev):
    g = torch.Generator().manual_seed(2)
    src = torch.randn(10, 64, generator=g).pin_memory()
    dst = torch.zeros(6, 64, device=dev)
    di = torch.tensor([4, 0, 2], dtype=torch.int32, device=dev)
    si = torch.tensor([9, 1, 5], dtype=torch.int32, device=dev)
    n = torch.tensor([2], dtype=torch.int64, device=dev)
    fast_index_copy_jit(dst, di, src, si, n)
    exp = torch.zeros(6, 64)
    exp[4], exp[0] = src[9], src[1]
    assert torch.equal(dst.cpu(), exp)
    with pytest.raises(NotImplementedError):
        fast_index_copy_jit(dst, di, src, si, priority="high")
    from plastic_infer.kernel.pinned import device_ptr

    dst2 = torch.zeros(6, 64, device=dev)
    dp = torch.tensor([dst.data_ptr(), dst2.data_ptr()], dtype=torch.int64, device=dev)
    sp = torch.tensor([device_ptr(src), device_ptr(src)], dtype=torch.int64, device=dev)
    fb = torch.tensor([256, 256], dtype=torch.int64, device=dev)
    fast_index_copy_multi_jit(dp, sp, fb, di, si)
    exp[2] = src[5]
    assert torch.equal(dst.cpu(), exp) and torch.equal(dst2.cpu(), exp)


# ---- staged (DMA, overlapped) decode path -----------------------------------------------------

def _check_routes(cache, banks, layer, ids, routes):
    """Every route's slot holds its expert's rows; in-HBM and copied groups partition the
    routes; returns (slot per route, copied mask) as numpy."""
    a, c = routes.in_hbm.cpu().numpy().reshape(-1), routes.copied.cpu().numpy().reshape(-1)
    assert ((a >= 0) != (c >= 0)).all()
    slots = np.maximum(a, c)
    _check_resident(cache, banks, layer, ids.reshape(-1), slots)
    return slots, c >= 0


def test_offload_cache_static_policy_staging(dev):
    """"static": resident experts sit in fixed slots from the start; every other routed expert
    goes through the host staging LRU (its decisions checked against the slot-cache oracle), is
    copied by DMA on the copy stream and marked as copied; rows bit-exact against the banks."""
    L, E, H, I, B, K, R = 3, 16, 128, 64, 5, 4, 6
    staging = E - R + 4
    banks = _banks(L, E, H, I, 21)
    resident = [[(3 * l + j) % E for j in range(R)] for l in range(L)]
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=L * R + staging, device=dev,
                            cache_policy="static", resident_per_layer=R)
    cache.set_bank_sources(banks, resident_experts=resident)
    for l in range(L):
        rs = sorted(resident[l])
        _check_resident(cache, banks, l, rs, [l * R + j for j in range(R)])
        assert cache.resident_experts(l).tolist() == rs
    st = SC.new_state(L * E, staging)
    rng = np.random.default_rng(22)
    compute = torch.cuda.current_stream(dev)
    for step in range(10):
        for layer in range(L):
            ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(B)])
            routes = cache.stage_layer(layer, torch.tensor(ids, dtype=torch.int32, device=dev))
            compute.wait_event(routes.ready)
            slots, copied = _check_routes(cache, banks, layer, ids, routes)
            flat = ids.reshape(-1)
            res = np.isin(flat, resident[layer])
            assert not copied[res].any()
            stage_ids = np.unique(flat[~res]) + layer * E
            out, src, dst, n, _ = SC.lru_ensure(st, stage_ids)
            exp = dict(zip(stage_ids.tolist(), (out + L * R).tolist()))
            for f, s_, cp in zip(flat[~res] + layer * E, slots[~res], copied[~res]):
                assert exp[int(f)] == s_
                assert cp == (int(f) in src.tolist())
            assert routes.copied_experts == n
    m = cache.decode_miss_stats()
    assert m["layer_calls"] == 10 * L and 0 < m["miss_rate"] < 1


def test_offload_cache_lru_policy_staged_matches_oracle(dev):
    """"lru" through stage_layer: the device admission's decisions equal the oracle's; the
    planned rows are copied by DMA; copied routes are exactly those of this call's plan."""
    L, E, H, I, B, K = 4, 16, 128, 64, 6, 4
    banks = _banks(L, E, H, I, 23)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=24, device=dev)
    cache.collect_stats = True
    cache.set_bank_sources(banks)
    st = SC.new_state(L * E, 24)
    rng = np.random.default_rng(24)
    compute = torch.cuda.current_stream(dev)
    for step in range(8):
        for layer in range(L):
            ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(B)])
            out, src, dst, n, _ = SC.lru_ensure(st, ids.reshape(-1), id_base=layer * E)
            routes = cache.stage_layer(layer, torch.tensor(ids, dtype=torch.int32, device=dev))
            compute.wait_event(routes.ready)
            slots, copied = _check_routes(cache, banks, layer, ids, routes)
            assert np.array_equal(slots, out)
            assert np.array_equal(copied, np.isin(out, dst))
    assert np.array_equal(cache.slot_for_id.cpu().numpy().reshape(-1), st["slot_of_id"])


@pytest.mark.parametrize("policy", ["lru", "static"])
def test_two_pass_routed_ffn_is_bit_identical(dev, policy):
    """The FFN over the in-HBM routes, then (after the copy event) the copied routes, summed
    once, equals one FFN over all routes on the same slots, bit for bit."""
    from plastic_infer.kernel import moe_sum_reduce
    from plastic_infer.moe.fused import fused_experts_decode_impl, routed_ffn_routes

    L, E, H, I, B, K = 2, 16, 256, 128, 9, 4
    banks = _banks(L, E, H, I, 25)
    size = 2 * 8 + (E - 8) if policy == "static" else 24
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=size, device=dev,
                            cache_policy=policy)
    cache.set_bank_sources(banks)
    g = torch.Generator().manual_seed(26)
    x = (torch.randn(B, H, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    logits = torch.randn(B, E, generator=g).to(dev)
    from plastic_infer.moe.fused import fused_topk

    for layer in (0, 1, 0):
        w, ids = fused_topk(x, logits, K, True)
        routes = cache.stage_layer(layer, ids)
        gu, dn = cache.bank_views()
        buf = torch.empty(B, K, H, dtype=x.dtype, device=dev)
        routed_ffn_routes(x, gu, dn, w, routes.in_hbm, buf)
        torch.cuda.current_stream(dev).wait_event(routes.ready)
        routed_ffn_routes(x, gu, dn, w, routes.copied, buf)
        two = torch.empty_like(x)
        moe_sum_reduce(buf, two)
        one = fused_experts_decode_impl(x, gu, dn, w, torch.maximum(routes.in_hbm, routes.copied))
        assert torch.equal(two.cpu(), one.cpu()), layer


def test_lru_ensure_wide_query_limits(dev):
    """More than 2048 ids a call are admitted for caches of up to 16384 slots; a longer query
    on a larger cache is refused before any launch (nothing changes)."""
    ds = DevState(dev, 40000, 20000)
    q = torch.arange(3000, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        lru_ensure(q, ds.slot_of_id, ds.id_of_slot, ds.usage, ds.step, q, ds.src, ds.dst, ds.num)
    assert int(ds.step) == 0 and int((ds.slot_of_id >= 0).sum()) == 0
    # 16384 slots, 3000 ids: the wide kernel, checked against the oracle, twice (hits second)
    st, ds = SC.new_state(40000, 16384), DevState(dev, 40000, 16384)
    rng = np.random.default_rng(8)
    for c in range(2):
        query = rng.choice(40000, size=3000)
        out, src, dst, n, _ = SC.lru_ensure(st, query)
        assert np.array_equal(ds.ensure(query, 0), out), c
        assert int(ds.num) == n and np.array_equal(ds.dst[:n].cpu().numpy(), dst)
        assert np.array_equal(ds.src[:n].cpu().numpy(), src)
        ds.assert_equal(st)
