"""GPU parity of the module functions of plastic_infer.moe.offload_kernels (reference
src/plastic_infer/moe/offload_kernels.py:19-94, 226-285, 413-431) on an OffloadMoeCache, and of
the cache's rebuild / validate_rebuild (reference src/plastic_infer/moe/offload_cache.py:410-496)
and routing statistics (:866-971).

Maps, usage, clock and copy plan are compared bit for bit with oracle/slot_cache.py; slot rows
bit for bit with the pinned host banks. The routing statistics are pinned by closed forms
(uniform and one-expert routing) and by a histogram counted on the host."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle.slot_cache as SC
from plastic_infer.moe import offload_kernels as OK
from plastic_infer.moe.offload_cache import OffloadMoeCache
from test_gpu_slot_cache import _banks, _check_resident

pytestmark = pytest.mark.gpu


def _assert_maps(cache, st):
    assert np.array_equal(cache.slot_for_id.cpu().numpy().reshape(-1), st["slot_of_id"])
    assert np.array_equal(cache.id_of_slot.cpu().numpy(), st["id_of_slot"])
    assert np.array_equal(cache.usage.cpu().numpy(), st["usage"])
    assert int(cache.step) == st["step"]


def _assert_plan(cache, src, dst, n):
    assert int(cache.num_indices) == n
    assert np.array_equal(cache.evict_slots[:n].cpu().numpy(), dst)
    assert np.array_equal(cache.src_indices[:n].cpu().numpy(), src)


def test_module_functions_match_oracle(dev):
    """ensure_experts, materialize_layer, prefill_hit_compact and reset_cache called through
    the module, as the reference's cache calls them, on a cache under the global LRU."""
    L, E, H, I, B, K, S = 4, 16, 128, 64, 6, 4, 40
    banks = _banks(L, E, H, I, 41)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=S, device=dev)
    cache.collect_stats = True
    cache.set_bank_sources(banks)
    st = SC.new_state(L * E, S)
    rng = np.random.default_rng(42)
    for step in range(6):
        for layer in range(L):
            ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(B)])
            out, src, dst, n, _ = SC.lru_ensure(st, ids.reshape(-1), id_base=layer * E)
            t = torch.tensor(ids, dtype=torch.int32, device=dev)
            OK.ensure_experts(cache, layer, t)
            assert np.array_equal(t.cpu().numpy().reshape(-1), out)
            _assert_plan(cache, src, dst, n)
            cache.copy_missing()
            _check_resident(cache, banks, layer, ids.reshape(-1), out)
    _assert_maps(cache, st)

    # prefill_hit_compact: the experts of a layer resident at or above slot 2E, in id order
    for layer in range(L):
        for buf in (0, 1):
            OK.prefill_hit_compact(cache, layer, buf)
            row = cache.slot_for_id[layer].cpu().numpy()
            d, s_, n = SC.prefill_hit_compact(row, buf * E, 2 * E)
            assert int(cache._prefill_hit_num) == n
            assert np.array_equal(cache._prefill_hit_dst[:n].cpu().numpy(), d)
            assert np.array_equal(cache._prefill_hit_src[:n].cpu().numpy(), s_)
    with pytest.raises(ValueError):
        OK.prefill_hit_compact(cache, L, 0)

    # materialize_layer: slots [0, E) take the layer in id order, the plan copies it all
    SC.materialize(st, 2, E)
    OK.materialize_layer(cache, 2)
    _assert_maps(cache, st)
    _assert_plan(cache, np.arange(E), np.arange(E), E)
    cache.copy_missing()
    _check_resident(cache, banks, 2, range(E), range(E))

    # decode continues on the materialized maps
    ids = rng.choice(E, size=(B, K))
    out, src, dst, n, _ = SC.lru_ensure(st, ids.reshape(-1), id_base=3 * E)
    t = torch.tensor(ids, dtype=torch.int32, device=dev)
    OK.ensure_experts(cache, 3, t)
    assert np.array_equal(t.cpu().numpy().reshape(-1), out)
    _assert_plan(cache, src, dst, n)

    SC.reset(st)
    OK.reset_cache(cache)
    _assert_maps(cache, st)
    with pytest.raises(NotImplementedError):
        OK.ensure_experts_hybrid(cache, 0, t, 4)


@pytest.mark.parametrize("policy", ["lru", "static"])
def test_rebuild_resizes_in_place(dev, policy):
    """rebuild(): same object, new slot count, maps and stats cold, host banks kept; decode on
    the rebuilt cache follows the oracle from a fresh state ("lru") and places the resident
    experts again ("static"). An invalid size is rejected with the cache unchanged."""
    L, E, H, I, B, K = 3, 16, 128, 64, 5, 4
    banks = _banks(L, E, H, I, 43)
    R = 4 if policy == "static" else None
    size0 = 40 if policy == "lru" else L * 4 + 2 * E     # room for the two prefill buffers
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=size0, device=dev,
                            cache_policy=policy, resident_per_layer=R, prefill_overlap=True)
    cache.collect_stats = True
    cache.collect_decode_freq = True
    resident = [[(5 * l + j) % E for j in range(4)] for l in range(L)] \
        if policy == "static" else None
    cache.set_bank_sources(banks, resident_experts=resident)
    rng = np.random.default_rng(44)
    for layer in range(L):
        t = torch.tensor(rng.choice(E, size=(B, K)), dtype=torch.int32, device=dev)
        cache.ensure_experts(layer, t)
        cache.copy_missing()
    assert int(cache.decode_freq.sum()) == L * B * K
    before = cache.slot_for_id.cpu().clone()

    with pytest.raises(ValueError):
        cache.rebuild(E - 1)
    assert cache.cache_size == size0 and torch.equal(cache.slot_for_id.cpu(), before)
    if policy == "static":
        with pytest.raises(ValueError):
            cache.validate_rebuild(L * 4 + (E - 4) - 1)   # staging short of one layer's others
        cache.validate_rebuild(L * 4 + (E - 4))

    new_size = 28 if policy == "lru" else L * 4 + (E - 4) + 2
    with pytest.warns(RuntimeWarning, match="prefill overlap"):
        cache.rebuild(new_size)
    assert cache.cache_size == new_size and not cache.prefill_overlap
    for t in cache.bank_views():
        assert t.shape[0] == new_size
    assert cache.id_of_slot.numel() == new_size and cache.usage.numel() == new_size
    assert int(cache.decode_freq.sum()) == 0 and int(cache.lru_stats.sum()) == 0
    assert cache.decode_miss_stats()["layer_calls"] == 0
    if policy == "lru":
        assert int((cache.slot_for_id >= 0).sum()) == 0 and int(cache.step) == 0
        st = SC.new_state(L * E, new_size)
        for step in range(4):
            for layer in range(L):
                ids = rng.choice(E, size=(B, K))
                out, _, _, _, _ = SC.lru_ensure(st, ids.reshape(-1), id_base=layer * E)
                t = torch.tensor(ids, dtype=torch.int32, device=dev)
                cache.ensure_experts(layer, t)
                cache.copy_missing()
                assert np.array_equal(t.cpu().numpy().reshape(-1), out)
                _check_resident(cache, banks, layer, ids.reshape(-1), out)
        _assert_maps(cache, st)
    else:
        for l in range(L):
            rs = sorted(resident[l])
            assert cache.resident_experts(l).tolist() == rs
            _check_resident(cache, banks, l, rs, [l * 4 + j for j in range(4)])
        for layer in range(L):
            ids = rng.choice(E, size=(B, K))
            t = torch.tensor(ids, dtype=torch.int32, device=dev)
            cache.ensure_experts(layer, t)
            _check_resident(cache, banks, layer, ids.reshape(-1), t.cpu().numpy().reshape(-1))
    # a size with room for the buffers again does not switch prefill overlap back on
    cache.rebuild(new_size + 2 * E)
    assert cache.cache_size == new_size + 2 * E and not cache.prefill_overlap


def test_decode_routing_stats_closed_forms(dev):
    """Uniform routing over all E experts: working set E, normalised entropy 1, 90 % of the
    routes need ceil(0.9 E) experts, and the oracle that keeps cache_size / L experts per
    layer hits (cache_size / L) / E of them. One-expert routing: working set 1, entropy 0, one
    expert for 90 %, oracle hit 1. A random routing: decode_freq equals the host histogram and
    layers that saw no routes are left out of the averages."""
    L, E, H, I = 3, 16, 128, 64
    banks = _banks(L, E, H, I, 45)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=24, device=dev)
    cache.set_bank_sources(banks)
    assert cache.decode_routing_stats() == {}
    cache.collect_decode_freq = True
    uniform = torch.arange(E, dtype=torch.int32, device=dev).repeat(3).view(-1, 4)
    for layer in range(L):
        cache.ensure_experts(layer, uniform.clone())
        cache.copy_missing()
    r = cache.decode_routing_stats()
    assert r["working_set_mean"] == E and r["working_set_max"] == E
    assert r["experts_for_90pct"] == math.ceil(0.9 * E)
    assert r["norm_entropy"] == pytest.approx(1.0, abs=1e-9)
    assert r["slots_per_layer"] == pytest.approx(24 / L)
    assert r["oracle_hit_at_slots"] == pytest.approx(round(24 / L) / E, abs=1e-12)

    cache.decode_freq.zero_()
    one = torch.full((8, 4), 5, dtype=torch.int32, device=dev)
    cache.ensure_experts(1, one)      # only layer 1 sees routes
    cache.copy_missing()
    r = cache.decode_routing_stats()
    assert r["working_set_mean"] == 1 and r["working_set_max"] == 1
    assert r["experts_for_90pct"] == 1 and r["oracle_hit_at_slots"] == 1.0
    assert r["norm_entropy"] == pytest.approx(0.0, abs=1e-9)

    cache.decode_freq.zero_()
    rng = np.random.default_rng(46)
    hist = np.zeros((L, E), np.int64)
    for step in range(5):
        for layer in range(L):
            ids = rng.choice(E, size=(6, 4))
            if step == 2 and layer == 0:
                ids[0, 0] = -1                               # an invalid id is not counted
            for e in ids.reshape(-1):
                if 0 <= e < E:
                    hist[layer, e] += 1
            t = torch.tensor(ids, dtype=torch.int32, device=dev)
            cache.stage_layer(layer, t)                      # the staged path counts too
    assert np.array_equal(cache.decode_freq.cpu().numpy(), hist)
    cache.record_decode_stats(0)                             # a no-op, kept for call sites
