"""GPU parity: slot scatter, block-table gather, page<->chunk copies and the HBM KV store
against the oracle — bit-exact (pure copies)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.paged_kv as OP
import oracle.workloads as W
from plastic_infer.kernel import kv_gather, kv_scatter, pages_chunk_copy, pages_chunks_copy
from plastic_infer.kv.kv_store import KVConfig, KVStore

pytestmark = pytest.mark.gpu


def test_decode_scatter_b32(dev):
    wl = W.decode_b32_small()
    kp, vp = wl.k_pages.clone(), wl.v_pages.clone()
    OP.scatter_slots(wl.k_new, wl.v_new, kp, vp, wl.slot_mapping.tolist())
    gk, gv = wl.k_pages.to(dev), wl.v_pages.to(dev)
    kv_scatter(wl.k_new.to(dev), wl.v_new.to(dev), gk, gv, wl.slot_mapping.to(dev))
    assert torch.equal(gk.cpu(), kp) and torch.equal(gv.cpu(), vp)


def test_prefill_scatter_and_gather_round_trip_8seq(dev):
    wl = W.prefill_write_workload()
    H, D, P = wl.k.shape[1], wl.k.shape[2], wl.page_size
    kp = torch.zeros(wl.num_pages, H, D, P, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    OP.scatter_slots(wl.k, wl.v, kp, vp, wl.slot_mapping.tolist())
    gk, gv = torch.zeros_like(kp, device=dev), torch.zeros_like(vp, device=dev)
    kv_scatter(wl.k.to(dev), wl.v.to(dev), gk, gv, wl.slot_mapping.to(dev))
    assert torch.equal(gk.cpu(), kp) and torch.equal(gv.cpu(), vp)
    k_back, v_back = kv_gather(gk, gv, wl.block_tables.to(dev), wl.cu_seqlens.to(dev), wl.max_len)
    assert torch.equal(k_back.cpu(), wl.k) and torch.equal(v_back.cpu(), wl.v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_scatter_edge_slots(dev, dtype):
    g = torch.Generator().manual_seed(11)
    N_, H, D, P = 6, 2, 8, 4
    kp = torch.randn(N_, H, D, P, generator=g).to(dtype)
    vp = torch.randn(N_, H, D, P, generator=g).to(dtype)
    k = torch.randn(9, H, D, generator=g).to(dtype)
    v = torch.randn(9, H, D, generator=g).to(dtype)
    slots = [3, -1, 23, 0, 24, 1000, 7, 8, 12]   # padding, last slot, out of range
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, [s if s < N_ * P else -1 for s in slots])
    gk, gv = kp.to(dev), vp.to(dev)
    kv_scatter(k.to(dev), v.to(dev), gk, gv, torch.tensor(slots, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)
    kv_scatter(k[:0].to(dev), v[:0].to(dev), gk, gv, torch.empty(0, dtype=torch.int64, device=dev))


def test_scatter_strided_rows_and_tile_path(dev):
    g = torch.Generator().manual_seed(12)
    H, D, P = 2, 16, 4
    src = torch.randn(13, 3, H, D, generator=g).to(torch.bfloat16)
    k, v = src[:, 0], src[:, 2]                    # token stride 3*H*D, rows [H, D] contiguous
    slots = list(range(8, 16)) + [40, 41, 42, 3, 2]   # two full aligned pages then scattered
    kp = torch.zeros(12, H, D, P, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, slots)
    gk, gv = kp.to(dev), vp.to(dev)
    gsrc = src.to(dev)
    kv_scatter(gsrc[:, 0], gsrc[:, 2], gk, gv, torch.tensor(slots, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


@pytest.mark.parametrize("reps", [1, 13])
@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16),
                                     (256, torch.bfloat16)])
def test_scatter16_slot_patterns(dev, D, dtype, reps):
    """16-bit pools with 16-token pages: runs starting at odd offsets and crossing pages, a run
    of whole pages, scattered decode slots, padding and out-of-range slots, a strided source.
    One copy of the pattern (87 tokens) takes the per-(token, kv head) kernel; 13 copies on
    disjoint pages (1131 tokens) take the page-segment kernel."""
    g = torch.Generator().manual_seed(15 + D)
    H, P, N_ = 3, 16, 40 * reps
    runs = []
    for r in range(reps):
        o = 16 * 40 * r
        runs += (list(range(o + 16 * 5 + 3, o + 16 * 5 + 3 + 37))   # offset 3, crosses 3 pages
                 + list(range(o + 16 * 20, o + 16 * 22))             # two whole pages
                 + [o + 16 * 30 + 7, -1, o + 16 * 31, N_ * P + 5, o + 16 * 33 + 15,
                    o + 16 * 34 + 14, o + 16 * 34 + 15]
                 + list(range(o + 16 * 36 + 1, o + 16 * 36 + 12)))   # odd start in one page
    n = len(runs)
    src = torch.randn(n, 2, H, D, generator=g).to(dtype)
    k, v = src[:, 0], src[:, 1]                        # token stride 2*H*D
    kp = torch.randn(N_, H, D, P, generator=g).to(dtype)
    vp = torch.randn(N_, H, D, P, generator=g).to(dtype)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, [s if s < N_ * P else -1 for s in runs])
    gk, gv, gsrc = kp.to(dev), vp.to(dev), src.to(dev)
    kv_scatter(gsrc[:, 0], gsrc[:, 1], gk, gv, torch.tensor(runs, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


@pytest.mark.parametrize("pool_off", [0, 2])
def test_scatter16_whole_pages_pool_alignment(dev, pool_off):
    """Whole-page segments (16 slots from a page start) go out as 16-byte stores when both pools
    are 16-byte aligned; pools 4 bytes off (pool_off = 2 elements) take the dword path. 1157
    tokens, so the page-segment kernel runs; a ragged run at offset 5 rides along. Both bit-exact
    against the oracle."""
    g = torch.Generator().manual_seed(77 + pool_off)
    H, D, P, N_ = 2, 128, 16, 90
    slots = list(range(16 * 3, 16 * 73)) + list(range(16 * 80 + 5, 16 * 80 + 5 + 37))
    n = len(slots)
    k = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    kp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    vp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, slots)
    numel = kp.numel()
    bk = torch.zeros(numel + 8, dtype=torch.bfloat16, device=dev)
    bv = torch.zeros(numel + 8, dtype=torch.bfloat16, device=dev)
    gk = bk[pool_off:pool_off + numel].view(N_, H, D, P)
    gv = bv[pool_off:pool_off + numel].view(N_, H, D, P)
    gk.copy_(kp.to(dev))
    gv.copy_(vp.to(dev))
    assert (gk.data_ptr() % 16 == 0) == (pool_off == 0)
    kv_scatter(k.to(dev), v.to(dev), gk, gv, torch.tensor(slots, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_scatter16_segment_ownership_layouts(dev, seed):
    """More than 1024 tokens (the page-segment kernel) of mixed segments on distinct pages:
    short segments that add up to 16 tokens after a page start, page-start runs followed by
    padding, single decode slots at offset 0, whole pages, the 21 / 11 / 40 ragged batch.
    Bit-exact against the oracle's per-token store."""
    from scatter_layouts import random_layout

    g = torch.Generator().manual_seed(300 + seed)
    H, D, P, N_ = 2, 128, 16, 4096
    slots = random_layout(seed, n_min=1100, n_pages=N_)
    n = len(slots)
    k = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    kp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    vp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, slots)
    gk, gv = kp.to(dev), vp.to(dev)
    kv_scatter(k.to(dev), v.to(dev), gk, gv, torch.tensor(slots, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


def test_scatter16_large_decode_batch_and_padded_runs(dev):
    """2048 single-token decode slots on pages 0..2047 (half at page offset 0) and 20 copies of
    the 21 / 11 / 40 ragged batch on pages from 2048, then a page-start run of 8 followed by 8
    padding slots. No slot repeats, so the result does not depend on write order."""
    from scatter_layouts import ragged_21_11_40

    g = torch.Generator().manual_seed(310)
    H, D, P, N_ = 2, 128, 16, 4096
    perm = torch.randperm(2048, generator=g).tolist()    # pages 0..2047: no slot repeats
    slots = [perm[i] * P + (0 if i % 2 else (i * 7) % P) for i in range(2048)]
    for r in range(20):
        slots += ragged_21_11_40(2048 + 8 * r)
    slots += [3000 * P + i for i in range(8)] + [-1] * 8
    n = len(slots)
    k = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    kp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    vp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, slots)
    gk, gv = kp.to(dev), vp.to(dev)
    kv_scatter(k.to(dev), v.to(dev), gk, gv, torch.tensor(slots, device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


def test_scatter_single_token_with_strided_heads(dev):
    """One token whose [H, D] row is not contiguous (a head_dim slice of a wider buffer, and a
    head-transposed view): the rows are copied before the kernel reads them."""
    g = torch.Generator().manual_seed(320)
    H, D, P, N_ = 4, 128, 16, 8
    wide = torch.randn(1, H, 2 * D, generator=g).to(torch.bfloat16)
    k = wide[:, :, :D]                               # stride(1) = 2D
    vt = torch.randn(1, D, H, generator=g).to(torch.bfloat16)
    v = vt.transpose(1, 2)                           # stride(2) = H
    kp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    vp = torch.randn(N_, H, D, P, generator=g).to(torch.bfloat16)
    ref_k, ref_v = kp.clone(), vp.clone()
    OP.scatter_slots(k, v, ref_k, ref_v, [5 * P + 3])
    gk, gv = kp.to(dev), vp.to(dev)
    kv_scatter(wide.to(dev)[:, :, :D], vt.to(dev).transpose(1, 2), gk, gv,
               torch.tensor([5 * P + 3], device=dev))
    assert torch.equal(gk.cpu(), ref_k) and torch.equal(gv.cpu(), ref_v)


def test_gather16_tables_with_invalid_pages(dev):
    g = torch.Generator().manual_seed(16)
    H, D, P = 4, 128, 16
    kp = torch.randn(30, H, D, P, generator=g).to(torch.bfloat16)
    vp = torch.randn(30, H, D, P, generator=g).to(torch.bfloat16)
    tables = [[7, 3, 29], [12], [0, 5, -1, 8], []]
    lens = [40, 16, 60, 0]
    bt = torch.full((4, 4), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t, dtype=torch.int32)
    cu = torch.tensor([0] + list(np.cumsum(lens)))
    k, v = kv_gather(kp.to(dev), vp.to(dev), bt.to(dev), cu.to(dev), 64)
    for b, t in enumerate(tables):
        if not lens[b]:
            continue
        ok = [p if p >= 0 else 0 for p in t]
        rk, rv = OP.gather_paged_kv(kp, vp, ok, P, lens[b])
        rk, rv = rk[0].clone(), rv[0].clone()
        for i, p in enumerate(t):
            if p < 0:                                   # an invalid page reads as zeros
                rk[i * P:(i + 1) * P] = 0
                rv[i * P:(i + 1) * P] = 0
        assert torch.equal(k[cu[b]:cu[b + 1]].cpu(), rk)
        assert torch.equal(v[cu[b]:cu[b + 1]].cpu(), rv)


def test_gather_matches_oracle_and_empty(dev):
    g = torch.Generator().manual_seed(13)
    kp = torch.randn(9, 3, 8, 5, generator=g)
    vp = torch.randn(9, 3, 8, 5, generator=g)
    tables = [[4, 0, 7], [2], [8, 1, 3]]
    lens = [13, 0, 15]
    bt = torch.zeros(3, 3, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t)
    cu = torch.tensor([0, 13, 13, 28])
    k, v = kv_gather(kp.to(dev), vp.to(dev), bt.to(dev), cu.to(dev), 15)
    for b, t in enumerate(tables):
        rk, rv = OP.gather_paged_kv(kp, vp, t, 5, lens[b])
        assert torch.equal(k[cu[b]:cu[b + 1]].cpu(), rk[0])
        assert torch.equal(v[cu[b]:cu[b + 1]].cpu(), rv[0])


def test_pages_chunk_copy_both_ways(dev):
    g = torch.Generator().manual_seed(14)
    pages = torch.randn(20, 2, 4, 4, generator=g)
    ids = [3, 9, -1, 0, 17, 5]                  # 2 layers x 3 pages per chunk, one absent
    ref = OP.pages_to_chunk(pages, ids, 2, 3)
    chunk = torch.zeros(2, 2, 4, 12, device=dev)
    pages_chunk_copy(chunk, pages.to(dev), torch.tensor(ids, device=dev), to_chunk=True)
    assert torch.equal(chunk.cpu(), ref)
    back = torch.zeros(20, 2, 4, 4, device=dev)
    pages_chunk_copy(chunk, back, torch.tensor(ids, device=dev), to_chunk=False)
    for l in range(2):
        for p in range(3):
            pid = ids[l * 3 + p]
            if pid >= 0:
                assert torch.equal(back[pid].cpu(), pages[pid])


@pytest.mark.parametrize("where", ["device", "pinned"])
@pytest.mark.parametrize("dtype,P", [(torch.float32, 4), (torch.bfloat16, 4),
                                     (torch.bfloat16, 16), (torch.bfloat16, 3)])
def test_pages_chunks_copy_many_chunks(dev, where, dtype, P):
    """Several chunks in one launch, each at its own address (HBM or pinned host memory),
    page rows of 16, 8 and 6 bytes (16-, 8- and 2-byte words), absent pages left alone."""
    g = torch.Generator().manual_seed(15 + P)
    L, H, D, ppc, n_pages, n_chunks = 3, 2, 8, 2, 40, 4
    pages = torch.randn(n_pages, H, D, P, generator=g).to(dtype)
    perm = torch.randperm(n_pages, generator=g).tolist()
    ids = perm[:n_chunks * L * ppc]
    ids[5] = -1
    ids[17] = -1
    if where == "pinned":
        chunks = [torch.zeros(L, H, D, ppc * P, dtype=dtype, pin_memory=True)
                  for _ in range(n_chunks)]
    else:
        chunks = [torch.zeros(L, H, D, ppc * P, dtype=dtype, device=dev) for _ in range(n_chunks)]
    ids_t = torch.tensor(ids, dtype=torch.int64, device=dev)
    pages_chunks_copy(chunks, pages.to(dev), ids_t, to_chunk=True)
    torch.cuda.synchronize()
    per = L * ppc
    for c in range(n_chunks):
        ref = OP.pages_to_chunk(pages, ids[c * per:(c + 1) * per], L, ppc)
        assert torch.equal(chunks[c].cpu(), ref), c
    back = torch.zeros(n_pages, H, D, P, dtype=dtype, device=dev)
    pages_chunks_copy(chunks, back, ids_t, to_chunk=False)
    back = back.cpu()
    listed = {pid for pid in ids if pid >= 0}
    for pid in range(n_pages):
        want = pages[pid] if pid in listed else torch.zeros_like(pages[pid])
        assert torch.equal(back[pid], want), pid


def test_pages_chunks_copy_rejects_pageable_and_bad_ids(dev):
    pages = torch.zeros(8, 2, 4, 4, device=dev)
    ids = torch.zeros(2 * 1 * 2, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        pages_chunks_copy([torch.zeros(1, 2, 4, 8), torch.zeros(1, 2, 4, 8)], pages, ids, True)
    good = [torch.zeros(1, 2, 4, 8, device=dev) for _ in range(2)]
    with pytest.raises(ValueError):
        pages_chunks_copy(good, pages, ids[:3], True)
    with pytest.raises(ValueError):
        pages_chunks_copy([good[0], torch.zeros(1, 2, 4, 4, device=dev)], pages, ids, True)


# ---- KV store (the reference's tests/test_kv_store.py scenarios, pools in HBM) ----------------

@pytest.fixture
def store(dev) -> KVStore:
    return KVStore(KVConfig(n_layers=2, n_kv_heads=2, head_dim=4, page_size=4, pages_per_chunk=2,
                            max_pages=64, max_host_chunks=8, dtype=torch.float32, device=dev))


def _kv(store, seed):
    g = torch.Generator().manual_seed(seed)
    c = store.config
    k = torch.randn(c.n_layers, c.n_kv_heads, c.head_dim, generator=g)
    v = torch.randn(c.n_layers, c.n_kv_heads, c.head_dim, generator=g)
    return k.to(store.gpu.device), v.to(store.gpu.device)


def test_store_rejects_host_device():
    with pytest.raises(ValueError):
        KVStore(KVConfig(n_layers=1, n_kv_heads=1, head_dim=4, device=torch.device("cpu")))


def test_store_append_and_placement(store):
    cache = store.new_request()
    for i in range(5):
        cache.append_token(*_kv(store, i))
    assert cache.length == 5 and cache.block_table.num_logical_pages(0) == 2
    assert store.gpu.allocator.used_pages == 4
    k, v = _kv(store, 4)
    phys = cache.block_table.get_page(1, 1)
    assert torch.equal(store.gpu.k_pages[phys, :, :, 0], k[1])
    assert torch.equal(store.gpu.v_pages[phys, :, :, 0], v[1])
    store.free_request(cache)
    assert store.gpu.allocator.free_pages == 64


def test_store_sink_round_trip_and_host_lru(store):
    cfg = store.config
    cache = store.new_request()
    n = cfg.tokens_per_chunk * (cfg.max_host_chunks + 3)
    for i in range(n):
        cache.append_token(*_kv(store, i * 7))
    cache.set_token_ids(list(range(n)))
    assert store.sink_completed_chunks(cache) == cfg.max_host_chunks + 3
    assert store.host_cache_size == cfg.max_host_chunks
    key = cache.chunk_keys[-1].full_key
    hk, hv = store._host_cache[key]
    c = len(cache.chunk_keys) - 1
    for layer in range(cfg.n_layers):
        for t in range(cfg.tokens_per_chunk):
            g = c * cfg.tokens_per_chunk + t
            phys = cache.block_table.get_page(layer, g // cfg.page_size)
            assert torch.equal(hk[layer, :, :, t], store.gpu.k_pages[phys, :, :, g % cfg.page_size].cpu())
            assert torch.equal(hv[layer, :, :, t], store.gpu.v_pages[phys, :, :, g % cfg.page_size].cpu())


def test_store_prefix_load(store):
    cfg = store.config
    C = cfg.tokens_per_chunk
    c1 = store.new_request()
    toks = list(range(2 * C))
    for i in range(len(toks)):
        c1.append_token(*_kv(store, i))
    c1.set_token_ids(toks)
    store.sink_completed_chunks(c1)
    ref = {}
    for layer in range(cfg.n_layers):
        for t in range(2 * C):
            phys = c1.block_table.get_page(layer, t // cfg.page_size)
            ref[(layer, t)] = store.gpu.k_pages[phys, :, :, t % cfg.page_size].clone()
    store.free_request(c1)
    c2 = store.new_request()
    matched, keys = store.load_prefix(c2, toks + [999])
    assert matched == 2 * C and len(keys) == 2 and c2.length == 2 * C
    for (layer, t), val in ref.items():
        phys = c2.block_table.get_page(layer, t // cfg.page_size)
        assert torch.equal(store.gpu.k_pages[phys, :, :, t % cfg.page_size], val)
    c3 = store.new_request()
    assert store.load_prefix(c3, [999, 998, 997]) == (0, [])


def test_store_evict_chunks(store):
    C = store.config.tokens_per_chunk
    cache = store.new_request()
    for i in range(4 * C):
        cache.append_token(*_kv(store, i))
    cache.set_token_ids(list(range(4 * C)))
    used = store.gpu.allocator.used_pages
    freed = store.evict_chunks(need_pages=1, protected_request=cache)
    assert freed >= 1 and store.gpu.allocator.used_pages == used - freed


def test_store_sink_and_load_many_bf16_chunks(dev):
    """Five 64-token chunks of a 4-layer bf16 store sink in one launch per pool and load back
    in one launch per pool; both directions bit-exact against the oracle's page<->chunk copy."""
    cfg = KVConfig(n_layers=4, n_kv_heads=2, head_dim=64, page_size=16, pages_per_chunk=4,
                   max_pages=256, max_host_chunks=16, dtype=torch.bfloat16, device=dev)
    store = KVStore(cfg)
    C = cfg.tokens_per_chunk
    n = 5 * C + 7
    cache = store.new_request()
    cache._ensure_pages(n)
    cache._length = n
    g = torch.Generator().manual_seed(21)
    kp = torch.randn(store.gpu.k_pages.shape, generator=g).to(torch.bfloat16)
    vp = torch.randn(store.gpu.v_pages.shape, generator=g).to(torch.bfloat16)
    store.gpu.k_pages.copy_(kp)
    store.gpu.v_pages.copy_(vp)
    toks = list(range(1000, 1000 + n))
    cache.set_token_ids(toks)
    assert store.sink_completed_chunks(cache) == 5
    assert store.sink_completed_chunks(cache) == 0
    for c, key in enumerate(cache.chunk_keys):
        ids = store._chunk_page_ids(cache, c)
        hk, hv = store._host_cache[key.full_key]
        assert hk.is_pinned() and hv.is_pinned()
        assert torch.equal(hk, OP.pages_to_chunk(kp, ids, cfg.n_layers, cfg.pages_per_chunk))
        assert torch.equal(hv, OP.pages_to_chunk(vp, ids, cfg.n_layers, cfg.pages_per_chunk))
    old_tables = [list(cache.block_table.pages[l]) for l in range(cfg.n_layers)]
    store.free_request(cache)
    store.gpu.k_pages.zero_()
    store.gpu.v_pages.zero_()
    c2 = store.new_request()
    matched, keys = store.load_prefix(c2, toks)
    assert matched == 5 * C and len(keys) == 5
    k_now, v_now = store.gpu.k_pages.cpu(), store.gpu.v_pages.cpu()
    for layer in range(cfg.n_layers):
        for lp in range(5 * cfg.pages_per_chunk):
            new_pid = c2.block_table.get_page(layer, lp)
            old_pid = old_tables[layer][lp]
            assert torch.equal(k_now[new_pid], kp[old_pid])
            assert torch.equal(v_now[new_pid], vp[old_pid])
