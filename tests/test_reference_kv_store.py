"""The reference's KV-store test cases (reference tests/test_kv_store.py), one for one, run on
this package's HBM store. The reference runs them on a CPU store; here the pools live on the HIP
device and every page write and chunk move goes through the HIP kernels. Same config, same token
ids, same expectations; data comparisons are exact (the reference allows 1e-6 on pure copies).
"""

from __future__ import annotations

import pytest
import torch

from plastic_infer.kv.kv_store import KVConfig, KVStore

pytestmark = pytest.mark.gpu


@pytest.fixture
def store(dev) -> KVStore:
    # reference tests/test_kv_store.py:15-33: 2 layers, 2 kv heads, head_dim 4, 4-token pages,
    # 2 pages per chunk (8 tokens), 64 pages, 8 host chunks, fp32
    return KVStore(KVConfig(n_layers=2, n_kv_heads=2, head_dim=4, page_size=4, pages_per_chunk=2,
                            max_pages=64, max_host_chunks=8, dtype=torch.float32, device=dev))


def _token_kv(store: KVStore, seed: int):
    """One token's K and V, [n_layers, n_kv_heads, head_dim], seeded (reference :36-41)."""
    c = store.config
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(c.n_layers, c.n_kv_heads, c.head_dim, generator=g)
    v = torch.randn(c.n_layers, c.n_kv_heads, c.head_dim, generator=g)
    return k.to(store.gpu.device), v.to(store.gpu.device)


def _write(cache, store, seeds):
    for s in seeds:
        cache.append_token(*_token_kv(store, s))


def _chunk_from_pages(store, cache, chunk, n_tok):
    """Chunk `chunk` of a request read token by token from its pages: [L, H, D, n_tok]."""
    c = store.config
    k = torch.zeros(c.n_layers, c.n_kv_heads, c.head_dim, n_tok)
    v = torch.zeros_like(k)
    kp, vp = store.gpu.k_pages.cpu(), store.gpu.v_pages.cpu()
    for layer in range(c.n_layers):
        for t in range(n_tok):
            pos = chunk * n_tok + t
            phys = cache.block_table.get_page(layer, pos // c.page_size)
            k[layer, :, :, t] = kp[phys, :, :, pos % c.page_size]
            v[layer, :, :, t] = vp[phys, :, :, pos % c.page_size]
    return k, v


# ---- TestBasicAppend (reference :43-86) ---------------------------------------------------------

def test_append_increments_length(store):
    cache = store.new_request()
    _write(cache, store, [0])
    assert cache.length == 1
    assert cache.block_table.num_logical_pages(0) == 1


def test_append_page_full_allocates_new_page(store):
    cache = store.new_request()
    P = store.config.page_size
    _write(cache, store, range(P + 1))
    assert cache.length == P + 1
    assert cache.block_table.num_logical_pages(0) == 2


def test_data_written_correctly(store):
    cache = store.new_request()
    k, v = _token_kv(store, 42)
    cache.append_token(k, v)
    phys = cache.block_table.get_page(0, 0)
    assert torch.equal(store.gpu.k_pages[phys, :, :, 0], k[0])
    assert torch.equal(store.gpu.v_pages[phys, :, :, 0], v[0])


def test_free_request_reclaims_pages(store):
    cache = store.new_request()
    _write(cache, store, range(20))
    assert store.gpu.allocator.used_pages > 0
    store.free_request(cache)
    assert store.gpu.allocator.used_pages == 0
    assert store.gpu.allocator.free_pages == store.config.max_pages


# ---- TestChunkSinking (reference :89-180) -------------------------------------------------------

def test_sink_one_chunk(store):
    cache = store.new_request()
    C = store.config.tokens_per_chunk
    _write(cache, store, range(C))
    cache.set_token_ids(list(range(C)))
    assert cache.num_complete_chunks() == 1
    assert len(cache.chunk_keys) == 1
    assert store.sink_completed_chunks(cache) == 1
    assert store.host_cache_size == 1


def test_sink_incremental(store):
    cache = store.new_request()
    C = store.config.tokens_per_chunk
    first = int(C * 1.5)
    _write(cache, store, range(first))
    cache.set_token_ids(list(range(first)))
    assert store.sink_completed_chunks(cache) == 1   # only the full chunk
    assert store.host_cache_size == 1
    _write(cache, store, range(first, 2 * C))
    cache.set_token_ids(list(range(2 * C)))
    assert store.sink_completed_chunks(cache) == 1   # the second chunk
    assert store.host_cache_size == 2


def test_sunk_data_roundtrip(store):
    cache = store.new_request()
    C = store.config.tokens_per_chunk
    _write(cache, store, [i * 7 for i in range(C)])
    cache.set_token_ids(list(range(C)))
    k_ref, v_ref = _chunk_from_pages(store, cache, 0, C)
    store.sink_completed_chunks(cache)
    host_k, host_v = store._host_cache[cache.chunk_keys[0].full_key]
    assert torch.equal(host_k.cpu(), k_ref) and torch.equal(host_v.cpu(), v_ref)


def test_host_eviction(store):
    cache = store.new_request()
    C = store.config.tokens_per_chunk
    n_chunks = store.config.max_host_chunks + 3
    _write(cache, store, [i * 11 for i in range(n_chunks * C)])
    cache.set_token_ids(list(range(n_chunks * C)))
    assert store.sink_completed_chunks(cache) == n_chunks
    assert store.host_cache_size == store.config.max_host_chunks


# ---- TestPrefixLoad (reference :183-268) --------------------------------------------------------

def test_load_existing_prefix(store):
    C = store.config.tokens_per_chunk
    cache1 = store.new_request()
    tokens = list(range(2 * C))
    _write(cache1, store, range(2 * C))
    cache1.set_token_ids(tokens)
    store.sink_completed_chunks(cache1)
    assert store.host_cache_size == 2
    ref = [_chunk_from_pages(store, cache1, ci, C) for ci in range(2)]
    store.free_request(cache1)

    cache2 = store.new_request()
    matched, keys = store.load_prefix(cache2, tokens)
    assert matched == 2 * C and len(keys) == 2 and cache2.length == 2 * C
    for ci in range(2):
        got = _chunk_from_pages(store, cache2, ci, C)
        assert torch.equal(got[0], ref[ci][0]) and torch.equal(got[1], ref[ci][1])


def test_prefix_partial_hit(store):
    C = store.config.tokens_per_chunk
    cache1 = store.new_request()
    _write(cache1, store, range(C))
    cache1.set_token_ids(list(range(C)))
    store.sink_completed_chunks(cache1)
    store.free_request(cache1)
    cache2 = store.new_request()
    matched, keys = store.load_prefix(cache2, list(range(3 * C)))
    assert matched == C and len(keys) == 1


def test_prefix_no_hit(store):
    cache = store.new_request()
    matched, keys = store.load_prefix(cache, [999, 998, 997])
    assert matched == 0 and keys == [] and cache.length == 0


def test_prefix_empty_cache(store):
    cache = store.new_request()
    matched, _ = store.load_prefix(cache, [1, 2, 3])
    assert matched == 0


# ---- TestEviction (reference :271-289) ----------------------------------------------------------

def test_evict_frees_pages(store):
    C = store.config.tokens_per_chunk
    cache = store.new_request()
    _write(cache, store, range(4 * C))
    cache.set_token_ids(list(range(4 * C)))
    store.sink_completed_chunks(cache)
    used_before = store.gpu.allocator.used_pages
    freed = store.evict_chunks(need_pages=1, protected_request=cache)
    assert freed >= 1
    assert store.gpu.allocator.used_pages == used_before - freed
