"""KV store: HBM page pool + per-request block tables + host chunk cache with prefix reuse.

Same API and bookkeeping as the reference (src/plastic_infer/kv/kv_store.py:46-406); the data
movement is the HIP library's:
  * append_token writes one token of every layer with ONE slot-mapped scatter launch
    (reference: per-layer advanced-index stores, kv_store.py:134-143);
  * sink_completed_chunks gathers the pages of all new chunks, all layers, with one
    page->chunk kernel per pool that writes their pinned host tensors directly (no device
    staging) and synchronizes once (reference: one blocking .to("cpu") per page,
    kv_store.py:230-276);
  * load_prefix scatters all matched host chunks into freshly allocated pages with one
    chunk->page kernel per pool reading the pinned host tensors directly (reference: per-page
    .to(device), :282-334).
The pools live on a HIP device; a non-HIP device is rejected at construction.
Storage layout: k_pages / v_pages = [total_pages, n_kv_heads, head_dim, page_size].
Host chunks: [n_layers, n_kv_heads, head_dim, tokens_per_chunk] CPU tensors (pinned).
"""

from __future__ import annotations

import array
import heapq
from dataclasses import dataclass, field
from typing import Optional

import torch

from .. import _native as N
from ..kernel.paged_kv import kv_scatter, pages_chunks_copy
from .chunk import ChunkKey, compute_prefix_hashes_and_final, longest_prefix_hits
from .paged import DEFAULT_CHUNK_PAGES, DEFAULT_PAGE_SIZE, BlockTable, PageAllocator


def _ids_tensor(ids: list[int], dev: torch.device) -> torch.Tensor:
    """int64 device tensor of a page-id list (through a packed host buffer: several times
    faster than torch.tensor on a list of tens of thousands of ints)."""
    buf = array.array("q", ids)
    return torch.frombuffer(buf, dtype=torch.int64).to(dev) if ids else \
        torch.empty(0, dtype=torch.int64, device=dev)


def _default_device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
        else torch.device("cuda")


@dataclass
class KVConfig:
    """Shape parameters of the KV store (device defaults to the current HIP device)."""
    n_layers: int
    n_kv_heads: int
    head_dim: int
    page_size: int = DEFAULT_PAGE_SIZE
    pages_per_chunk: int = DEFAULT_CHUNK_PAGES
    max_pages: int = 1024
    max_host_chunks: int = 256
    dtype: torch.dtype = torch.float32
    device: torch.device = field(default_factory=_default_device)

    @property
    def bytes_per_page(self) -> int:
        """K + V bytes of one page (one layer's slice of page_size tokens)."""
        elt = torch.empty((), dtype=self.dtype).element_size()
        return 2 * self.n_kv_heads * self.head_dim * self.page_size * elt

    @property
    def tokens_per_chunk(self) -> int:
        return self.page_size * self.pages_per_chunk


class KVPagedStorage:
    """The K and V page pools of one HIP device plus their page allocator."""

    def __init__(self, config: KVConfig, total_pages: int,
                 device: Optional[torch.device] = None,
                 dtype: Optional[torch.dtype] = None) -> None:
        self.config = config
        self.device = torch.device(device or config.device)
        if self.device.type != "cuda" or torch.version.hip is None:
            raise ValueError(
                f"KV pages live in HBM: device must be a HIP device, got {self.device}")
        self.dtype = dtype or config.dtype
        self.total_pages = total_pages
        self.allocator = PageAllocator(total_pages)
        shape = (total_pages, config.n_kv_heads, config.head_dim, config.page_size)
        self.k_pages = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self.v_pages = torch.zeros(shape, dtype=self.dtype, device=self.device)

    def get_page_k(self, page_id: int) -> torch.Tensor:
        return self.k_pages[page_id]

    def get_page_v(self, page_id: int) -> torch.Tensor:
        return self.v_pages[page_id]


class KVRequestCache:
    """Block table, length and chunk keys of one request."""

    def __init__(self, store: "KVStore", request_id: int = 0) -> None:
        self.store = store
        self.request_id = request_id
        self.cfg = store.config
        self.block_table = BlockTable(n_layers=self.cfg.n_layers, page_size=self.cfg.page_size)
        self._length = 0
        self.chunk_keys: list[ChunkKey] = []
        self._final_hash: Optional[bytes] = None

    @property
    def length(self) -> int:
        return self._length

    def num_complete_chunks(self) -> int:
        return self._length // self.cfg.tokens_per_chunk

    def _ensure_pages(self, n_tokens: int) -> None:
        """Allocate pages so every layer covers n_tokens (layer by layer per new page index,
        the order the reference's append path allocates in)."""
        P = self.cfg.page_size
        need = (n_tokens + P - 1) // P
        alloc = self.store.gpu.allocator
        for page_idx in range(self.block_table.num_logical_pages(0), need):
            for layer in range(self.cfg.n_layers):
                if self.block_table.num_logical_pages(layer) <= page_idx:
                    self.block_table.append_page(layer, alloc.alloc())

    def slot_mapping(self, layer: int, start_pos: int, n: int) -> list[int]:
        """Flat slots (page * page_size + offset) of positions start_pos..start_pos+n-1."""
        P = self.cfg.page_size
        row = self.block_table.pages[layer]
        return [row[p // P] * P + p % P for p in range(start_pos, start_pos + n)]

    def append_token(self, k_token: torch.Tensor, v_token: torch.Tensor) -> None:
        """Append one token's K/V of every layer: k_token, v_token [n_layers, n_kv_heads, head_dim]
        (device tensors of the pool's dtype)."""
        cfg = self.cfg
        pos = self._length
        self._ensure_pages(pos + 1)
        P = cfg.page_size
        slots = [self.block_table.get_page(l, pos // P) * P + pos % P for l in range(cfg.n_layers)]
        gpu = self.store.gpu
        slot_t = torch.tensor(slots, dtype=torch.int64).to(gpu.device, non_blocking=True)
        kv_scatter(k_token, v_token, gpu.k_pages, gpu.v_pages, slot_t)
        self._length += 1

    def set_token_ids(self, token_ids: list[int]) -> None:
        """Set the request's token ids and recompute the keys of its complete chunks."""
        n_full = len(token_ids) // self.cfg.tokens_per_chunk
        if n_full == 0:
            self.chunk_keys = []
            self._final_hash = None
            return
        keys, final_h = compute_prefix_hashes_and_final(
            token_ids[:n_full * self.cfg.tokens_per_chunk], chunk_size=self.cfg.tokens_per_chunk)
        self.chunk_keys = keys
        self._final_hash = final_h

    def get_block_table_for_layer(self, layer: int) -> list[int]:
        return list(self.block_table.pages[layer])

    def block_table_tensor(self, layer: int) -> torch.Tensor:
        """The layer's block table as an int32 device row (for the batched kernels)."""
        return torch.tensor(self.block_table.pages[layer], dtype=torch.int32).to(
            self.store.gpu.device, non_blocking=True)


class KVStore:
    """HBM page pool + host L1 chunk cache + prefix index."""

    def __init__(self, config: KVConfig) -> None:
        self.config = config
        self.gpu = KVPagedStorage(config, total_pages=config.max_pages,
                                  device=config.device, dtype=config.dtype)
        self._host_cache: dict[bytes, tuple[torch.Tensor, torch.Tensor]] = {}
        # Host chunks are replaced least recently used first. Each use stamps its key with the
        # next tick; the heap keeps (tick, key) for every stamp handed out, and a popped entry
        # whose tick is no longer its key's latest is dropped on the spot.
        self._host_tick = 0
        self._host_stamp: dict[bytes, int] = {}
        self._host_heap: list[tuple[int, bytes]] = []
        self._max_host_chunks = config.max_host_chunks
        self._prefix_index: dict[bytes, ChunkKey] = {}
        self._host_reads: Optional[torch.cuda.Event] = None

    # -- request lifecycle --------------------------------------------------------------------

    def new_request(self, request_id: int = 0) -> KVRequestCache:
        return KVRequestCache(self, request_id=request_id)

    def free_request(self, cache: KVRequestCache) -> None:
        self.gpu.allocator.free_many(list(cache.block_table.all_page_ids()))

    # -- chunk sinking (HBM -> host) ----------------------------------------------------------

    def _chunk_page_ids(self, cache: KVRequestCache, chunk_idx: int) -> list[int]:
        """Layer-major page ids of one chunk, -1 where a layer lacks the page."""
        cfg = self.config
        lo = chunk_idx * cfg.pages_per_chunk
        ids: list[int] = []
        for layer in range(cfg.n_layers):
            row = cache.block_table.pages[layer]
            ids.extend(row[p] if p < len(row) else -1 for p in range(lo, lo + cfg.pages_per_chunk))
        return ids

    def _chunk_shape(self) -> tuple[int, int, int, int]:
        cfg = self.config
        return (cfg.n_layers, cfg.n_kv_heads, cfg.head_dim, cfg.tokens_per_chunk)

    def sink_completed_chunks(self, cache: KVRequestCache) -> int:
        """Copy every complete chunk not yet cached to host. Returns the number newly sunk.

        The host-cache bookkeeping runs chunk by chunk in the reference's order (a cached chunk
        is touched; a new one first evicts the LRU entries it needs room for); the data of all
        new chunks that are still cached at the end then moves in ONE page->chunk launch per
        pool, written straight into their pinned host tensors, followed by one synchronize."""
        dev = self.gpu.device
        sunk = 0
        new: list[tuple[int, bytes]] = []
        for chunk_idx, key in enumerate(cache.chunk_keys):
            full_key = key.full_key
            if full_key in self._host_cache:
                self._touch_host(full_key)
                continue
            while len(self._host_cache) >= self._max_host_chunks:
                self._evict_host_lru()
            shape = self._chunk_shape()
            self._host_cache[full_key] = (
                torch.empty(shape, dtype=self.gpu.dtype, pin_memory=True),
                torch.empty(shape, dtype=self.gpu.dtype, pin_memory=True))
            self._prefix_index[full_key] = key
            self._touch_host(full_key)
            new.append((chunk_idx, full_key))
            sunk += 1
        # A chunk evicted again by a later one of the same call never needs its data.
        live = [(idx, k) for idx, k in new if k in self._host_cache]
        if live:
            ids: list[int] = []
            for idx, _ in live:
                ids.extend(self._chunk_page_ids(cache, idx))
            ids_t = _ids_tensor(ids, dev)
            for side, pool in ((0, self.gpu.k_pages), (1, self.gpu.v_pages)):
                pages_chunks_copy([self._host_cache[k][side] for _, k in live], pool, ids_t,
                                  to_chunk=True)
            torch.cuda.current_stream(dev).synchronize()
        return sunk

    # -- prefix loading (host -> HBM) ---------------------------------------------------------

    def load_prefix(self, cache: KVRequestCache, tokens: list[int]
                    ) -> tuple[int, list[ChunkKey]]:
        """Load the longest cached prefix of `tokens` into freshly allocated pages.
        Returns (matched_tokens, matched chunk keys).

        All matched chunks move in ONE chunk->page launch per pool that reads their pinned
        host tensors directly; the call returns with the copy in flight on the current stream
        (kernels queued behind it see the pages), and the host tensors are kept from eviction
        until it has finished."""
        cfg = self.config
        matches, _ = longest_prefix_hits(self._prefix_index, tokens,
                                         chunk_size=cfg.tokens_per_chunk)
        if not matches:
            return 0, []
        need = len(matches) * cfg.n_layers * cfg.pages_per_chunk
        if self.gpu.allocator.free_pages < need:
            self.evict_chunks(need - self.gpu.allocator.free_pages)
        dev = self.gpu.device
        # Page ids in the order the reference's per-page alloc() loop (chunk, layer, page)
        # hands them out; alloc_many yields exactly that sequence.
        ids = self.gpu.allocator.alloc_many(need)
        ppc = cfg.pages_per_chunk
        for m in range(len(matches)):
            for layer in range(cfg.n_layers):
                lo = (m * cfg.n_layers + layer) * ppc
                cache.block_table.pages[layer].extend(ids[lo:lo + ppc])
        ids_t = _ids_tensor(ids, dev)
        for side, pool in ((0, self.gpu.k_pages), (1, self.gpu.v_pages)):
            pages_chunks_copy([self._host_cache[k.full_key][side] for k in matches], pool, ids_t,
                              to_chunk=False)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(dev))
        self._host_reads = done
        cache._length = len(matches) * cfg.tokens_per_chunk
        cache.chunk_keys = list(matches)
        cache._final_hash = matches[-1].cumulative_key
        for key in matches:
            self._touch_host(key.full_key)
        return cache._length, matches

    # -- eviction (HBM pages) -----------------------------------------------------------------

    def evict_chunks(self, need_pages: int,
                     protected_request: Optional[KVRequestCache] = None) -> int:
        """Free pages of the oldest complete chunks of `protected_request` (never its newest
        complete chunk) until need_pages are freed. Without a request nothing is evicted."""
        if protected_request is None:
            return 0
        cfg = self.config
        freed = 0
        for chunk_idx in range(protected_request.num_complete_chunks() - 1):
            if freed >= need_pages:
                break
            ids = [p for p in self._chunk_page_ids(protected_request, chunk_idx) if p >= 0]
            self.gpu.allocator.free_many(ids)
            freed += len(ids)
        return freed

    # -- host LRU -----------------------------------------------------------------------------

    def _touch_host(self, full_key: bytes) -> None:
        """Mark a cached chunk as used now."""
        self._host_tick += 1
        self._host_stamp[full_key] = self._host_tick
        heapq.heappush(self._host_heap, (self._host_tick, full_key))
        if len(self._host_heap) > 4 * len(self._host_stamp) + 64:  # mostly superseded stamps
            self._host_heap = [(t, k) for k, t in self._host_stamp.items()]
            heapq.heapify(self._host_heap)

    def _evict_host_lru(self) -> None:
        """Drop the cached chunk whose last use is the oldest (nothing when the cache is empty)."""
        while self._host_heap:
            tick, key = heapq.heappop(self._host_heap)
            if self._host_stamp.get(key) != tick:
                continue
            del self._host_stamp[key]
            if self._host_reads is not None:
                # A prefix load may still be reading this chunk's pinned memory.
                self._host_reads.synchronize()
                self._host_reads = None
            del self._host_cache[key]
            self._prefix_index.pop(key, None)
            return

    @property
    def host_cache_size(self) -> int:
        return len(self._host_cache)
