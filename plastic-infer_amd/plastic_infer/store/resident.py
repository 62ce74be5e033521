"""Byte-budgeted residency tracker with pin counts (host bookkeeping of what is in HBM).

Public surface of the reference's LruPool (src/plastic_infer/store/resident.py:43-208), with
this contract:
  * a tracked object (Page) has a key, a byte size, a tier and a pin count; pinned > 0 means
    some consumer is using it and it must not be evicted or removed;
  * every add / pin / unpin / set_tier counts as a use: the object becomes the most recent;
  * only objects on the GPU tier count against the byte budget;
  * evict_lru(n) removes unpinned GPU-tier objects from the least recent on until at least n
    bytes are freed or none is left, and returns them in that order;
  * removing a pinned object, unpinning an unpinned one or adding a duplicate key raises
    AssertionError.

Structure: each page carries the stamp of its last use from a monotone clock, and a min-heap
holds (stamp, key) entries. A use pushes a new entry instead of moving the old one, so heap
entries whose stamp is no longer the page's are stale and dropped when they surface; the heap
is rebuilt from the live pages when stale entries outnumber them, so it stays O(live pages).
Eviction pops from the heap in stamp order, sets pinned or off-GPU pages aside and pushes them
back afterwards. Single-threaded: the owner thread drives it; copies overlap through streams.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field
from typing import Generic, Hashable, Iterator, TypeVar

from .tiers import Tier

K = TypeVar("K", bound=Hashable)


@dataclass
class Page(Generic[K]):
    """A tracked object: key, size, tier and pin count (pinned > 0: in use, not evictable)."""
    key: K
    bytes_: int
    tier: Tier
    pinned: int = 0
    stamp: int = field(default=0, repr=False, compare=False)   # clock value of the last use


class LruPool(Generic[K]):
    """Residency tracker: budget in bytes, pages by key, eviction by least recent use."""

    def __init__(self, budget_bytes: int) -> None:
        self._budget = int(budget_bytes)
        self._resident_bytes = 0               # GPU-tier bytes only
        self._pages: dict[K, Page[K]] = {}
        self._clock = 0
        self._heap: list[tuple[int, int, K]] = []   # (stamp, tiebreak, key); may hold stale
        self._tiebreak = 0

    # ---- state ---------------------------------------------------------------------------------

    @property
    def budget_bytes(self) -> int:
        return self._budget

    @property
    def used_bytes(self) -> int:
        return self._resident_bytes

    @property
    def free_bytes(self) -> int:
        return self._budget - self._resident_bytes

    def can_fit(self, bytes_: int) -> bool:
        return self._resident_bytes + bytes_ <= self._budget

    def __len__(self) -> int:
        return len(self._pages)

    def __contains__(self, key: K) -> bool:
        return key in self._pages

    def __getitem__(self, key: K) -> Page[K]:
        return self._pages[key]

    def get(self, key: K) -> Page[K] | None:
        return self._pages.get(key)

    def lru_keys(self) -> list[K]:
        """Keys from least to most recently used."""
        return [p.key for p in sorted(self._pages.values(), key=lambda p: p.stamp)]

    def all_pinned(self) -> bool:
        """True when nothing on the GPU tier could be evicted."""
        return not any(p.pinned == 0 and p.tier == Tier.GPU for p in self._pages.values())

    # ---- use stamps ----------------------------------------------------------------------------

    def _use(self, page: Page[K]) -> None:
        self._clock += 1
        page.stamp = self._clock
        self._tiebreak += 1
        heapq.heappush(self._heap, (page.stamp, self._tiebreak, page.key))
        if len(self._heap) > 2 * len(self._pages) + 64:
            self._heap = [(p.stamp, i, p.key) for i, p in enumerate(self._pages.values())]
            heapq.heapify(self._heap)
            self._tiebreak = len(self._heap)

    def _oldest_first(self) -> Iterator[Page[K]]:
        """Pops live pages in stamp order (stale heap entries are dropped on the way)."""
        while self._heap:
            stamp, _, key = heapq.heappop(self._heap)
            page = self._pages.get(key)
            if page is not None and page.stamp == stamp:
                yield page

    # ---- membership ----------------------------------------------------------------------------

    def add(self, key: K, bytes_: int, tier: Tier = Tier.GPU) -> Page[K]:
        assert key not in self._pages, f"key {key!r} is already tracked"
        assert bytes_ >= 0, "negative size"
        page = Page(key=key, bytes_=int(bytes_), tier=tier)
        self._pages[key] = page
        if tier == Tier.GPU:
            self._resident_bytes += page.bytes_
        self._use(page)
        return page

    def remove(self, key: K) -> Page[K]:
        page = self._pages[key]
        assert page.pinned == 0, f"{key!r} is pinned and cannot be removed"
        del self._pages[key]                     # its heap entries are now stale
        if page.tier == Tier.GPU:
            self._resident_bytes -= page.bytes_
        return page

    # ---- pins ----------------------------------------------------------------------------------

    def pin(self, key: K) -> Page[K]:
        page = self._pages[key]
        page.pinned += 1
        self._use(page)
        return page

    def unpin(self, key: K) -> None:
        page = self._pages[key]
        assert page.pinned > 0, f"{key!r} is not pinned"
        page.pinned -= 1
        self._use(page)

    # ---- tiers ---------------------------------------------------------------------------------

    def set_tier(self, key: K, new_tier: Tier) -> None:
        page = self._pages[key]
        was_gpu, now_gpu = page.tier == Tier.GPU, new_tier == Tier.GPU
        self._resident_bytes += page.bytes_ * (int(now_gpu) - int(was_gpu))
        page.tier = new_tier
        self._use(page)

    # ---- eviction ------------------------------------------------------------------------------

    def evict_lru(self, need_bytes: int) -> list[Page[K]]:
        """Remove unpinned GPU-tier pages, least recent first, until need_bytes are freed."""
        evicted: list[Page[K]] = []
        kept: list[Page[K]] = []
        freed = 0
        if need_bytes > 0:
            for page in self._oldest_first():
                if page.pinned or page.tier != Tier.GPU:
                    kept.append(page)
                    continue
                evicted.append(self.remove(page.key))
                freed += page.bytes_
                if freed >= need_bytes:
                    break
        for page in kept:                        # back in the heap with their own stamps
            self._tiebreak += 1
            heapq.heappush(self._heap, (page.stamp, self._tiebreak, page.key))
        return evicted

    def evict_to_fit(self, bytes_: int) -> list[Page[K]]:
        """Evict just enough for bytes_ more to fit (nothing when it already fits)."""
        if self.can_fit(bytes_):
            return []
        return self.evict_lru(bytes_ - self.free_bytes)
