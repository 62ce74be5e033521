"""Byte-budgeted LRU pool with pin reference counts (host bookkeeping of HBM residency).

Contract of the reference's LruPool (src/plastic_infer/store/resident.py:43-208):
  * eviction never takes a page with pinned > 0 (the single safety invariant);
  * pin / unpin / add / set_tier mark a page most recently used;
  * unpin of an unpinned page and remove of a pinned page raise AssertionError;
  * evict_lru walks oldest -> newest, skipping pinned and non-GPU pages, until the freed bytes
    reach the request (or nothing evictable is left);
  * used_bytes counts pages on the GPU tier only (set_tier moves bytes in and out of it).
Single-threaded: the owner thread drives it; copies overlap through streams, not threads.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Generic, Hashable, TypeVar

from .tiers import Tier

K = TypeVar("K", bound=Hashable)


@dataclass
class Page(Generic[K]):
    """A tracked object: key, size, tier and pin count (pinned > 0 = in use, not evictable)."""
    key: K
    bytes_: int
    tier: Tier
    pinned: int = 0
    _lru_seq: int = field(default=0, repr=False, compare=False)


class LruPool(Generic[K]):
    def __init__(self, budget_bytes: int) -> None:
        self._budget = budget_bytes
        self._pages: dict[K, Page[K]] = {}
        self._order: OrderedDict[K, None] = OrderedDict()   # oldest first
        self._seq = 0
        self._used = 0

    # -- queries ------------------------------------------------------------------------------
    @property
    def budget_bytes(self) -> int:
        return self._budget

    @property
    def used_bytes(self) -> int:
        return self._used

    @property
    def free_bytes(self) -> int:
        return self._budget - self._used

    def __contains__(self, key: K) -> bool:
        return key in self._pages

    def get(self, key: K) -> Page[K] | None:
        return self._pages.get(key)

    def __getitem__(self, key: K) -> Page[K]:
        return self._pages[key]

    def __len__(self) -> int:
        return len(self._pages)

    def lru_keys(self) -> list[K]:
        """Keys from least to most recently used."""
        return list(self._order)

    # -- insertion / removal ------------------------------------------------------------------
    def add(self, key: K, bytes_: int, tier: Tier = Tier.GPU) -> Page[K]:
        assert key not in self._pages, f"duplicate key {key}"
        assert bytes_ >= 0
        page = Page(key=key, bytes_=bytes_, tier=tier)
        self._pages[key] = page
        if tier == Tier.GPU:
            self._used += bytes_
        self._touch(page)
        return page

    def remove(self, key: K) -> Page[K]:
        page = self._pages[key]
        assert page.pinned == 0, f"cannot remove pinned page {key}"
        del self._pages[key]
        del self._order[key]
        if page.tier == Tier.GPU:
            self._used -= page.bytes_
        return page

    # -- pin counts ---------------------------------------------------------------------------
    def pin(self, key: K) -> Page[K]:
        page = self._pages[key]
        page.pinned += 1
        self._touch(page)
        return page

    def unpin(self, key: K) -> None:
        page = self._pages[key]
        assert page.pinned > 0, f"unpin of already-unpinned page {key}"
        page.pinned -= 1
        self._touch(page)

    # -- eviction -----------------------------------------------------------------------------
    def can_fit(self, bytes_: int) -> bool:
        return self._used + bytes_ <= self._budget

    def evict_lru(self, need_bytes: int) -> list[Page[K]]:
        out: list[Page[K]] = []
        freed = 0
        for key in list(self._order):
            if freed >= need_bytes:
                break
            page = self._pages[key]
            if page.pinned > 0 or page.tier != Tier.GPU:
                continue
            out.append(self.remove(key))
            freed += page.bytes_
        return out

    def evict_to_fit(self, bytes_: int) -> list[Page[K]]:
        if self.can_fit(bytes_):
            return []
        return self.evict_lru(bytes_ - self.free_bytes)

    def all_pinned(self) -> bool:
        return all(p.pinned > 0 or p.tier != Tier.GPU for p in self._pages.values())

    # -- tiers --------------------------------------------------------------------------------
    def set_tier(self, key: K, new_tier: Tier) -> None:
        page = self._pages[key]
        if page.tier == Tier.GPU and new_tier != Tier.GPU:
            self._used -= page.bytes_
        elif page.tier != Tier.GPU and new_tier == Tier.GPU:
            self._used += page.bytes_
        page.tier = new_tier
        self._touch(page)

    def _touch(self, page: Page[K]) -> None:
        self._seq += 1
        page._lru_seq = self._seq
        self._order.pop(page.key, None)
        self._order[page.key] = None
