"""Page allocator and per-request block table (host bookkeeping of the HBM page pool).

Same contract as the reference's kv.paged (src/plastic_infer/kv/paged.py:30-157):
  * PageAllocator hands out global page ids LIFO: a fresh allocator yields 0, 1, 2, ...;
    a freed page is the next one handed out. Exhaustion raises IndexError; freeing a page
    that is not in use raises AssertionError.
  * BlockTable maps (layer, logical page) -> physical page; logical page i of a layer holds
    tokens [i*page_size, (i+1)*page_size).
Pure host logic: no tensors, no device calls. Block tables are exported to the device as int32
rows by the KV store when a kernel needs them.
"""

from __future__ import annotations

from dataclasses import dataclass, field

DEFAULT_PAGE_SIZE: int = 16   # tokens per page
DEFAULT_CHUNK_PAGES: int = 16  # pages per chunk (256 tokens)


@dataclass
class BlockTable:
    """Logical-to-physical page map of one request, one list per layer."""

    n_layers: int
    page_size: int
    pages: list[list[int]] = field(default_factory=list)

    def __post_init__(self) -> None:
        if not self.pages:
            self.pages = [[] for _ in range(self.n_layers)]

    def num_logical_pages(self, layer: int) -> int:
        return len(self.pages[layer])

    def num_tokens(self, layer: int) -> int:
        """Token capacity of the layer's pages (a multiple of page_size)."""
        return len(self.pages[layer]) * self.page_size

    def get_page(self, layer: int, logical_page_idx: int) -> int:
        return self.pages[layer][logical_page_idx]

    def get_page_for_token(self, layer: int, token_idx: int) -> int:
        return self.pages[layer][token_idx // self.page_size]

    def append_page(self, layer: int, phys_page_id: int) -> None:
        self.pages[layer].append(phys_page_id)

    def all_page_ids(self) -> set[int]:
        out: set[int] = set()
        for row in self.pages:
            out.update(row)
        return out

    def chunk_page_ids(self, chunk_idx: int, pages_per_chunk: int) -> list[int]:
        """Pages of logical range [chunk_idx*ppc, (chunk_idx+1)*ppc) in every layer, layer-major;
        a partially written chunk yields only the pages that exist."""
        lo = chunk_idx * pages_per_chunk
        hi = lo + pages_per_chunk
        out: list[int] = []
        for row in self.pages:
            out.extend(row[lo:hi])
        return out

    def is_chunk_complete(self, chunk_idx: int, pages_per_chunk: int) -> bool:
        need = (chunk_idx + 1) * pages_per_chunk
        return all(len(row) >= need for row in self.pages)


class PageAllocator:
    """LIFO free list over page ids 0..total_pages-1."""

    def __init__(self, total_pages: int) -> None:
        assert total_pages > 0, "total_pages must be positive"
        self._total = total_pages
        # Stack top is the end of the list: page 0 is handed out first on a fresh allocator.
        self._stack: list[int] = list(range(total_pages - 1, -1, -1))
        self._in_use = bytearray(total_pages)

    @property
    def total_pages(self) -> int:
        return self._total

    @property
    def free_pages(self) -> int:
        return len(self._stack)

    @property
    def used_pages(self) -> int:
        return self._total - len(self._stack)

    def is_used(self, page_id: int) -> bool:
        return 0 <= page_id < self._total and bool(self._in_use[page_id])

    def alloc(self) -> int:
        if not self._stack:
            raise IndexError("out of pages")
        pid = self._stack.pop()
        self._in_use[pid] = 1
        return pid

    def alloc_many(self, count: int) -> list[int]:
        if count > len(self._stack):
            raise IndexError(f"need {count} pages, only {len(self._stack)} free")
        if count <= 0:
            return []
        ids = self._stack[-count:][::-1]   # the order repeated alloc() calls would give
        del self._stack[-count:]
        for pid in ids:
            self._in_use[pid] = 1
        return ids

    def free(self, page_id: int) -> None:
        assert self.is_used(page_id), f"page {page_id} not in use"
        self._in_use[page_id] = 0
        self._stack.append(page_id)

    def free_many(self, page_ids: list[int]) -> None:
        """Free several pages; they are pushed in list order (the last one is reused first)."""
        seen: set[int] = set()
        for pid in page_ids:
            assert self.is_used(pid) and pid not in seen, f"page {pid} not in use"
            seen.add(pid)
        for pid in page_ids:
            self._in_use[pid] = 0
        self._stack.extend(page_ids)
