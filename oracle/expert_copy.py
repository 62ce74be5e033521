"""ORACLE (test infrastructure only): row index copy and the expert slot-pool LRU policy."""

from __future__ import annotations

from collections import OrderedDict

import numpy as np


def index_copy_rows(dst: np.ndarray, dst_idx, src: np.ndarray, src_idx, n: int | None = None) -> None:
    """reference src/plastic_infer/kernel/csrc/jit/fast_index_copy.cuh:190-286 (row semantics):
    dst[dst_idx[i]] = src[src_idx[i]] for i < n (n defaults to len(dst_idx)); rows with a
    negative index are skipped. dst/src are [rows, ...] arrays of equal row size."""
    di = np.asarray(dst_idx, dtype=np.int64).reshape(-1)
    si = np.asarray(src_idx, dtype=np.int64).reshape(-1)
    count = di.size if n is None else min(n, di.size)
    for i in range(count):
        if di[i] < 0 or si[i] < 0:
            continue
        dst[di[i]] = src[si[i]]


class SlotPoolPolicy:
    """The residency decisions of ExpertSlotPool + LruPool (reference
    src/plastic_infer/store/experts.py:178-223, src/plastic_infer/store/resident.py:82-170)
    over keys with byte sizes, without any tensors: which ensure() visits are hits, which
    misses, what gets evicted."""

    def __init__(self, sizes: dict, budget: int) -> None:
        self.sizes = sizes
        self.budget = budget
        self.order: OrderedDict = OrderedDict()   # resident keys, least recent first
        self.pins: dict = {}
        self.used = 0
        self.hits = 0
        self.misses = 0
        self.evicted: list = []

    def _touch(self, key) -> None:
        self.order.pop(key, None)
        self.order[key] = None

    def ensure(self, layer: int, ids) -> None:
        for e in ids:
            key = (layer, int(e))
            if key not in self.order:
                need = self.used + self.sizes[key] - self.budget
                if need > 0:
                    freed = 0
                    for k in list(self.order):
                        if freed >= need:
                            break
                        if self.pins.get(k, 0) > 0:
                            continue
                        del self.order[k]
                        self.pins.pop(k, None)
                        self.used -= self.sizes[k]
                        freed += self.sizes[k]
                        self.evicted.append(k)
                self.order[key] = None
                self.used += self.sizes[key]
                self.misses += 1
            else:
                self.hits += 1
            self.pins[key] = self.pins.get(key, 0) + 1
            self._touch(key)

    def release(self, layer: int, ids) -> None:
        for e in ids:
            key = (layer, int(e))
            assert self.pins.get(key, 0) > 0
            self.pins[key] -= 1
            self._touch(key)

    def resident(self) -> set:
        return set(self.order)
