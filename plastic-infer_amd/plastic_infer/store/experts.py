"""Expert residency: host bank of every expert + HBM slot pool of the routed subset.

Contract of the reference (src/plastic_infer/store/experts.py:29-223):
  * ExpertBank maps (layer, expert_id) -> ExpertWeights (w1 gate [I, H], w2 down [H, I],
    w3 up [I, H]); duplicate add raises AssertionError.
  * ExpertSlotPool(bank, budget_bytes, device) keeps a byte-budgeted LRU of experts in HBM.
    ensure(layer, ids) visits ids in order; a miss evicts least-recently-used UNPINNED experts
    until the new one fits, loads it and counts a miss; a hit counts a hit; every visited expert
    is pinned at once, so nothing requested by the same call can be evicted by a later miss.
    release() unpins (double release raises). A hit returns the very same tensors.
Data movement: a miss is copied from PINNED host memory by the DMA engines (hipMemcpyAsync
through the HIP library) on the pool's own copy stream. The destination is allocated on that
stream and recorded on the consumer stream, and the consumer stream waits on one event per
ensure() call — so the copies overlap whatever is already queued on the consumer stream, and an
evicted expert's memory is not reused before the work that read it has finished.
"""

from __future__ import annotations

import torch

from .. import _native as N
from ..kernel.index_copy import copy_rows_async
from .resident import LruPool
from .tiers import Tier


class ExpertWeights:
    """Weights of one SwiGLU expert: w1 (gate) [I, H], w2 (down) [H, I], w3 (up) [I, H]."""

    __slots__ = ("w1", "w2", "w3")

    def __init__(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> None:
        self.w1, self.w2, self.w3 = w1, w2, w3

    def tensors(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return (self.w1, self.w2, self.w3)

    def bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors())

    def __repr__(self) -> str:
        return f"ExpertWeights(w1={tuple(self.w1.shape)}, w2={tuple(self.w2.shape)}, " \
               f"w3={tuple(self.w3.shape)}, dtype={self.w1.dtype})"


class ExpertBank:
    """Every expert's weights in host memory, looked up by (layer, expert_id).

    The bank is the source side of expert streaming: the slot pool copies an entry into HBM
    when it is routed to and not resident. Entries are immutable once added (a second add of
    the same key is an error), and each remembers its byte size so budgets need no tensor
    walks. pin_memory() moves every entry into page-locked memory, which the DMA copies need.
    """

    def __init__(self) -> None:
        self._entries: dict[tuple[int, int], tuple[ExpertWeights, int]] = {}
        self._total = 0

    def add(self, layer: int, expert_id: int, weights: ExpertWeights) -> None:
        key = (int(layer), int(expert_id))
        assert key not in self._entries, f"expert {key} is already in the bank"
        size = weights.bytes()
        self._entries[key] = (weights, size)
        self._total += size

    def __contains__(self, key: tuple[int, int]) -> bool:
        return key in self._entries

    def __getitem__(self, key: tuple[int, int]) -> ExpertWeights:
        return self._entries[key][0]

    def __len__(self) -> int:
        return len(self._entries)

    def bytes(self, key: tuple[int, int]) -> int:
        return self._entries[key][1]

    def keys(self):
        return self._entries.keys()

    @property
    def total_bytes(self) -> int:
        return self._total

    def pin_memory(self) -> None:
        """Re-home every entry in contiguous page-locked host memory (the DMA copy source)."""
        for key, (w, size) in list(self._entries.items()):
            if all(t.device.type == "cpu" and t.is_pinned() and t.is_contiguous()
                   for t in w.tensors()):
                continue
            pinned = ExpertWeights(*(t.detach().to("cpu").contiguous().pin_memory()
                                     for t in w.tensors()))
            self._entries[key] = (pinned, size)


class ExpertSlotPool:
    """HBM LRU cache of the routed expert subset, budgeted in bytes."""

    def __init__(self, bank: ExpertBank, budget_bytes: int,
                 device: torch.device | None = None) -> None:
        if len(bank) > 0:
            assert budget_bytes >= max(bank.bytes(k) for k in bank.keys()), \
                "slot budget smaller than a single expert"
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        if self.device.type != "cuda" or torch.version.hip is None:
            raise ValueError(f"expert slots live in HBM: device must be a HIP device, "
                             f"got {self.device}")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        N.load()
        self.bank = bank
        self.bank.pin_memory()
        self.pool: LruPool[tuple[int, int]] = LruPool(budget_bytes)
        self._tensors: dict[tuple[int, int], ExpertWeights] = {}
        self.hits = 0
        self.misses = 0
        self.bytes_loaded = 0
        self.copy_stream = torch.cuda.Stream(device=self.device)

    def ensure(self, layer: int, expert_ids) -> dict[int, ExpertWeights]:
        """Make the experts of `layer` resident and pinned; returns {expert_id: weights}.
        Call release(layer, expert_ids) after the compute that reads them is enqueued."""
        eids = [int(e) for e in expert_ids]
        consumer = torch.cuda.current_stream(self.device)
        loaded = False
        for e in eids:
            key = (layer, e)
            if key not in self.pool:
                for page in self.pool.evict_to_fit(self.bank.bytes(key)):
                    del self._tensors[page.key]
                self.pool.add(key, self.bank.bytes(key), tier=Tier.GPU)
                self._tensors[key] = self._load(key, consumer)
                self.misses += 1
                loaded = True
            else:
                self.hits += 1
            self.pool.pin(key)
        if loaded:
            done = torch.cuda.Event()
            done.record(self.copy_stream)
            consumer.wait_event(done)
        return {e: self._tensors[(layer, e)] for e in eids}

    def release(self, layer: int, expert_ids) -> None:
        for e in expert_ids:
            self.pool.unpin((layer, int(e)))

    @property
    def hit_rate(self) -> float:
        total = self.hits + self.misses
        return self.hits / total if total else 0.0

    def _load(self, key: tuple[int, int], consumer: torch.cuda.Stream) -> ExpertWeights:
        src = self.bank[key]
        out = []
        with torch.cuda.stream(self.copy_stream):
            for t in src.tensors():
                dst = torch.empty(t.shape, dtype=t.dtype, device=self.device)
                copy_rows_async(dst.view(1, -1), [0], t.view(1, -1), [0], stream=self.copy_stream)
                dst.record_stream(consumer)
                out.append(dst)
        self.bytes_loaded += src.bytes()
        return ExpertWeights(*out)
