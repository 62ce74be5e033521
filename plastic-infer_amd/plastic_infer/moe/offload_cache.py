"""HBM slot cache of MoE expert weights over pinned host banks.

Drop-in for the reference's OffloadMoeCache (src/plastic_infer/moe/offload_cache.py; decode
admission :347-408 and copy_missing :973-1024, prefill double buffer :568-803) on this
package's HIP kernels and the DMA engines. Every layer's experts live in pinned host banks
(one [num_experts, ...] tensor per layer and bank: "gate_up" [E, 2I, H], "down" [E, H, I]);
the cache holds `cache_size` expert rows per bank in HBM.

Residency policies
------------------
"lru"     One least-recently-used cache over all slots and every layer's experts: the
          reference's policy. ensure_experts runs the HIP admission kernel, which rewrites the
          routed ids to slot ids and leaves a device copy plan; copy_missing executes the plan
          with one multi-bank index-copy launch whose CUs read the pinned banks through their
          device mapping. No host synchronisation, so the chain can be graph-captured.
"static"  `resident_per_layer` chosen experts of every layer stay in the first slots for
          good (filled once by set_bank_sources); the remaining slots are a staging area under
          a host LRU with the same victim rule as the device kernel. A decode layer's misses are
          planned on the host (its routing is read back, 4 bytes per route) and copied by the
          DMA engines (hipMemcpyAsync) on the cache's copy stream.

For overlap, stage_layer(layer, topk_ids) serves either policy: it returns the routes split
into those whose expert is already in HBM and those being copied, plus the event that marks
the copies done. The routed FFN runs the first group on the compute stream while the copies
are in flight, waits on the event, then runs the second (exec.runner_moe_paged does this).
Under "lru" the device plan of the admission kernel is read back and turned into DMA runs.

Prefill
-------
Two whole-layer buffers (slots [b, b + 2E), b = 0 under "lru", the staging area's start under
"static") filled on the copy stream under ready / release events, so layer l + 1's experts
cross the host link while layer l computes. Experts already in HBM (prefill_hit_d2d under
"lru"; the resident set under "static") are gathered device-side instead.

Only bf16 / fp16 expert banks (the "bf16" schema) and decode on the GPU are built here.
"""

from __future__ import annotations

import math
import warnings
from dataclasses import dataclass

import numpy as np
import torch

from .. import _native as N
from ..kernel.index_copy import copy_rows_async, device_ptr, fast_index_copy_multi
from ..kernel.lru_ensure import N_STATS, Stat, lru_ensure

BANK_NAMES = ("gate_up", "down")
PINNED = "pinned"
POLICIES = ("lru", "static")

# Banks whose rows are smaller than this are copied as a whole layer during prefill (and
# kept out of the device-side gather), so every DMA transfer stays large.
_SMALL_ROW_BYTES = 256 * 1024


# ---------------------------------------------------------------------------------------------
# Device maps: what every HIP slot-cache kernel reads and writes
# ---------------------------------------------------------------------------------------------

class _DeviceSlotMaps:
    """slot_of_id [L, E] (flat ids layer * E + expert), id_of_slot [S], usage [S] and the clock,
    plus the copy plan of the last admission (dst slots, src rows, count) and per-layer stats."""

    def __init__(self, num_layers: int, num_experts: int, num_slots: int, dev: torch.device):
        self.L, self.E, self.S = num_layers, num_experts, num_slots
        self.slot_of_id = torch.full((num_layers, num_experts), -1, dtype=torch.int32, device=dev)
        self.id_of_slot = torch.full((num_slots,), -1, dtype=torch.int32, device=dev)
        self.usage = torch.zeros(num_slots, dtype=torch.int64, device=dev)
        self.clock = torch.zeros((), dtype=torch.int64, device=dev)
        plan = max(num_experts, num_slots)
        self.plan_dst = torch.zeros(plan, dtype=torch.int32, device=dev)
        self.plan_src = torch.zeros(plan, dtype=torch.int32, device=dev)
        self.plan_len = torch.zeros(1, dtype=torch.int64, device=dev)
        self.stats = torch.zeros((num_layers, N_STATS), dtype=torch.int64, device=dev)

    def _stream(self) -> int:
        return N.stream_of(self.slot_of_id.device)

    def admit(self, layer: int, ids: torch.Tensor, with_stats: bool) -> None:
        """LRU admission of `ids` (layer-local expert ids, int32, rewritten to slots in place)."""
        lru_ensure(ids, self.slot_of_id.view(-1), self.id_of_slot, self.usage, self.clock, ids,
                   self.plan_src, self.plan_dst, self.plan_len,
                   stats=self.stats[layer] if with_stats else None, id_base=layer * self.E)

    def materialize(self, layer: int) -> None:
        """Slots [0, E) take the layer's experts in id order; the plan copies the whole layer."""
        N.call("pia_slot_cache_materialize", self.slot_of_id.data_ptr(), self.L * self.E,
               self.id_of_slot.data_ptr(), self.usage.data_ptr(), self.S, self.clock.data_ptr(),
               self.plan_dst.data_ptr(), self.plan_src.data_ptr(), self.plan_len.data_ptr(),
               int(layer), self.E, self._stream())

    def reset(self) -> None:
        N.call("pia_slot_cache_reset", self.slot_of_id.data_ptr(), self.L * self.E,
               self.id_of_slot.data_ptr(), self.usage.data_ptr(), self.S, self.clock.data_ptr(),
               None, 0, self.plan_len.data_ptr(), self._stream())

    def invalidate(self, lo: int, hi: int) -> None:
        """Slots [lo, hi) emptied: owners unmapped, usage 0 (first to be reused)."""
        N.call("pia_slot_cache_invalidate", self.slot_of_id.data_ptr(), self.L * self.E,
               self.id_of_slot.data_ptr(), self.usage.data_ptr(), self.S, int(lo), int(hi),
               self._stream())


# ---------------------------------------------------------------------------------------------
# Banks: pinned host sources, HBM slot tensors, copy descriptors
# ---------------------------------------------------------------------------------------------

class _BankSet:
    """One HBM tensor [num_slots, ...] per bank over per-layer pinned host banks [E, ...].

    Rows move three ways: by the multi-bank index-copy kernel from a device plan (the CUs read
    pinned memory through its device mapping), by DMA runs (hipMemcpyAsync) from a host plan,
    or slot to slot inside HBM (prefill gathers). The multi-bank descriptor needs 16-byte rows
    and bases; without it the kernel copies bank by bank."""

    def __init__(self, sources: dict[str, list[torch.Tensor]], num_layers: int,
                 num_experts: int, num_slots: int, dev: torch.device, multi_bank: bool):
        self.names = tuple(n for n in BANK_NAMES if n in sources)
        if set(self.names) != set(sources):
            raise ValueError(f"expert banks must be {BANK_NAMES}, got {sorted(sources)}")
        self.sources: dict[str, list[torch.Tensor]] = {}
        self.caches: dict[str, torch.Tensor] = {}
        for name in self.names:
            per_layer = list(sources[name])
            if len(per_layer) != num_layers:
                raise ValueError(f"bank {name!r}: {len(per_layer)} layers, expected {num_layers}")
            head = per_layer[0]
            for l, t in enumerate(per_layer):
                if t.device.type != "cpu" or not t.is_pinned():
                    raise ValueError(f"bank {name!r} layer {l} must be pinned host memory")
                if not t.is_contiguous() or t.shape != head.shape or t.dtype != head.dtype:
                    raise ValueError(f"bank {name!r} layer {l}: every layer must be a contiguous "
                                     f"{tuple(head.shape)} {head.dtype} tensor")
                if t.shape[0] != num_experts:
                    raise ValueError(f"bank {name!r} layer {l} has {t.shape[0]} experts, "
                                     f"expected {num_experts}")
            if head.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                raise NotImplementedError("expert banks are built for bf16, fp16 and fp32 "
                                          "storage")
            self.sources[name] = per_layer
            self.caches[name] = torch.empty((num_slots, *head.shape[1:]), dtype=head.dtype,
                                            device=dev)
        self.row_bytes = [math.prod(self.caches[n].shape[1:]) * self.caches[n].element_size()
                          for n in self.names]
        self.multi_ok = False
        if multi_bank and all(b % 16 == 0 for b in self.row_bytes):
            dst = [self.caches[n].data_ptr() for n in self.names]
            src = [[device_ptr(self.sources[n][l]) for n in self.names] for l in range(num_layers)]
            if all(p % 16 == 0 for p in dst) and all(p % 16 == 0 for row in src for p in row):
                self.dst_table = torch.tensor(dst, dtype=torch.int64, device=dev)
                self.src_tables = [torch.tensor(r, dtype=torch.int64, device=dev) for r in src]
                self.row_table = torch.tensor(self.row_bytes, dtype=torch.int64, device=dev)
                big = [i for i, b in enumerate(self.row_bytes) if b >= _SMALL_ROW_BYTES]
                self.big_banks = big
                self.gather_dst = self.dst_table[big].contiguous() if big else None
                self.gather_rows = self.row_table[big].contiguous() if big else None
                self.multi_ok = True

    def views(self, n: int | None = None) -> tuple[torch.Tensor, ...]:
        return tuple(self.caches[name] if n is None else self.caches[name][:n]
                     for name in self.names)

    def copy_planned(self, layer: int, dst: torch.Tensor, src: torch.Tensor,
                     count: torch.Tensor) -> None:
        """Rows src[i] of the layer's host banks -> slots dst[i], i < count (device plan)."""
        if self.multi_ok:
            fast_index_copy_multi(self.dst_table, self.src_tables[layer], self.row_table, dst, src,
                                  count)
            return
        from ..kernel.index_copy import fast_index_copy

        for name in self.names:
            fast_index_copy(self.caches[name], dst, self.sources[name][layer], src, count)

    def copy_dma(self, layer: int, slots: np.ndarray, rows: np.ndarray,
                 stream: torch.cuda.Stream, only_large: bool = False) -> int:
        """hipMemcpyAsync of host rows -> slots for every bank on `stream`; returns bytes."""
        moved = 0
        for i, name in enumerate(self.names):
            if only_large and self.row_bytes[i] < _SMALL_ROW_BYTES:
                continue
            copy_rows_async(self.caches[name], slots, self.sources[name][layer], rows,
                            stream=stream)
            moved += self.row_bytes[i] * len(rows)
        return moved

    def expert_bytes(self) -> int:
        return sum(self.row_bytes)


# ---------------------------------------------------------------------------------------------
# Host LRU of the staging slots ("static" policy)
# ---------------------------------------------------------------------------------------------

class _StagingLru:
    """Least-recently-used map of flat expert ids onto `n` staging slots, decided on the host.

    Same rule as the device admission kernel: each call advances a clock; ids already staged
    are hits and take the current clock; the distinct missing ids, in ascending order, take the
    untouched slots in ascending (last use, slot) order."""

    def __init__(self, n: int):
        self.n = n
        self.owner = np.full(n, -1, np.int64)
        self.last_use = np.zeros(n, np.int64)
        self.slot_of: dict[int, int] = {}
        self.clock = 0

    def place(self, flat_ids: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """flat_ids: distinct ids. Returns (slot of each id, ids copied in, their slots)."""
        self.clock += 1
        slots = np.full(flat_ids.size, -1, np.int64)
        miss = []
        for i, f in enumerate(flat_ids.tolist()):
            s = self.slot_of.get(f)
            if s is None:
                miss.append(i)
            else:
                slots[i] = s
                self.last_use[s] = self.clock
        if not miss:
            return slots, np.empty(0, np.int64), np.empty(0, np.int64)
        if len(miss) > self.n - (flat_ids.size - len(miss)):
            raise RuntimeError(f"{len(miss)} experts to stage but only "
                               f"{self.n - (flat_ids.size - len(miss))} free staging slots")
        key = np.where(self.last_use == self.clock, np.iinfo(np.int64).max, self.last_use)
        victims = np.lexsort((np.arange(self.n), key))[:len(miss)]
        order = np.argsort(flat_ids[miss], kind="stable")
        new_ids = flat_ids[miss][order]
        for f, s in zip(new_ids.tolist(), victims.tolist()):
            old = int(self.owner[s])
            if old >= 0:
                del self.slot_of[old]
            self.owner[s] = f
            self.slot_of[f] = s
            self.last_use[s] = self.clock
        slots[np.asarray(miss)[order]] = victims
        return slots, new_ids, victims.astype(np.int64)

    def forget_range(self, lo: int, hi: int) -> None:
        """Staging slots [lo, hi) emptied (borrowed by the prefill buffers)."""
        for s in range(lo, hi):
            old = int(self.owner[s])
            if old >= 0:
                del self.slot_of[old]
            self.owner[s] = -1
            self.last_use[s] = 0

    def reset(self) -> None:
        self.__init__(self.n)


@dataclass
class StagedRoutes:
    """A decode layer's routes split for an overlapped FFN (ids are slots; -1 = not in group).

    in_hbm:  routes whose expert was in HBM before this call (resident, or an LRU hit);
    copied:  routes whose expert is being copied; run them after the compute stream waits on
             `ready` (recorded on the copy stream after the copies)."""
    layer: int
    in_hbm: torch.Tensor
    copied: torch.Tensor
    ready: torch.cuda.Event
    experts: int          # distinct experts routed to
    copied_experts: int   # distinct experts copied by this call
    copied_bytes: int
    issued: torch.cuda.Event | None = None   # copy stream, before the copies (timing only)


# ---------------------------------------------------------------------------------------------
# Prefill double buffer
# ---------------------------------------------------------------------------------------------

class _PrefillBuffers:
    """Two whole-layer buffers [E, ...] per bank at slots [base, base + 2E) of the caches."""

    def __init__(self, banks: _BankSet, num_experts: int, base: int, dev: torch.device):
        E = num_experts
        self.base = base
        self.views = [banks.caches[n][base:base + 2 * E].view(2, E, *banks.caches[n].shape[1:])
                      for n in banks.names]
        self.stream = torch.cuda.Stream(device=dev)
        self.ready = [torch.cuda.Event() for _ in range(2)]
        self.released = [torch.cuda.Event() for _ in range(2)]
        self.begin = torch.cuda.Event()
        self.layer: list[int | None] = [None, None]
        self.free = [True, True]
        self.ever_released = [False, False]


# ---------------------------------------------------------------------------------------------
# The cache
# ---------------------------------------------------------------------------------------------

class OffloadMoeCache:
    """Expert slot cache in HBM (see the module docstring for the policies)."""

    def __init__(self, num_layers: int, num_experts: int, cache_size: int,
                 device: torch.device | str, cache_policy: str = "lru",
                 prefill_overlap: bool = False, prefill_hit_d2d: bool = False,
                 quant_format: str = "bf16", decode_target: str = "gpu",
                 resident_per_layer: int | None = None, multi_bank_copy: bool = True) -> None:
        if cache_policy not in POLICIES:
            raise ValueError(f"cache_policy must be one of {POLICIES}, got {cache_policy!r}")
        if quant_format != "bf16":
            raise NotImplementedError(f"quant_format {quant_format!r}: only bf16 / fp16 expert "
                                      "banks are built")
        if decode_target != "gpu":
            raise NotImplementedError(f"decode_target {decode_target!r} needs a CPU expert "
                                      "executor, which is not part of this build")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("OffloadMoeCache lives on the HIP device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.num_layers, self.num_experts = int(num_layers), int(num_experts)
        self.cache_policy = cache_policy
        self.prefill_overlap = bool(prefill_overlap)
        self.prefill_hit_d2d = bool(prefill_hit_d2d)
        self.multi_bank_copy = bool(multi_bank_copy)
        self.quant_format = quant_format
        self.decode_target = decode_target
        L, E = self.num_layers, self.num_experts
        if cache_policy == "static":
            R = E // 2 if resident_per_layer is None else int(resident_per_layer)
            if not 0 <= R <= E:
                raise ValueError(f"resident_per_layer must be in [0, {E}]")
            self.resident_per_layer = R
        else:
            self.resident_per_layer = 0
        self.validate_rebuild(int(cache_size))
        if self.prefill_overlap and not self._overlap_fits(int(cache_size)):
            raise ValueError("prefill overlap borrows two whole-layer buffers from the cache: "
                             f"cache_size {cache_size} leaves fewer than 2 * num_experts "
                             "borrowable slots")
        self.cache_size = int(cache_size)
        self._banks: _BankSet | None = None
        self._prefill: _PrefillBuffers | None = None
        self._resident_slot = np.full((L, E), -1, np.int64)   # "static": fixed slot or -1
        self._resident_choice: list[list[int]] | None = None
        self._pending_layer: int | None = None
        self._copy_stream = torch.cuda.Stream(device=self.device)
        self._host_ids = torch.empty(0, dtype=torch.int32, pin_memory=True)
        self.collect_stats = False
        self.record_copy_start = False      # StagedRoutes.issued (overlap measurement)
        # Opt-in routing histogram [L, E] (raw expert ids counted before they become slots):
        # decode_routing_stats() reads it.
        self.collect_decode_freq = False
        self.decode_freq = torch.zeros((L, E), dtype=torch.int64, device=self.device)
        # prefill_hit_compact (moe.offload_kernels) output: buffer rows, cache slots, count
        self._prefill_hit_dst = torch.zeros(E, dtype=torch.int32, device=self.device)
        self._prefill_hit_src = torch.zeros(E, dtype=torch.int32, device=self.device)
        self._prefill_hit_num = torch.zeros(1, dtype=torch.int64, device=self.device)
        self._set_geometry()

    def _set_geometry(self) -> None:
        """cache_size-shaped state: staging split, device maps and plan, host plan buffer,
        stats (all cold)."""
        L, E, S = self.num_layers, self.num_experts, self.cache_size
        if self.cache_policy == "static":
            self.staging_base = L * self.resident_per_layer
            self._staging = _StagingLru(S - self.staging_base)
        else:
            self.staging_base = 0
            self._staging = None
        self._maps = _DeviceSlotMaps(L, E, S, self.device)
        self._host_plan = torch.empty(3 * max(E, S) + 2, dtype=torch.int64, pin_memory=True)
        self._host_stats = np.zeros((L, N_STATS), np.int64)   # "static" and staged calls
        self.copied_bytes = 0
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0

    def validate_rebuild(self, cache_size: int) -> None:
        """Geometry check of a cache size, with no side effect (reference :410-423): at least
        num_experts slots; under "static" also the resident experts of every layer plus a
        staging area for one layer's other experts. rebuild() and the constructor call it, so an
        invalid size is rejected with the current cache intact."""
        L, E = self.num_layers, self.num_experts
        if cache_size < E:
            raise ValueError(f"cache_size {cache_size} < num_experts {E}")
        if self.cache_policy == "static":
            staging = cache_size - L * self.resident_per_layer
            if staging < E - self.resident_per_layer:
                raise ValueError(f"cache_size {cache_size}: {L} x {self.resident_per_layer} "
                                 f"resident slots leave {staging} staging slots, "
                                 f"{E - self.resident_per_layer} needed")

    def _overlap_fits(self, cache_size: int) -> bool:
        """Whether the two whole-layer prefill buffers fit in the slots that may be borrowed."""
        free = cache_size - (self.num_layers * self.resident_per_layer
                             if self.cache_policy == "static" else 0)
        return free >= 2 * self.num_experts

    # ---- state views (the reference's attribute names) ----------------------------------------

    @property
    def slot_for_id(self) -> torch.Tensor:
        return self._maps.slot_of_id

    @property
    def id_of_slot(self) -> torch.Tensor:
        return self._maps.id_of_slot

    @property
    def step(self) -> torch.Tensor:
        return self._maps.clock

    @property
    def usage(self) -> torch.Tensor:
        """[cache_size] int64: clock value at each slot's last use."""
        return self._maps.usage

    @property
    def evict_slots(self) -> torch.Tensor:
        """Copy plan of the last admission: destination slots (first num_indices entries)."""
        return self._maps.plan_dst

    @property
    def src_indices(self) -> torch.Tensor:
        """Copy plan of the last admission: layer-local host bank rows."""
        return self._maps.plan_src

    @property
    def num_indices(self) -> torch.Tensor:
        """[1] int64: entries in the copy plan of the last admission."""
        return self._maps.plan_len

    @property
    def lru_stats(self) -> torch.Tensor:
        """[L, 3] int64: distinct experts routed, experts copied in, calls (cumulative)."""
        if self.cache_policy == "static":
            return torch.from_numpy(self._host_stats.copy())
        return self._maps.stats + torch.from_numpy(self._host_stats).to(self.device)

    @property
    def bank_caches(self) -> dict[str, torch.Tensor]:
        assert self._banks is not None, "set_bank_sources first"
        return self._banks.caches

    @property
    def copy_stream(self) -> torch.cuda.Stream:
        return self._copy_stream

    def bank_views(self, n: int | None = None) -> tuple[torch.Tensor, ...]:
        """The slot caches (decode ids are slots), or their first n slots."""
        assert self._banks is not None, "set_bank_sources first"
        return self._banks.views(n)

    def resident_experts(self, layer: int) -> np.ndarray:
        """Experts of `layer` that stay in HBM ("static"; empty under "lru")."""
        return np.nonzero(self._resident_slot[layer] >= 0)[0]

    # ---- banks ---------------------------------------------------------------------------------

    def set_bank_sources(self, sources: dict[str, list[torch.Tensor]],
                         layer_residency: list[str] | None = None,
                         resident_experts: list[list[int]] | None = None) -> None:
        """Attach the pinned per-layer host banks and allocate the HBM slot caches.

        "static": resident_experts[l] lists the experts of layer l to keep in HBM (default the
        first resident_per_layer ids); they are copied in now, on the copy stream, and the
        call returns when they have landed."""
        if layer_residency is not None and any(str(getattr(r, "value", r)) != PINNED
                                               for r in layer_residency):
            raise NotImplementedError("every layer's banks must be pinned (LOCKED / PAGEABLE "
                                      "layers decode on a CPU executor, not part of this build)")
        self._banks = _BankSet(sources, self.num_layers, self.num_experts, self.cache_size,
                               self.device, self.multi_bank_copy)
        if self.cache_policy == "static":
            self._place_resident(resident_experts)
        if self.prefill_overlap:
            self._prefill = _PrefillBuffers(self._banks, self.num_experts, self.staging_base,
                                            self.device)

    def _place_resident(self, resident_experts) -> None:
        L, E, R = self.num_layers, self.num_experts, self.resident_per_layer
        self._resident_choice = resident_experts
        self._resident_slot.fill(-1)
        for l in range(L):
            chosen = np.arange(R) if resident_experts is None else \
                np.unique(np.asarray(resident_experts[l], np.int64))
            if chosen.size != R or (chosen.size and (chosen.min() < 0 or chosen.max() >= E)):
                raise ValueError(f"layer {l}: resident_experts must list {R} distinct ids < {E}")
            self._resident_slot[l, chosen] = l * R + np.arange(R)
        # device maps mirror the resident set (slot_for_id is the public residency view)
        flat = torch.from_numpy(self._resident_slot.astype(np.int32)).to(self.device)
        self._maps.slot_of_id.copy_(flat)
        owners = np.full(self.cache_size, -1, np.int32)
        ls, es = np.nonzero(self._resident_slot >= 0)
        owners[self._resident_slot[ls, es]] = (ls * E + es).astype(np.int32)
        self._maps.id_of_slot.copy_(torch.from_numpy(owners).to(self.device))
        with torch.cuda.stream(self._copy_stream):
            self._copy_stream.wait_stream(torch.cuda.current_stream(self.device))
            for l in range(L):
                rows = np.nonzero(self._resident_slot[l] >= 0)[0]
                if rows.size:
                    self._banks.copy_dma(l, self._resident_slot[l, rows], rows,
                                         self._copy_stream)
        self._copy_stream.synchronize()

    # ---- decode: the reference's in-place path --------------------------------------------------

    def ensure_experts(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        """Make this layer's routed experts (int32 ids) resident and rewrite them to slot ids
        in place. "lru": device admission (no host sync); copy_missing() moves the rows.
        "static": staged through stage_layer; the current stream waits for the copies, so
        copy_missing() has nothing left to do."""
        if expert_ids.dtype != torch.int32 or not expert_ids.is_contiguous():
            raise ValueError("expert_ids must be a contiguous int32 tensor")
        if self.cache_policy == "lru":
            self._count_routes(int(layer_id), expert_ids)
            self._pending_layer = int(layer_id)
            self._maps.admit(int(layer_id), expert_ids.view(-1), self.collect_stats)
            return
        routes = self.stage_layer(layer_id, expert_ids)
        torch.cuda.current_stream(self.device).wait_event(routes.ready)
        expert_ids.copy_(torch.maximum(routes.in_hbm, routes.copied).view(expert_ids.shape))
        self._pending_layer = None

    def copy_missing(self) -> None:
        """Execute the copy plan of the last ensure_experts / materialize_layer ("lru")."""
        assert self._banks is not None, "set_bank_sources first"
        if self.cache_policy == "static":
            return
        layer = self._pending_layer
        assert layer is not None, "no pending plan (ensure_experts / materialize_layer first)"
        self._banks.copy_planned(layer, self._maps.plan_dst, self._maps.plan_src,
                                 self._maps.plan_len)

    def materialize_layer(self, layer_id: int) -> None:
        """Slots [0, E) take the layer's experts in id order ("lru"); copy_missing() copies."""
        if self.cache_policy != "lru":
            raise NotImplementedError("materialize_layer belongs to the lru policy")
        self._pending_layer = int(layer_id)
        self._maps.materialize(int(layer_id))

    # ---- decode: staged, overlapped path --------------------------------------------------------

    def stage_layer(self, layer_id: int, topk_ids: torch.Tensor) -> StagedRoutes:
        """Plan the layer's misses on the host and copy them with the DMA engines on the copy
        stream. Reads the routing back, which blocks the host until everything enqueued on the
        compute stream so far has run; so no earlier reader of a slot is still in flight when
        its new rows are copied. Returns the routes split into in-HBM and being-copied groups
        (see StagedRoutes)."""
        assert self._banks is not None, "set_bank_sources first"
        layer = int(layer_id)
        dev, E = self.device, self.num_experts
        ids = topk_ids.contiguous().view(-1)
        if ids.dtype != torch.int32:
            raise ValueError("topk_ids must be int32")
        n = ids.numel()
        self._count_routes(layer, ids)
        compute = torch.cuda.current_stream(dev)
        if self._host_ids.numel() < n:
            self._host_ids = torch.empty(max(n, 2 * self._host_ids.numel()), dtype=torch.int32,
                                         pin_memory=True)
        if self.cache_policy == "lru":
            return self._stage_lru(layer, ids, topk_ids.shape, compute)
        hid = self._host_ids[:n]
        hid.copy_(ids, non_blocking=True)
        done = torch.cuda.Event()
        done.record(compute)
        done.synchronize()
        rid = hid.numpy().astype(np.int64)
        valid = (rid >= 0) & (rid < E)
        distinct = np.unique(rid[valid])
        res = self._resident_slot[layer, distinct]
        stage_ids = distinct[res < 0]
        slot_of_expert = np.full(E, -1, np.int64)
        slot_of_expert[distinct[res >= 0]] = res[res >= 0]
        new_ids = np.empty(0, np.int64)
        victims = np.empty(0, np.int64)
        if stage_ids.size:
            st_slots, new_flat, victims = self._staging.place(layer * E + stage_ids)
            slot_of_expert[stage_ids] = self.staging_base + st_slots
            new_ids = new_flat - layer * E
        copied_mask = np.zeros(E, bool)
        copied_mask[new_ids] = True
        rslot = np.where(valid, slot_of_expert[np.clip(rid, 0, E - 1)], -1)
        rcopied = valid & copied_mask[np.clip(rid, 0, E - 1)]
        in_hbm = np.where(rcopied, -1, rslot).astype(np.int32)
        copied = np.where(rcopied, rslot, -1).astype(np.int32)
        moved = 0
        issued = self._copy_start_event()
        if new_ids.size:
            with torch.cuda.stream(self._copy_stream):
                order = np.argsort(victims)
                moved = self._banks.copy_dma(layer, self.staging_base + victims[order],
                                             new_ids[order], self._copy_stream)
        ready = torch.cuda.Event(enable_timing=self.record_copy_start)
        ready.record(self._copy_stream)
        self._host_stats[layer] += (distinct.size, new_ids.size, 1)
        self.copied_bytes += moved
        return StagedRoutes(layer, self._to_device(in_hbm, topk_ids.shape),
                            self._to_device(copied, topk_ids.shape), ready, int(distinct.size),
                            int(new_ids.size), moved, issued)

    def _stage_lru(self, layer: int, ids: torch.Tensor, shape, compute) -> StagedRoutes:
        """"lru" policy: device admission, then its plan read back and copied by DMA."""
        slots = ids.clone()
        self._maps.admit(layer, slots, self.collect_stats)
        n = ids.numel()
        hp = self._host_plan
        E, S = self.num_experts, self.cache_size
        plan = min(n, S)
        buf = torch.cat([self._maps.plan_len, self._maps.plan_dst[:plan].long(),
                         self._maps.plan_src[:plan].long()])
        hp[:buf.numel()].copy_(buf, non_blocking=True)
        hid = self._host_ids[:n]
        hid.copy_(slots, non_blocking=True)
        done = torch.cuda.Event()
        done.record(compute)
        done.synchronize()
        cnt = int(hp[0])
        dst = hp[1:1 + cnt].numpy().copy()
        src = hp[1 + plan:1 + plan + cnt].numpy().copy()
        new_slot = np.zeros(S, bool)
        new_slot[dst] = True
        hs = hid.numpy().astype(np.int64)
        fresh = (hs >= 0) & new_slot[np.clip(hs, 0, S - 1)]
        in_hbm = np.where(fresh, -1, hs).astype(np.int32)
        copied = np.where(fresh, hs, -1).astype(np.int32)
        moved = 0
        issued = self._copy_start_event()
        if cnt:
            with torch.cuda.stream(self._copy_stream):
                order = np.argsort(dst)
                moved = self._banks.copy_dma(layer, dst[order], src[order], self._copy_stream)
        ready = torch.cuda.Event(enable_timing=self.record_copy_start)
        ready.record(self._copy_stream)
        self.copied_bytes += moved
        return StagedRoutes(layer, self._to_device(in_hbm, shape), self._to_device(copied, shape),
                            ready, int(np.unique(hs[hs >= 0]).size), cnt, moved, issued)

    def _count_routes(self, layer: int, ids: torch.Tensor) -> None:
        """decode_freq[layer][e] += routes to expert e (ids outside [0, E) are not counted),
        when collect_decode_freq is set; on the current stream, no host synchronisation."""
        if not self.collect_decode_freq:
            return
        E = self.num_experts
        flat = ids.reshape(-1)
        valid = (flat >= 0) & (flat < E)
        self.decode_freq[layer].index_add_(0, flat.clamp(0, E - 1).long(), valid.long())

    def _copy_start_event(self) -> torch.cuda.Event | None:
        if not self.record_copy_start:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(self._copy_stream)
        return ev

    def _to_device(self, a: np.ndarray, shape) -> torch.Tensor:
        return torch.from_numpy(a).to(self.device).view(shape)

    # ---- prefill double buffer ------------------------------------------------------------------

    def begin_prefill(self) -> None:
        """Start a prefill: its buffer copies queue behind everything on the compute stream."""
        pb = self._prefill
        if pb is None:
            return
        pb.layer = [None, None]
        pb.free = [True, True]
        pb.begin.record(torch.cuda.current_stream(self.device))
        pb.stream.wait_event(pb.begin)
        self._snapshot = None
        if self.cache_policy == "lru" and self.prefill_hit_d2d and self._banks.multi_ok \
                and self.cache_size > 2 * self.num_experts:
            snap = torch.empty((self.num_layers, self.num_experts), dtype=torch.int32,
                               pin_memory=True)
            with torch.cuda.stream(pb.stream):
                snap.copy_(self._maps.slot_of_id, non_blocking=True)
            pb.stream.synchronize()
            self._snapshot = snap.numpy()

    def _empty_buffer_slots(self, buf: int) -> None:
        E = self.num_experts
        lo = self._prefill.base + buf * E
        if self.cache_policy == "lru":
            self._maps.invalidate(lo, lo + E)
        else:
            self._staging.forget_range(lo - self.staging_base, lo - self.staging_base + E)

    def prefetch_prefill_layer(self, layer_id: int) -> None:
        """Queue the copy of a whole layer into buffer layer_id % 2 (no-op when queued)."""
        pb = self._prefill
        if pb is None or layer_id >= self.num_layers:
            return
        if layer_id < 0:
            raise ValueError(f"invalid prefill layer {layer_id}")
        buf, E = layer_id % 2, self.num_experts
        if pb.layer[buf] == layer_id:
            return
        if pb.layer[buf] is not None and not pb.free[buf]:
            raise RuntimeError("prefill buffer reused before release_prefill_layer")
        # experts already in HBM are gathered slot -> buffer row on the compute stream
        in_hbm = np.empty(0, np.int64)
        hbm_slot = np.empty(0, np.int64)
        if self.cache_policy == "static":
            rs = self._resident_slot[layer_id]
            in_hbm = np.nonzero(rs >= 0)[0]
            hbm_slot = rs[in_hbm]
        elif self._snapshot is not None:
            row = self._snapshot[layer_id].astype(np.int64)
            in_hbm = np.nonzero(row >= 2 * E)[0]
            hbm_slot = row[in_hbm]
        if self.prefill_hit_d2d or self.cache_policy == "static":
            self.prefill_hit_rows += int(in_hbm.size)
            self.prefill_total_rows += E
        if in_hbm.size and self._banks.multi_ok and self._banks.gather_dst is not None:
            dst = torch.from_numpy((pb.base + buf * E + in_hbm).astype(np.int32)).to(self.device)
            src = torch.from_numpy(hbm_slot.astype(np.int32)).to(self.device)
            fast_index_copy_multi(self._banks.gather_dst, self._banks.gather_dst,
                                  self._banks.gather_rows, dst, src)
            gathered = True
        else:
            gathered = False
        if not gathered:
            in_hbm = np.empty(0, np.int64)
        rest = np.setdiff1d(np.arange(E), in_hbm)
        with torch.cuda.stream(pb.stream):
            if pb.ever_released[buf]:
                pb.stream.wait_event(pb.released[buf])
            self._empty_buffer_slots(buf)
            base = pb.base + buf * E
            if gathered:     # large banks: only the rest; small banks: the whole layer
                all_rows = np.arange(E)
                for i, name in enumerate(self._banks.names):
                    rows = rest if self._banks.row_bytes[i] >= _SMALL_ROW_BYTES else all_rows
                    if rows.size:
                        copy_rows_async(self._banks.caches[name], base + rows,
                                        self._banks.sources[name][layer_id], rows, stream=pb.stream)
            else:
                self._banks.copy_dma(layer_id, base + rest, rest, pb.stream)
            pb.ready[buf].record(pb.stream)
        pb.layer[buf] = layer_id
        pb.free[buf] = False

    def wait_prefill_layer(self, layer_id: int) -> tuple[torch.Tensor, ...]:
        """[E, ...] views of every bank for layer_id, ordered after its copies."""
        pb = self._prefill
        assert pb is not None, "prefill_overlap is off"
        self.prefetch_prefill_layer(layer_id)
        buf = layer_id % 2
        torch.cuda.current_stream(self.device).wait_event(pb.ready[buf])
        return tuple(v[buf] for v in pb.views)

    def release_prefill_layer(self, layer_id: int) -> None:
        """The layer's consumers are enqueued: its buffer may be refilled after them."""
        pb = self._prefill
        if pb is None:
            return
        buf = layer_id % 2
        if pb.layer[buf] != layer_id:
            return
        pb.released[buf].record(torch.cuda.current_stream(self.device))
        pb.ever_released[buf] = True
        pb.free[buf] = True

    # ---- lifecycle and stats --------------------------------------------------------------------

    def reset(self) -> None:
        """Forget every cached expert ("static": the resident set stays)."""
        if self.cache_policy == "lru":
            self._maps.reset()
        else:
            self._staging.reset()
            self._maps.clock.zero_()
        self._pending_layer = None

    def rebuild(self, cache_size: int) -> None:
        """Resize the HBM slot cache to `cache_size` slots in place (reference :425-496).

        The pinned host banks are kept and nothing is read again from the caller; the old slot
        caches and prefill buffers (views of them) are dropped before the new ones are
        allocated, the maps, plan and statistics restart cold, and under "static" the resident
        experts (the same choice as before) are copied into their new slots before the call
        returns. Prefill overlap is switched off when the new size leaves fewer than
        2 * num_experts borrowable slots. The object stays the same, so holders of the cache
        stay valid; tensors taken from it earlier (bank_views, the maps) do not."""
        assert self._banks is not None, "set_bank_sources must run before rebuild"
        self.validate_rebuild(int(cache_size))
        sources = self._banks.sources
        self._prefill = None
        self._banks = None
        self._maps = None
        self._pending_layer = None
        torch.cuda.synchronize(self.device)
        torch.cuda.empty_cache()
        self.cache_size = int(cache_size)
        self._set_geometry()
        self.decode_freq.zero_()
        if self.prefill_overlap and not self._overlap_fits(self.cache_size):
            warnings.warn(f"prefill overlap switched off by rebuild: cache_size "
                          f"{self.cache_size} leaves fewer than 2 * num_experts borrowable "
                          "slots", RuntimeWarning, stacklevel=2)
            self.prefill_overlap = False
        self._banks = _BankSet(sources, self.num_layers, self.num_experts, self.cache_size,
                               self.device, self.multi_bank_copy)
        if self.cache_policy == "static":
            self._place_resident(self._resident_choice)
        if self.prefill_overlap:
            self._prefill = _PrefillBuffers(self._banks, self.num_experts, self.staging_base,
                                            self.device)

    def reset_stats(self) -> None:
        self._maps.stats.zero_()
        self._host_stats[:] = 0
        self.copied_bytes = 0
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0

    def decode_miss_stats(self) -> dict:
        active, missing, calls = (int(x) for x in self.lru_stats.sum(0))
        return {
            "layer_calls": calls,
            "active_per_layer": active / calls if calls else 0.0,
            "missing_per_layer": missing / calls if calls else 0.0,
            "miss_rate": missing / active if active else 0.0,
            "hit_rate": 1.0 - missing / active if active else 0.0,
            "copied_bytes": self.copied_bytes,
            "prefill_hit_rows": self.prefill_hit_rows,
            "prefill_rows": self.prefill_total_rows,
        }

    def decode_miss_stats_per_layer(self) -> dict:
        st = self.lru_stats.cpu().numpy()
        rows = []
        for l in range(self.num_layers):
            a, m, c = (int(v) for v in st[l, [Stat.ACTIVE, Stat.MISS, Stat.CALLS]])
            rows.append({"layer": l, "steps": c, "active_per_step": a / c if c else 0.0,
                         "missing_per_step": m / c if c else 0.0,
                         "miss_rate": m / a if a else 0.0})
        return {"per_layer": rows}

    def record_decode_stats(self, layer_id: int) -> None:
        """No-op: the admission accumulates lru_stats itself (reference :874-880)."""

    def decode_routing_stats(self) -> dict:
        """Routing concentration per layer from the decode_freq histogram (collect_decode_freq),
        averaged over the layers that saw routes (reference :941-971): the mean and largest
        working set (experts routed to at least once), the experts that cover 90 % of the
        routes, the entropy of the routing normalised by log(num_experts), and the hit rate
        of an oracle that keeps each layer's cache_size / num_layers most routed experts.
        Empty when nothing was counted."""
        freq = self.decode_freq.double().cpu()
        total = freq.sum(dim=1)
        valid = total > 0
        if not bool(valid.any()):
            return {}
        per_layer = self.cache_size / self.num_layers
        keep = max(1, int(round(per_layer)))
        ranked = torch.sort(freq, dim=1, descending=True).values
        f, t, r = freq[valid], total[valid], ranked[valid]
        working = (f > 0).sum(dim=1).double()
        share = torch.cumsum(r, dim=1) / t.unsqueeze(1)
        cover90 = (share < 0.9).sum(dim=1).double() + 1
        p = f / t.unsqueeze(1)
        entropy = -(p * torch.log(p.clamp(min=1e-12))).sum(dim=1)
        return {
            "slots_per_layer": per_layer,
            "working_set_mean": working.mean().item(),
            "working_set_max": int(working.max().item()),
            "experts_for_90pct": cover90.mean().item(),
            "oracle_hit_at_slots": (r[:, :keep].sum(dim=1) / t).mean().item(),
            "norm_entropy": (entropy / math.log(self.num_experts)).mean().item(),
        }


__all__ = ["OffloadMoeCache", "StagedRoutes", "POLICIES", "BANK_NAMES"]
