"""Unified GPU slot cache of MoE expert weights streamed from pinned host banks
(reference src/plastic_infer/moe/offload_cache.py: OffloadMoeCache).

Decode: ``ensure_experts`` runs the device LRU admission (HIP ``pia_lru_ensure``), rewriting
the routed expert ids to slot ids and writing the copy plan; ``copy_missing`` moves the planned
rows of every bank from the pinned host banks in one multi-bank index-copy launch (the kernel
reads host memory through its device mapping). Neither synchronises with the host.

Prefill overlap: two whole-layer buffers borrowed from the first 2E slots, filled on a side
copy stream with the DMA engines (``copy_rows_async``) under ready / release events, so layer
l+1's experts cross PCIe while layer l computes. With ``prefill_hit_d2d``, experts already
resident above slot 2E are gathered device-side instead and only the misses cross PCIe.

Supported here: decode on the GPU (``decode_target="gpu"``) with every layer's banks pinned.
The reference's CPU-executor modes ("cpu", "hybrid") and LOCKED / PAGEABLE host residency
depend on its CPU expert executor, which is outside this build; they raise
NotImplementedError.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass

import numpy as np
import torch

from ..kernel.index_copy import copy_rows_async
from ..kernel.lru_ensure import N_STATS, Stat

_FUSED_COPY = os.getenv("FREETOKEN_FUSED_COPY", "1").strip().lower() not in {"0", "false", "no", "off"}

# Banks whose rows are smaller than this are prefetched as one whole-layer copy (and left out
# of the prefill hit gather), as in the reference, so every per-run copy stays large.
_SMALL_BANK_FEAT_BYTES = 256 * 1024

# quant_format -> bank names in registration order (reference offload_cache.py:34-85); the
# cache machinery is layout-agnostic and only moves rows.
_BANK_SCHEMAS: dict[str, tuple[str, ...]] = {
    "bf16": ("gate_up", "down"),
    "fp8_block": ("gate_up", "gate_up_scale", "down", "down_scale"),
    "q4_0": ("gate_up", "down"),
    "nvfp4": ("gate_up_packed", "gate_up_scale", "gate_up_global",
              "down_packed", "down_scale", "down_global"),
    "nvfp4_marlin": ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"),
    "nvfp4_b12x": ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"),
    "mxfp4_triton": ("gate_up_blocks", "gate_up_scales", "gate_up_bias",
                     "down_blocks", "down_scales", "down_bias"),
    "ds_fp4": ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"),
}

MARLIN_MAX_CACHE_SIZE = 992
PINNED = "pinned"


@dataclass
class OffloadMoeCache:
    num_layers: int
    num_experts: int
    cache_size: int
    device: torch.device
    cache_policy: str = "lru"
    prefill_overlap: bool = False
    prefill_hit_d2d: bool = False
    quant_format: str = "bf16"
    decode_target: str = "gpu"
    hybrid_max_fetch: int = 1
    hybrid_fetch_fraction: float = 0.0

    def __post_init__(self) -> None:
        policy_ids = {"lru": 0}
        assert self.cache_policy in policy_ids
        assert self.decode_target in ("gpu", "cpu", "hybrid"), self.decode_target
        assert self.quant_format in _BANK_SCHEMAS, f"unknown quant_format {self.quant_format!r}"
        if self.decode_target != "gpu":
            raise NotImplementedError(
                f"decode_target={self.decode_target!r} needs the CPU expert executor, which "
                "is not part of this build")
        self.device = torch.device(self.device)
        if self.device.type != "cuda":
            raise ValueError("OffloadMoeCache lives on the HIP device")
        self.cpu_executor = None
        self.cpu_layer_ids: frozenset = frozenset()
        self.validate_rebuild(self.cache_size)
        assert not self.prefill_overlap or self.cache_size >= 2 * self.num_experts, (
            "Prefill overlap borrows two full expert-layer buffers from the unified MoE "
            "cache, so cache_size must be at least 2 * num_experts")
        self.cache_policy_id = policy_ids[self.cache_policy]
        dev = self.device
        self.slot_for_id = torch.full((self.num_layers, self.num_experts), -1, dtype=torch.int32,
                                      device=dev)
        self.id_of_slot = torch.full((self.cache_size,), -1, dtype=torch.int32, device=dev)
        self.usage = torch.zeros((self.cache_size,), dtype=torch.int64, device=dev)
        self.step = torch.zeros((), dtype=torch.int64, device=dev)
        self.active_mask = torch.zeros((self.num_experts,), dtype=torch.int32, device=dev)
        plan_slots = max(self.num_experts, self.cache_size)
        self.evict_slots = torch.empty((plan_slots,), dtype=torch.int32, device=dev)
        self.src_indices = torch.empty((plan_slots,), dtype=torch.int32, device=dev)
        self.num_indices = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.num_missing_full = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.expert_recency = torch.full((self.num_layers, self.num_experts), -1,
                                         dtype=torch.int64, device=dev)
        self.bank_schema = _BANK_SCHEMAS[self.quant_format]
        self.bank_sources: dict[str, list[torch.Tensor]] = {}
        self.bank_caches: dict[str, torch.Tensor] = {}
        self.layer_residency: list[str] = []
        self._unpinned_layers: frozenset = frozenset()
        self.gate_up_alpha: torch.Tensor | None = None
        self.down_alpha: torch.Tensor | None = None
        self.collect_stats = False
        self.lru_stats = torch.zeros((self.num_layers, N_STATS), dtype=torch.int64, device=dev)
        self.stat_missing = torch.zeros((), dtype=torch.int64, device=dev)
        self.stat_active = torch.zeros((), dtype=torch.int64, device=dev)
        self.stat_calls = torch.zeros((), dtype=torch.int64, device=dev)
        self.stat_fetched = torch.zeros((), dtype=torch.int64, device=dev)
        self.stat_missing_layer = torch.zeros(self.num_layers, dtype=torch.int64, device=dev)
        self.stat_active_layer = torch.zeros(self.num_layers, dtype=torch.int64, device=dev)
        self.stat_fetched_layer = torch.zeros(self.num_layers, dtype=torch.int64, device=dev)
        self.stat_steps_layer = torch.zeros(self.num_layers, dtype=torch.int64, device=dev)
        self.collect_decode_freq = False
        self.decode_freq = torch.zeros((self.num_layers, self.num_experts), dtype=torch.int64,
                                       device=dev)
        self.banks: list[tuple[list[torch.Tensor], torch.Tensor]] = []
        self._copy_fused_ok = False
        self._copy_dst_ptrs: torch.Tensor | None = None
        self._copy_src_ptrs: list[torch.Tensor] | None = None
        self._copy_feat_bytes: torch.Tensor | None = None
        self._copy_dst_ptrs_host: list[int] = []
        self._copy_src_ptrs_host: list[list[int]] = []
        self._copy_feat_bytes_host: list[int] = []
        self._gather_bank_ids: list[int] = []
        self._gather_dst_ptrs: torch.Tensor | None = None
        self._gather_feat_bytes: torch.Tensor | None = None
        self._pending_src_layer: int | None = None
        self._pending_whole_layer = False
        self.prefill_bank_buffers: list[torch.Tensor] = []
        self.prefill_copy_stream: torch.cuda.Stream | None = None
        self.prefill_begin_event: torch.cuda.Event | None = None
        self.prefill_ready_events: list[torch.cuda.Event] = []
        self.prefill_release_events: list[torch.cuda.Event] = []
        self._prefill_buffer_layer: list[int | None] = [None, None]
        self._prefill_buffer_released: list[bool] = [True, True]
        self._prefill_buffer_has_release_event: list[bool] = [False, False]
        self._prefill_slot_snapshot: torch.Tensor | None = None
        self._prefill_snapshot_np = None
        self._prefill_hit_d2d_active = False
        self._hit_d2d_fallback_logged = False
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0

    # ---- banks -------------------------------------------------------------------------------

    def set_bank_sources(self, sources: dict[str, list[torch.Tensor]],
                         layer_residency: list[str] | None = None) -> None:
        """Attach the pinned host banks (one ``[num_experts, ...]`` tensor per layer and bank,
        in the format's schema) and allocate one GPU slot cache ``[cache_size, ...]`` per bank."""
        assert set(sources) == set(self.bank_schema), (
            f"banks {sorted(sources)} do not match the {self.quant_format!r} schema "
            f"{self.bank_schema}")
        residency = [str(getattr(r, "value", r)) for r in
                     (layer_residency or [PINNED] * self.num_layers)]
        assert len(residency) == self.num_layers, (len(residency), self.num_layers)
        if any(r != PINNED for r in residency):
            raise NotImplementedError(
                "LOCKED / PAGEABLE host banks decode on the CPU executor, which is not part of "
                "this build; every layer must be pinned")
        self._unpinned_layers = frozenset()
        self.layer_residency = residency
        for name in self.bank_schema:
            per_layer = sources[name]
            assert len(per_layer) == self.num_layers, (name, len(per_layer))
            head = per_layer[0]
            for layer_id, source in enumerate(per_layer):
                assert source.is_contiguous(), f"bank {name!r} layer {layer_id} must be contiguous"
                assert source.size(0) == self.num_experts, (name, layer_id, source.shape)
                assert source.shape == head.shape and source.dtype == head.dtype, (
                    name, layer_id, source.shape, source.dtype)
                if source.device.type != "cpu" or not source.is_pinned():
                    raise ValueError(f"bank {name!r} layer {layer_id} must be pinned host memory")
            self.bank_sources[name] = list(per_layer)
            self.bank_caches[name] = torch.empty((self.cache_size, *head.shape[1:]),
                                                 dtype=head.dtype, device=self.device)
        self.banks = [(self.bank_sources[n], self.bank_caches[n]) for n in self.bank_schema]
        self._build_copy_plan()
        if self.prefill_overlap:
            self._init_prefill_overlap_buffers()

    def _build_copy_plan(self) -> None:
        """Fused multi-bank copy descriptor: per-bank slot-cache base, per-layer host-bank
        device aliases and row bytes, as device int64 tensors (fixed for the cache's
        lifetime). Left disabled when a row size or base is not 16-byte aligned, or with
        FREETOKEN_FUSED_COPY=0; copy_missing then copies bank by bank."""
        self._copy_fused_ok = False
        self._copy_dst_ptrs = None
        self._copy_src_ptrs = None
        self._copy_feat_bytes = None
        self._copy_dst_ptrs_host = []
        self._copy_src_ptrs_host = []
        self._copy_feat_bytes_host = []
        self._gather_bank_ids = []
        self._gather_dst_ptrs = None
        self._gather_feat_bytes = None
        if not _FUSED_COPY or not self.banks:
            return
        from ..kernel.pinned import device_ptr

        dst_ptrs, feats = [], []
        layer_src_ptrs: list[list[int]] = [[] for _ in range(self.num_layers)]
        for per_layer, cache in self.banks:
            feat = math.prod(per_layer[0].shape[1:]) * per_layer[0].element_size()
            if feat % 16 != 0 or cache.data_ptr() % 16 != 0:
                return
            for layer_id, source in enumerate(per_layer):
                src_dev = device_ptr(source)
                if src_dev % 16 != 0:
                    return
                layer_src_ptrs[layer_id].append(src_dev)
            dst_ptrs.append(cache.data_ptr())
            feats.append(feat)
        dev = self.device
        self._copy_dst_ptrs = torch.tensor(dst_ptrs, dtype=torch.int64, device=dev)
        self._copy_src_ptrs = [torch.tensor(p, dtype=torch.int64, device=dev)
                               for p in layer_src_ptrs]
        self._copy_feat_bytes = torch.tensor(feats, dtype=torch.int64, device=dev)
        self._copy_dst_ptrs_host = dst_ptrs
        self._copy_src_ptrs_host = layer_src_ptrs
        self._copy_feat_bytes_host = feats
        self._gather_bank_ids = [i for i, f in enumerate(feats) if f >= _SMALL_BANK_FEAT_BYTES]
        if len(self._gather_bank_ids) == len(feats):
            self._gather_dst_ptrs = self._copy_dst_ptrs
            self._gather_feat_bytes = self._copy_feat_bytes
        elif self._gather_bank_ids:
            self._gather_dst_ptrs = self._copy_dst_ptrs[self._gather_bank_ids].contiguous()
            self._gather_feat_bytes = self._copy_feat_bytes[self._gather_bank_ids].contiguous()
        self._copy_fused_ok = True

    def validate_rebuild(self, cache_size: int) -> None:
        if cache_size < self.num_experts:
            raise ValueError(f"cache_size {cache_size} < num_experts {self.num_experts}")
        if self.quant_format == "nvfp4_marlin" and cache_size > MARLIN_MAX_CACHE_SIZE:
            raise ValueError(f"moe_cache_size={cache_size} exceeds the marlin slot limit of "
                             f"{MARLIN_MAX_CACHE_SIZE}")

    def rebuild(self, cache_size: int) -> None:
        """Resize the slot cache in place (cold start); the host banks are kept."""
        assert self.bank_sources, "set_bank_sources must run before rebuild"
        self.validate_rebuild(cache_size)
        self.prefill_bank_buffers = []
        self.prefill_copy_stream = None
        self.prefill_begin_event = None
        self.prefill_ready_events = []
        self.prefill_release_events = []
        self._prefill_buffer_layer = [None, None]
        self._prefill_buffer_released = [True, True]
        self._prefill_buffer_has_release_event = [False, False]
        self.banks = []
        self.bank_caches = {}
        self.cache_size = cache_size
        torch.cuda.synchronize(self.device)
        torch.cuda.empty_cache()
        for name in self.bank_schema:
            head = self.bank_sources[name][0]
            self.bank_caches[name] = torch.empty((cache_size, *head.shape[1:]), dtype=head.dtype,
                                                 device=self.device)
        self.banks = [(self.bank_sources[n], self.bank_caches[n]) for n in self.bank_schema]
        self._build_copy_plan()
        dev = self.device
        self.slot_for_id.fill_(-1)
        self.id_of_slot = torch.full((cache_size,), -1, dtype=torch.int32, device=dev)
        self.usage = torch.zeros((cache_size,), dtype=torch.int64, device=dev)
        plan_slots = max(self.num_experts, cache_size)
        self.evict_slots = torch.empty((plan_slots,), dtype=torch.int32, device=dev)
        self.src_indices = torch.empty((plan_slots,), dtype=torch.int32, device=dev)
        self.step.zero_()
        self.active_mask.zero_()
        self.num_indices.zero_()
        self.num_missing_full.zero_()
        self.expert_recency.fill_(-1)
        self.lru_stats.zero_()
        for t in (self.stat_missing, self.stat_active, self.stat_calls, self.stat_fetched,
                  self.stat_missing_layer, self.stat_active_layer, self.stat_fetched_layer,
                  self.stat_steps_layer, self.decode_freq):
            t.zero_()
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0
        self._hit_d2d_fallback_logged = False
        if self.prefill_overlap and cache_size < 2 * self.num_experts:
            self.prefill_overlap = False
        if self.prefill_overlap:
            self._init_prefill_overlap_buffers()

    def set_alphas(self, gate_up_alpha: torch.Tensor | None,
                   down_alpha: torch.Tensor | None) -> None:
        """Per-expert global scales ``[L*E]`` kept on the GPU, looked up per slot."""
        if gate_up_alpha is None and down_alpha is None:
            return
        assert gate_up_alpha is not None and down_alpha is not None
        total = self.num_layers * self.num_experts
        assert gate_up_alpha.shape == down_alpha.shape == (total,)
        self.gate_up_alpha = gate_up_alpha.to(self.device)
        self.down_alpha = down_alpha.to(self.device)

    def set_cpu_executor(self, executor) -> None:
        raise NotImplementedError("the CPU expert executor is not part of this build")

    def is_cpu_layer(self, layer_id: int) -> bool:
        return layer_id in self.cpu_layer_ids

    def is_unpinned_layer(self, layer_id: int) -> bool:
        return layer_id in self._unpinned_layers

    def alphas_for_slots(self, layer_id: int):
        if self.gate_up_alpha is None:
            return None
        idx = layer_id * self.num_experts + (self.id_of_slot.clamp(min=0).long() % self.num_experts)
        return self.gate_up_alpha[idx], self.down_alpha[idx]

    def alphas_for_layer(self, layer_id: int):
        if self.gate_up_alpha is None:
            return None
        lo = layer_id * self.num_experts
        return self.gate_up_alpha[lo:lo + self.num_experts], self.down_alpha[lo:lo + self.num_experts]

    def bank_views(self, n: int | None = None) -> tuple[torch.Tensor, ...]:
        """Per-bank slot caches (decode) or their first ``n`` slots (a materialized layer)."""
        assert self.banks, "set_bank_sources must register the banks first"
        if n is None:
            return tuple(cache for _, cache in self.banks)
        return tuple(cache[:n] for _, cache in self.banks)

    # ---- prefill double buffer ---------------------------------------------------------------

    def _init_prefill_overlap_buffers(self) -> None:
        assert self.banks, "set_bank_sources must register the banks first"
        E = self.num_experts
        self._prefill_buffer_layer = [None, None]
        self._prefill_buffer_released = [True, True]
        self._prefill_buffer_has_release_event = [False, False]
        self.prefill_bank_buffers = [cache[:2 * E].view(2, E, *cache.shape[1:])
                                     for _, cache in self.banks]
        self.prefill_copy_stream = torch.cuda.Stream(device=self.device)
        self.prefill_ready_events = [torch.cuda.Event() for _ in range(2)]
        self.prefill_release_events = [torch.cuda.Event() for _ in range(2)]
        self.prefill_begin_event = torch.cuda.Event()
        if self.prefill_hit_d2d:
            self._prefill_slot_snapshot = torch.empty((self.num_layers, E), dtype=torch.int32,
                                                      pin_memory=True)
            self._prefill_snapshot_np = self._prefill_slot_snapshot.numpy()
            self._prefill_hit_dst = torch.empty((E,), dtype=torch.int32, device=self.device)
            self._prefill_hit_src = torch.empty((E,), dtype=torch.int32, device=self.device)
            self._prefill_hit_num = torch.zeros((1,), dtype=torch.int64, device=self.device)

    def _invalidate_prefill_buffer(self, buffer_id: int) -> None:
        """The buffer's slots are about to be overwritten: their owners become non-resident
        and the slots the oldest (reference :597-605)."""
        from .offload_kernels import invalidate_slots

        invalidate_slots(self, buffer_id * self.num_experts, (buffer_id + 1) * self.num_experts)

    def begin_prefill(self) -> None:
        if not self.prefill_overlap:
            return
        self._prefill_buffer_layer = [None, None]
        self._prefill_buffer_released = [True, True]
        # fence this prefill's copies behind everything already queued on the compute stream
        # (a decode still running may read slots the buffers borrow)
        self.prefill_begin_event.record(torch.cuda.current_stream(self.device))
        self.prefill_copy_stream.wait_event(self.prefill_begin_event)
        self._prefill_hit_d2d_active = self.prefill_hit_d2d and self._hit_d2d_usable()
        if self._prefill_hit_d2d_active:
            with torch.cuda.stream(self.prefill_copy_stream):
                self._prefill_slot_snapshot.copy_(self.slot_for_id, non_blocking=True)
            self.prefill_copy_stream.synchronize()

    def _copy_whole_layer(self, layer_id: int, buffer_id: int) -> None:
        E = self.num_experts
        rows = np.arange(E, dtype=np.int64)
        for (per_layer, _), buffer in zip(self.banks, self.prefill_bank_buffers):
            copy_rows_async(buffer[buffer_id], rows, per_layer[layer_id], rows,
                            stream=torch.cuda.current_stream(self.device))

    def prefetch_prefill_layer(self, layer_id: int) -> None:
        if not self.prefill_overlap or layer_id >= self.num_layers:
            return
        if layer_id < 0:
            raise ValueError(f"Invalid prefill layer id: {layer_id}")
        assert self.banks and self.prefill_bank_buffers
        buffer_id = layer_id % 2
        if self._prefill_buffer_layer[buffer_id] == layer_id:
            return
        if self._prefill_buffer_layer[buffer_id] is not None:
            assert self._prefill_buffer_released[buffer_id], (
                "Prefill overlap buffer is being reused before release")
        if self._prefill_hit_d2d_active:
            self._prefetch_split(layer_id, buffer_id)
        else:
            with torch.cuda.stream(self.prefill_copy_stream):
                if self._prefill_buffer_has_release_event[buffer_id]:
                    self.prefill_copy_stream.wait_event(self.prefill_release_events[buffer_id])
                self._invalidate_prefill_buffer(buffer_id)
                self._copy_whole_layer(layer_id, buffer_id)
                self.prefill_ready_events[buffer_id].record(self.prefill_copy_stream)
        self._prefill_buffer_layer[buffer_id] = layer_id
        self._prefill_buffer_released[buffer_id] = False

    def _hit_d2d_usable(self) -> bool:
        from ..kernel.fast_index_copy import _skip_fast_index_copy_enabled

        if self._prefill_slot_snapshot is None or self.prefill_copy_stream is None:
            return False
        if _skip_fast_index_copy_enabled() or not self._copy_fused_ok:
            return False
        return self.cache_size > 2 * self.num_experts

    def _prefetch_split(self, layer_id: int, buffer_id: int) -> None:
        """Resident experts (slots >= 2E) gathered cache -> buffer on the current stream, the
        misses copied host -> buffer as coalesced runs on the copy stream (reference
        :708-778, with per-run hipMemcpyAsync in place of its batched memcpy)."""
        from ..kernel.fast_index_copy import fast_index_copy_multi_jit
        from .offload_kernels import prefill_hit_compact

        E = self.num_experts
        snap = self._prefill_snapshot_np[layer_id]
        hit_mask = snap >= 2 * E
        self.prefill_hit_rows += int(hit_mask.sum())
        self.prefill_total_rows += E
        if self._gather_dst_ptrs is not None:
            prefill_hit_compact(self, layer_id, buffer_id)
            fast_index_copy_multi_jit(self._gather_dst_ptrs, self._gather_dst_ptrs,
                                      self._gather_feat_bytes, self._prefill_hit_dst,
                                      self._prefill_hit_src, self._prefill_hit_num)
        miss = np.nonzero(~hit_mask)[0].astype(np.int64)
        with torch.cuda.stream(self.prefill_copy_stream):
            if self._prefill_buffer_has_release_event[buffer_id]:
                self.prefill_copy_stream.wait_event(self.prefill_release_events[buffer_id])
            self._invalidate_prefill_buffer(buffer_id)
            stream = torch.cuda.current_stream(self.device)
            all_rows = np.arange(E, dtype=np.int64)
            for b, ((per_layer, _), buffer) in enumerate(zip(self.banks,
                                                             self.prefill_bank_buffers)):
                if self._copy_feat_bytes_host[b] < _SMALL_BANK_FEAT_BYTES:
                    copy_rows_async(buffer[buffer_id], all_rows, per_layer[layer_id], all_rows,
                                    stream=stream)
                elif miss.size:
                    copy_rows_async(buffer[buffer_id], miss, per_layer[layer_id], miss,
                                    stream=stream)
            self.prefill_ready_events[buffer_id].record(self.prefill_copy_stream)

    def wait_prefill_layer(self, layer_id: int) -> tuple[torch.Tensor, ...]:
        """Full-layer ``[num_experts, ...]`` views of every bank for ``layer_id``."""
        assert self.prefill_overlap
        assert self.prefill_bank_buffers
        self.prefetch_prefill_layer(layer_id)
        buffer_id = layer_id % 2
        assert self._prefill_buffer_layer[buffer_id] == layer_id
        torch.cuda.current_stream(self.device).wait_event(self.prefill_ready_events[buffer_id])
        return tuple(buffer[buffer_id] for buffer in self.prefill_bank_buffers)

    def release_prefill_layer(self, layer_id: int) -> None:
        if not self.prefill_overlap:
            return
        buffer_id = layer_id % 2
        if self._prefill_buffer_layer[buffer_id] != layer_id:
            return
        self.prefill_release_events[buffer_id].record(torch.cuda.current_stream(self.device))
        self._prefill_buffer_has_release_event[buffer_id] = True
        self._prefill_buffer_released[buffer_id] = True

    # ---- decode -----------------------------------------------------------------------------

    def ensure_experts(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        """Make ``expert_ids`` (int32, this layer's routed experts) resident; rewritten in
        place to slot ids, with the copy plan in evict_slots / src_indices / num_indices."""
        from .offload_kernels import ensure_experts

        if self.collect_decode_freq:
            ids = expert_ids.reshape(-1).long()
            self.decode_freq[layer_id].scatter_add_(0, ids, torch.ones_like(ids))
        self._pending_src_layer = layer_id
        self._pending_whole_layer = False
        ensure_experts(self, layer_id, expert_ids)

    def ensure_experts_hybrid(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        raise NotImplementedError("hybrid CPU/GPU expert decode is not part of this build")

    def materialize_layer(self, layer_id: int) -> None:
        from .offload_kernels import materialize_layer

        self._pending_src_layer = layer_id
        self._pending_whole_layer = True
        materialize_layer(self, layer_id)

    def reset(self) -> None:
        from .offload_kernels import reset_cache

        reset_cache(self)
        self.expert_recency.fill_(-1)

    def reset_stats(self) -> None:
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0
        self.lru_stats.zero_()
        for t in (self.stat_missing, self.stat_active, self.stat_calls, self.stat_fetched,
                  self.stat_missing_layer, self.stat_active_layer, self.stat_fetched_layer,
                  self.stat_steps_layer):
            t.zero_()

    def record_decode_stats(self, layer_id: int) -> None:
        """No-op: ensure_experts accumulates lru_stats inside its own launch."""

    def record_decode_stats_hybrid(self, layer_id: int) -> None:
        raise NotImplementedError("hybrid CPU/GPU expert decode is not part of this build")

    def decode_miss_stats(self) -> dict:
        active, missing, calls = (int(x) for x in self.lru_stats.sum(0))
        fetched = int(self.stat_fetched.item())
        return {
            "layer_calls": calls,
            "active_per_layer": (active / calls) if calls else 0.0,
            "missing_per_layer": (missing / calls) if calls else 0.0,
            "miss_rate": (missing / active) if active else 0.0,
            "fetched_per_layer": (fetched / calls) if calls else 0.0,
            "cpu_per_layer": ((missing - fetched) / calls) if calls else 0.0,
            "fetch_rate": (fetched / missing) if missing else 0.0,
            "prefill_hit_rows": self.prefill_hit_rows,
            "prefill_rows": self.prefill_total_rows,
        }

    def decode_miss_stats_per_layer(self) -> dict:
        cols = self.lru_stats.t().tolist()
        active, missing, steps = cols[Stat.ACTIVE], cols[Stat.MISS], cols[Stat.CALLS]
        fetched = self.stat_fetched_layer.tolist()
        per_layer = []
        for L in range(self.num_layers):
            s, m, a, f = steps[L], missing[L], active[L], fetched[L]
            per_layer.append({
                "layer": L, "steps": s,
                "active_per_step": (a / s) if s else 0.0,
                "missing_per_step": (m / s) if s else 0.0,
                "miss_rate": (m / a) if a else 0.0,
                "fetched_per_step": (f / s) if s else 0.0,
            })
        return {"per_layer": per_layer}

    def decode_routing_stats(self) -> dict:
        """Per-layer routing concentration from the ``collect_decode_freq`` histogram
        (reference :941-971)."""
        freq = self.decode_freq.float()
        total = freq.sum(dim=1)
        valid = total > 0
        if int(valid.sum()) == 0:
            return {}
        C = max(1, int(round(self.cache_size / self.num_layers)))
        sorted_f, _ = torch.sort(freq, dim=1, descending=True)
        oracle_hit = (sorted_f[:, :C].sum(dim=1)[valid] / total[valid]).mean().item()
        ws = (freq > 0).sum(dim=1).float()
        cdf = torch.cumsum(sorted_f, dim=1) / total.clamp(min=1).unsqueeze(1)
        cover90 = ((cdf < 0.9).sum(dim=1).float() + 1)[valid]
        p = freq / total.clamp(min=1).unsqueeze(1)
        ent = -(p * p.clamp(min=1e-12).log()).sum(dim=1)[valid]
        norm_ent = (ent / torch.log(torch.tensor(float(self.num_experts)))).mean().item()
        return {
            "slots_per_layer": self.cache_size / self.num_layers,
            "working_set_mean": ws[valid].mean().item(),
            "working_set_max": int(ws[valid].max().item()),
            "experts_for_90pct": cover90.mean().item(),
            "oracle_hit_at_slots": oracle_hit,
            "norm_entropy": norm_ent,
        }

    def copy_missing(self) -> None:
        """Copy the rows planned by the last ensure_experts / materialize_layer from that
        layer's pinned banks into their slots: one multi-bank launch, or one launch per bank
        when the fused descriptor is unavailable. The count stays on the device."""
        assert self.banks, "set_bank_sources must register the banks first"
        layer_id = self._pending_src_layer
        assert layer_id is not None, "no staged misses (ensure_experts/materialize_layer first)"
        if self._copy_fused_ok:
            from ..kernel.fast_index_copy import fast_index_copy_multi_jit

            fast_index_copy_multi_jit(self._copy_dst_ptrs, self._copy_src_ptrs[layer_id],
                                      self._copy_feat_bytes, self.evict_slots, self.src_indices,
                                      self.num_indices)
            return
        from ..kernel.fast_index_copy import fast_index_copy_jit

        for per_layer, cache in self.banks:
            fast_index_copy_jit(cache, self.evict_slots, per_layer[layer_id], self.src_indices,
                                self.num_indices)
