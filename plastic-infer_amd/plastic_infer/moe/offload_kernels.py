"""Device-side bookkeeping of OffloadMoeCache (reference src/plastic_infer/moe/offload_kernels.py),
on the HIP slot-cache kernels. Every call is one launch on the current stream with no host
synchronisation, so the decode-time admission -> copy -> GEMM chain stays capturable."""

from __future__ import annotations

import torch

from .. import _native as N
from ..kernel.lru_ensure import lru_ensure


def ensure_experts(cache, layer_id: int, expert_ids: torch.Tensor) -> None:
    """Make this layer's routed experts resident and rewrite ``expert_ids`` to slot ids in
    place (reference :19-40). ``id_base`` puts the layer's experts in the flat
    ``layer * num_experts + expert`` id space of the maps and takes the plan back to
    layer-local rows, so ``copy_missing`` reads this layer's own host bank."""
    lru_ensure(
        expert_ids,
        cache.slot_for_id.view(-1),
        cache.id_of_slot,
        cache.usage,
        cache.step,
        expert_ids,
        cache.src_indices,
        cache.evict_slots,
        cache.num_indices,
        stats=cache.lru_stats[layer_id] if cache.collect_stats else None,
        id_base=layer_id * cache.num_experts,
    )


def ensure_experts_hybrid(cache, layer_id: int, expert_ids: torch.Tensor, max_fetch: int,
                          fetch_fraction: float = 0.0) -> None:
    """The capped-fetch variant feeds a CPU expert executor, which this build does not have."""
    raise NotImplementedError("hybrid CPU/GPU expert decode is not part of this build")


def prefill_hit_compact(cache, layer_id: int, buffer_id: int) -> None:
    """Compact this layer's experts resident at or above slot 2E (the double buffers own the
    slots below) into fixed-shape gather indices (reference :63-82): buffer rows in
    ``_prefill_hit_dst``, cache slots in ``_prefill_hit_src``, the count in
    ``_prefill_hit_num``."""
    E = cache.num_experts
    row = cache.slot_for_id[layer_id]
    N.call("pia_prefill_hit_compact", row.data_ptr(), cache._prefill_hit_dst.data_ptr(),
           cache._prefill_hit_src.data_ptr(), cache._prefill_hit_num.data_ptr(), buffer_id * E,
           2 * E, E, N.stream_of(row.device))


def materialize_layer(cache, layer_id: int) -> None:
    """Slots [0, E) take this layer's experts in id order; the plan copies the whole layer
    (reference :249-285)."""
    dev = cache.slot_for_id.device
    N.call("pia_slot_cache_materialize", cache.slot_for_id.data_ptr(), cache.slot_for_id.numel(),
           cache.id_of_slot.data_ptr(), cache.usage.data_ptr(), cache.id_of_slot.numel(),
           cache.step.data_ptr(), cache.evict_slots.data_ptr(), cache.src_indices.data_ptr(),
           cache.num_indices.data_ptr(), int(layer_id), cache.num_experts, N.stream_of(dev))


def reset_cache(cache) -> None:
    """Every expert non-resident, every slot empty, clock and plan zeroed (reference
    :226-246)."""
    dev = cache.slot_for_id.device
    N.call("pia_slot_cache_reset", cache.slot_for_id.data_ptr(), cache.slot_for_id.numel(),
           cache.id_of_slot.data_ptr(), cache.usage.data_ptr(), cache.id_of_slot.numel(),
           cache.step.data_ptr(), cache.active_mask.data_ptr(), cache.num_experts,
           cache.num_indices.data_ptr(), N.stream_of(dev))


def invalidate_slots(cache, slot_begin: int, slot_end: int) -> None:
    """Empty slots [slot_begin, slot_end): owners become non-resident, usage 0 (the oldest)."""
    dev = cache.slot_for_id.device
    N.call("pia_slot_cache_invalidate", cache.slot_for_id.data_ptr(), cache.slot_for_id.numel(),
           cache.id_of_slot.data_ptr(), cache.usage.data_ptr(), cache.id_of_slot.numel(),
           int(slot_begin), int(slot_end), N.stream_of(dev))
