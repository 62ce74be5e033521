"""Device-side bookkeeping of OffloadMoeCache (reference src/plastic_infer/moe/offload_kernels.py),
on the HIP slot-cache kernels. Every call is one launch on the current stream with no host
synchronisation, so the decode-time admission -> copy -> GEMM chain stays capturable.

The functions take the cache as their first argument, as the reference's do, and act on its
device maps (``slot_for_id``, ``id_of_slot``, ``usage``, ``step``) and copy plan
(``evict_slots``, ``src_indices``, ``num_indices``)."""

from __future__ import annotations

import torch

from .. import _native as N


def ensure_experts(cache, layer_id: int, expert_ids: torch.Tensor) -> None:
    """Make this layer's routed experts resident and rewrite ``expert_ids`` (int32) to slot ids
    in place (reference :19-40). Under the "lru" policy this is the device admission kernel
    with ``id_base = layer * num_experts`` (the maps index flat ``layer * E + expert`` ids and
    the plan holds layer-local rows, so ``cache.copy_missing()`` reads this layer's own host
    banks); under "static" the misses are staged by DMA before the call returns its stream
    order."""
    cache.ensure_experts(int(layer_id), expert_ids)


def ensure_experts_hybrid(cache, layer_id: int, expert_ids: torch.Tensor, max_fetch: int,
                          fetch_fraction: float = 0.0) -> None:
    """The capped-fetch variant feeds a CPU expert executor, which this build does not have."""
    raise NotImplementedError("hybrid CPU/GPU expert decode is not part of this build")


def prefill_hit_compact(cache, layer_id: int, buffer_id: int) -> None:
    """Compact this layer's experts resident at or above slot 2E (the double buffers own the
    slots below) into fixed-shape gather indices (reference :63-82): buffer rows
    ``buffer_id * E + e`` in ``cache._prefill_hit_dst``, their cache slots in
    ``cache._prefill_hit_src`` (ascending e), the count in ``cache._prefill_hit_num``."""
    E = cache.num_experts
    if not 0 <= int(layer_id) < cache.num_layers:
        raise ValueError(f"layer_id {layer_id} outside [0, {cache.num_layers})")
    if int(buffer_id) not in (0, 1):
        raise ValueError(f"buffer_id must be 0 or 1, got {buffer_id}")
    row = cache.slot_for_id[int(layer_id)]
    N.call("pia_prefill_hit_compact", row.data_ptr(), cache._prefill_hit_dst.data_ptr(),
           cache._prefill_hit_src.data_ptr(), cache._prefill_hit_num.data_ptr(),
           int(buffer_id) * E, 2 * E, E, N.stream_of(row.device))


def materialize_layer(cache, layer_id: int) -> None:
    """Slots [0, E) take this layer's experts in id order and the plan copies the whole layer
    (reference :85-86, :191-206, kernel :249-285); ``cache.copy_missing()`` moves the rows."""
    cache.materialize_layer(int(layer_id))


def reset_cache(cache) -> None:
    """Every expert non-resident, every slot empty, clock and plan count zeroed (reference
    :89-94, kernel :226-246)."""
    cache.reset()


__all__ = ["ensure_experts", "ensure_experts_hybrid", "prefill_hit_compact", "materialize_layer",
           "reset_cache"]
