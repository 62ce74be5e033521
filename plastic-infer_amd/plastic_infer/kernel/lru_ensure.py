"""Device-side LRU admission for a GPU slot cache over an out-of-core table.

Same call as the reference's ``lru_ensure`` (src/plastic_infer/kernel/lru_ensure.py:371-438),
run by the HIP kernel ``pia_lru_ensure``: one launch on the current stream, fixed shapes, no
host synchronisation. The reference routes between two strategies that it documents as
bit-identical (register-resident argmins; a streaming insert for caches of 40000+ slots).
Here caches of up to 16384 slots keep their state in LDS (victims by rounds of smallest
usage), larger ones (up to 2^24 slots) stream it from global memory (a radix select of the
victims' usage); both make the same decisions, so ``strategy`` only selects among the same
results.
"""

from __future__ import annotations

from enum import IntEnum

import torch

from .. import _native as N


class Stat(IntEnum):
    """Columns of the optional ``stats`` accumulator (cumulative; zero the tensor to reset)."""

    ACTIVE = 0  #: distinct queried ids
    MISS = 1  #: distinct missing ids admitted (the sum of ``num_copy``)
    CALLS = 2  #: number of calls


N_STATS = len(Stat)
_STRATEGIES = ("seq", "insert")
MAX_QUERY = 2048         # queries held in LDS; longer ones take the wide-query kernel
MAX_QUERY_WIDE = 1 << 24
MAX_CACHED_WIDE = 16384  # the wide-query kernel's cache limit
MAX_CACHED = 1 << 24     # caches above 16384 slots take the streaming kernel


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def lru_ensure(
    query: torch.Tensor,
    slot_of_id: torch.Tensor,
    id_of_slot: torch.Tensor,
    lru_usage: torch.Tensor,
    lru_step: torch.Tensor,
    out_indices: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    num_copy: torch.Tensor,
    stats: torch.Tensor | None = None,
    id_base: int = 0,
    strategy: str | None = None,
    **tuning,
) -> None:
    """Make every id in ``query`` resident and emit the plan that fills the new slots.

    query (K,) int32 ids (plus ``id_base``); slot_of_id (num_total,) int32 in/out; id_of_slot
    (num_cached,) int32 in/out; lru_usage (num_cached,) int64 in/out; lru_step () int64 in/out;
    out_indices (K,) int32 out (may alias query); src_indices / dst_indices (>= min(K,
    num_cached),) int32 out; num_copy int64 [1] or () out; stats (3,) int64 accumulator or None.
    The distinct missing ids, ascending, take the least-recently-used slots not touched by
    this call, lowest slot first on equal usage. num_cached <= 2^24; K <= 2048, or up to 2^24
    with num_cached <= 16384 (a query longer than 2048 ids is admitted in ascending batches of
    2048 distinct misses, with the same decisions).
    """
    if strategy is not None and strategy not in _STRATEGIES:
        raise KeyError(strategy)
    unknown = set(tuning) - {"block_c_tile"}
    if unknown:
        raise TypeError(f"unexpected tuning arguments {sorted(unknown)}")
    dev = N.require_device(query, slot_of_id, id_of_slot, lru_usage, lru_step, out_indices,
                           src_indices, dst_indices, num_copy,
                           names=("query", "slot_of_id", "id_of_slot", "lru_usage", "lru_step",
                                  "out_indices", "src_indices", "dst_indices", "num_copy"))
    k, num_cached = query.numel(), id_of_slot.numel()
    _check(query.dtype == torch.int32 and query.is_contiguous(), "query must be contiguous int32")
    _check(slot_of_id.dtype == torch.int32 and id_of_slot.dtype == torch.int32,
           "slot maps must be int32")
    _check(slot_of_id.is_contiguous() and id_of_slot.is_contiguous(), "slot maps must be contiguous")
    _check(out_indices.dtype == torch.int32 and out_indices.numel() == k
           and out_indices.is_contiguous(), "out_indices must be contiguous int32 [K]")
    _check(lru_usage.dtype == lru_step.dtype, "lru_usage and lru_step must share a dtype")
    if lru_usage.dtype != torch.int64:
        raise ValueError("lru_usage / lru_step must be int64")
    _check(lru_usage.numel() == num_cached and lru_usage.is_contiguous(),
           "lru_usage must be contiguous [num_cached]")
    _check(lru_step.numel() == 1, "lru_step must hold one value")
    plan = min(k, num_cached)
    _check(src_indices.numel() >= plan and dst_indices.numel() >= plan,
           "plan tensors shorter than min(K, num_cached)")
    _check(src_indices.dtype == torch.int32 and dst_indices.dtype == torch.int32,
           "plan tensors must be int32")
    _check(num_copy.dtype == torch.int64 and num_copy.numel() == 1, "num_copy must be int64 [1]")
    if stats is not None:
        N.require_device(stats, names=("stats",))
        _check(stats.dtype == torch.int64 and stats.numel() == N_STATS and stats.is_contiguous(),
               "stats must be a contiguous int64 [3] tensor")
    if num_cached > MAX_CACHED or k > MAX_QUERY_WIDE or \
            (k > MAX_QUERY and num_cached > MAX_CACHED_WIDE):
        raise ValueError(f"lru_ensure supports num_cached <= {MAX_CACHED} with K <= {MAX_QUERY}, "
                         f"and K <= {MAX_QUERY_WIDE} with num_cached <= {MAX_CACHED_WIDE}")
    N.call("pia_lru_ensure", query.data_ptr(), k, slot_of_id.data_ptr(), slot_of_id.numel(),
           id_of_slot.data_ptr(), lru_usage.data_ptr(), num_cached, lru_step.data_ptr(),
           out_indices.data_ptr(), src_indices.data_ptr(), dst_indices.data_ptr(),
           num_copy.data_ptr(), N.ptr(stats), int(id_base), N.stream_of(dev))
