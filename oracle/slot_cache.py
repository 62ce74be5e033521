"""ORACLE (test infrastructure only): CPU restatement of the reference's device-side slot cache
(LRU admission and the OffloadMoeCache bookkeeping kernels), numpy, one call at a time.

State is a dict of numpy arrays: slot_of_id [num_total] i32, id_of_slot [num_cached] i32,
usage [num_cached] i64, step int. Every function mutates it in place as the reference kernel
mutates the device tensors.
"""

from __future__ import annotations

import numpy as np

USAGE_MAX = np.iinfo(np.int64).max


def new_state(num_total: int, num_cached: int) -> dict:
    return {"slot_of_id": np.full(num_total, -1, np.int32),
            "id_of_slot": np.full(num_cached, -1, np.int32),
            "usage": np.zeros(num_cached, np.int64), "step": 0}


def lru_ensure(st: dict, query, id_base: int = 0):
    """reference src/plastic_infer/kernel/lru_ensure.py:200-245 (_lru_ensure_kernel, the
    sequential strategy; the streaming one is documented bit-identical, :262-276) with
    _phase1 (:62-107): step += 1; hits get usage = step; the distinct missing ids in
    ascending order take, one by one, the argmin-usage slot among those not touched by this
    call (lowest slot on ties), unmapping its previous owner.
    Returns (out, src_plan, dst_plan, num_copy, (distinct, misses, 1))."""
    sid, ios, usage = st["slot_of_id"], st["id_of_slot"], st["usage"]
    st["step"] += 1
    step = st["step"]
    q = np.asarray(query, np.int64).reshape(-1) + id_base
    K = q.size
    s = sid[q].astype(np.int64)
    hit = s >= 0
    miss = s == -1
    first = np.array([not np.any(q[:i] == q[i]) for i in range(K)], dtype=bool)
    first_miss = miss & first
    fm_ids = q[first_miss]
    rank = np.array([int(np.sum(fm_ids < q[i])) for i in range(K)], dtype=np.int64)
    M = int(first_miss.sum())
    usage[s[hit]] = step
    out = np.where(hit, s, -1)
    src, dst = [], []
    if M:
        u = usage.copy()
        u[u == step] = USAGE_MAX
        for i in range(M):
            victim = int(np.argmin(u))
            old = int(ios[victim])
            if old >= 0:
                sid[old] = -1
            e = int(np.sort(fm_ids)[i])
            ios[victim] = e
            sid[e] = victim
            usage[victim] = step
            dst.append(victim)
            src.append(e - id_base)
            out = np.where((rank == i) & miss, victim, out)
            u[victim] = USAGE_MAX
    return (out.astype(np.int32), np.asarray(src, np.int32), np.asarray(dst, np.int32), M,
            (int(first.sum()), M, 1))


def materialize(st: dict, layer_id: int, num_experts: int):
    """reference src/plastic_infer/moe/offload_kernels.py:249-285 (_materialize_layer_kernel):
    slots [0, E) take this layer's experts in id order. Returns (evict_slots, src, num)."""
    sid, ios, usage = st["slot_of_id"], st["id_of_slot"], st["usage"]
    E, base = num_experts, layer_id * num_experts
    old = ios.copy()
    slots = np.arange(ios.size)
    same = (old >= base) & (old < base + E)
    ios[same] = -1
    usage[same] = 0
    old_valid = (slots < E) & (old >= 0) & ~same
    sid[old[old_valid]] = -1
    st["step"] += 1
    ios[:E] = base + np.arange(E)
    sid[base:base + E] = np.arange(E)
    usage[:E] = st["step"]
    return np.arange(E, dtype=np.int32), np.arange(E, dtype=np.int32), E


def reset(st: dict) -> None:
    """reference src/plastic_infer/moe/offload_kernels.py:226-246 (_reset_cache_kernel)."""
    st["slot_of_id"][:] = -1
    st["id_of_slot"][:] = -1
    st["usage"][:] = 0
    st["step"] = 0


def invalidate(st: dict, slot_begin: int, slot_end: int) -> None:
    """reference src/plastic_infer/moe/offload_cache.py:597-605 (_invalidate_prefill_buffer)."""
    old = st["id_of_slot"][slot_begin:slot_end]
    st["slot_of_id"][old[old >= 0]] = -1
    old[:] = -1
    st["usage"][slot_begin:slot_end] = 0


def prefill_hit_compact(slot_row, buffer_base: int, threshold: int):
    """reference src/plastic_infer/moe/offload_kernels.py:413-431: (dst rows, src slots, n)."""
    slot_row = np.asarray(slot_row, np.int64)
    e = np.nonzero(slot_row >= threshold)[0]
    return (buffer_base + e).astype(np.int32), slot_row[e].astype(np.int32), int(e.size)
