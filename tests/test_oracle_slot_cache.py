"""Pins oracle/slot_cache.py (the reference's device LRU admission has no test of its own):
hand-derived known answers from the kernel's stated rule, invariants over random call
sequences checked by brute force, and planted mistakes that those checks must catch."""

from __future__ import annotations

import numpy as np
import pytest

import oracle.slot_cache as SC


def test_known_answer_sequence():
    st = SC.new_state(10, 4)
    # call 1: all miss; distinct misses ascending (1, 3) take slots 0, 1 (usage ties -> slot)
    out, src, dst, n, stats = SC.lru_ensure(st, [3, 1, 3])
    assert out.tolist() == [1, 0, 1] and src.tolist() == [1, 3] and dst.tolist() == [0, 1]
    assert n == 2 and stats == (2, 2, 1) and st["step"] == 1
    # call 2: 3 hits slot 1 (bumped to 2); 5 takes the oldest untouched slot: 2 (usage 0)
    out, src, dst, n, _ = SC.lru_ensure(st, [5, 3])
    assert out.tolist() == [2, 1] and dst.tolist() == [2] and n == 1
    assert st["usage"].tolist() == [1, 2, 2, 0]
    # call 3: three misses against usages (1, 2, 2, 0): victims slot 3, 0, 1 in that order
    out, src, dst, n, _ = SC.lru_ensure(st, [9, 8, 7])
    assert dst.tolist() == [3, 0, 1] and src.tolist() == [7, 8, 9]
    assert out.tolist() == [1, 0, 3]
    assert st["slot_of_id"][1] == -1 and st["slot_of_id"][3] == -1   # evicted owners
    assert st["id_of_slot"].tolist() == [8, 9, 5, 7]
    # id_base: partition-local ids in the plan, global ids in the maps
    out, src, dst, n, _ = SC.lru_ensure(st, [0, 1], id_base=5)   # global 5 (hit), 6 (miss)
    assert out[0] == 2 and src.tolist() == [1] and st["id_of_slot"][dst[0]] == 6


def _check_call(before: dict, after: dict, query, out, src, dst, n, id_base):
    q = np.asarray(query) + id_base
    sid, ios, usage = after["slot_of_id"], after["id_of_slot"], after["usage"]
    step = after["step"]
    # every queried id is resident where out says, maps are inverse of each other
    assert np.all(sid[q] == out) and np.all(out >= 0)
    res = np.nonzero(sid >= 0)[0]
    assert np.all(ios[sid[res]] == res)
    held = ios[ios >= 0]
    assert np.all(sid[held] == np.nonzero(ios >= 0)[0])
    # hits kept their slot; misses are exactly the plan, distinct ids ascending
    was = before["slot_of_id"][q]
    assert np.all(out[was >= 0] == was[was >= 0])
    missing = np.unique(q[was < 0])
    assert n == missing.size and np.all(src + id_base == missing)
    # victims are the least-recently-used slots not touched by this call, lowest slot first
    touched = set(out[was >= 0].tolist())
    cand = sorted((int(before["usage"][c]), c) for c in range(ios.size) if c not in touched)
    assert [c for _, c in cand[:n]] == dst.tolist()
    assert np.all(usage[out] == step)


@pytest.mark.parametrize("seed,total,cached,k", [(0, 64, 16, 8), (1, 300, 40, 32),
                                                 (2, 20, 20, 20), (3, 1000, 8, 5)])
def test_invariants_random_sequences(seed, total, cached, k):
    rng = np.random.default_rng(seed)
    st = SC.new_state(total, cached)
    for _ in range(60):
        base = int(rng.integers(0, 4)) * (total // 4)
        span = total // 4
        n_distinct = min(cached, k, span)
        ids = rng.choice(span, size=int(rng.integers(1, n_distinct + 1)), replace=False)
        query = rng.choice(ids, size=int(rng.integers(1, k + 1)))
        before = {key: (v.copy() if isinstance(v, np.ndarray) else v) for key, v in st.items()}
        out, src, dst, n, _ = SC.lru_ensure(st, query, id_base=base)
        _check_call(before, st, query, out, src, dst, n, base)


def test_materialize_invalidate_reset_compact():
    st = SC.new_state(3 * 4, 6)
    SC.lru_ensure(st, [0, 1, 2, 3], id_base=8)      # layer 2 resident in slots 0..3
    SC.lru_ensure(st, [1], id_base=4)               # layer 1 expert 1 -> slot 4
    ev, src, n = SC.materialize(st, 1, 4)           # layer 1 takes slots 0..3
    assert n == 4 and ev.tolist() == [0, 1, 2, 3] and src.tolist() == [0, 1, 2, 3]
    assert st["id_of_slot"][:4].tolist() == [4, 5, 6, 7]
    assert st["id_of_slot"][4] == -1 and st["usage"][4] == 0   # its old copy emptied
    assert np.all(st["slot_of_id"][8:12] == -1)               # layer 2 evicted
    assert st["slot_of_id"][4:8].tolist() == [0, 1, 2, 3]
    SC.invalidate(st, 0, 2)
    assert st["slot_of_id"][4] == -1 and st["slot_of_id"][5] == -1
    assert st["id_of_slot"][:2].tolist() == [-1, -1] and st["usage"][:2].tolist() == [0, 0]
    dst, srcs, n = SC.prefill_hit_compact([3, -1, 9, 4, 2], buffer_base=5, threshold=4)
    assert dst.tolist() == [7, 8] and srcs.tolist() == [9, 4] and n == 2
    SC.reset(st)
    assert np.all(st["slot_of_id"] == -1) and np.all(st["id_of_slot"] == -1) and st["step"] == 0


# ---- planted mistakes: the checks above must catch each of them ----------------------------

def _planted(monkeypatch, mutate):
    orig = np.sort

    def bad_sort(a, *args, **kw):
        return mutate(orig(a, *args, **kw))

    monkeypatch.setattr(SC.np, "sort", bad_sort)


def test_planted_descending_pairing_is_caught(monkeypatch):
    # pairing the misses with victims in descending id order instead of ascending
    _planted(monkeypatch, lambda a: a[::-1])
    with pytest.raises(AssertionError):
        test_known_answer_sequence()


def test_planted_most_recently_used_victim_is_caught(monkeypatch):
    orig = np.argmin

    def argmax_finite(u, *a, **k):
        v = np.where(u == SC.USAGE_MAX, -1, u)
        return int(np.argmax(v)) if np.any(v >= 0) else int(orig(u))

    monkeypatch.setattr(SC.np, "argmin", argmax_finite)
    with pytest.raises(AssertionError):
        test_invariants_random_sequences(1, 300, 40, 32)
