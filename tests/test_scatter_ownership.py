"""CPU emulation of the page-segment scatter kernel's ownership rules (kv_scatter16_kernel in
plastic-infer_amd/csrc/kv_cache.hip), checked against the oracle's per-token store.

The kernel gives input group g (tokens 16g .. 16g+15) to one wave. Lane j looks at token
16g - 1 + j; a lane flags a segment start where the slot does not continue the previous one
inside its page. The wave owns every segment starting in lanes 1..16 (with the spill of the
last into the next group) and writes either a whole page (one 16-token segment from a page
start) or token pairs. This emulation follows that decision per wave and composes the writes;
the union must equal the oracle's slot -> token map for every layout. With the one-segment
test of the whole-page path removed (the earlier kernel), the ragged layouts fail, which shows
that these layouts reach the case.
"""

from __future__ import annotations

import pytest

from scatter_layouts import P, ragged_21_11_40, random_layout


def _emulate(slots: list[int], total_slots: int, one_segment_check: bool = True) -> dict:
    """slot -> input token index, as the kernel's waves write them (16-byte pools)."""
    n = len(slots)
    writes: dict[int, int] = {}

    def put(slot: int, tok: int) -> None:
        assert slot not in writes, f"slot {slot} written twice"
        writes[slot] = tok

    for i0 in range(0, n, P):
        s = []
        for j in range(64):
            tj = i0 - 1 + j
            v = -1
            if j < 33 and 0 <= tj < n:
                v = slots[tj]
                if v < 0 or v >= total_slots:
                    v = -1
            s.append(v)
        starts = 0
        for j in range(1, 33):
            tj = i0 - 1 + j
            sp = s[j - 1]
            if s[j] < 0 or sp < 0 or s[j] != sp + 1 or s[j] % P == 0 or tj >= n:
                starts |= 1 << j
        low = starts & 0x1FFFE
        a = (low & -low).bit_length() - 1
        after = starts & ~0x1FFFF
        b = (after & -after).bit_length() - 1 if after else 33
        m = max(0, min(b, min(n - i0 + 1, 33)) - a)
        t0 = i0 - 1 + a
        if m == 0:
            continue
        sfirst = s[a & 63]
        one_seg = ((starts >> (a + 1)) & 0x7FFF) == 0
        full = m == P and sfirst >= 0 and sfirst % P == 0 and (one_seg or not one_segment_check)
        if full:
            for j in range(P):
                put(sfirst + j, t0 + j)
            continue
        for pi in range(16):
            for e in (0, 1):
                idx = 2 * pi + e
                sv = s[(a + idx) & 63]
                if idx < m and sv >= 0:
                    put(sv, t0 + idx)
    return writes


def _oracle(slots: list[int], total_slots: int) -> dict:
    return {s: i for i, s in enumerate(slots) if 0 <= s < total_slots}


@pytest.mark.parametrize("seed", range(12))
def test_random_layouts_match_oracle(seed):
    slots = random_layout(seed)
    total = 4096 * P
    assert _emulate(slots, total) == _oracle(slots, total)


def test_ragged_21_11_40_and_padding():
    slots = []
    for r in range(20):
        slots += ragged_21_11_40(8 * r)
    slots += [500 * P + i for i in range(8)] + [-1] * 8      # page-start run, then padding
    slots += [(600 + i) * P for i in range(40)]              # decode slots at offset 0
    total = 4096 * P
    assert _emulate(slots, total) == _oracle(slots, total)


def test_old_whole_page_condition_fails_on_these_layouts():
    """Planted mistake: without the one-segment test the 21/11/40 layout writes the second
    sequence's 11 tokens over the first sequence's page."""
    slots = ragged_21_11_40(0) * 1
    total = 64 * P
    with pytest.raises(AssertionError):
        assert _emulate(slots, total, one_segment_check=False) == _oracle(slots, total)
    pad = [3 * P + i for i in range(8)] + [-1] * 8
    with pytest.raises(AssertionError):
        assert _emulate(pad, total, one_segment_check=False) == _oracle(pad, total)
