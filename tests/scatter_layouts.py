"""Slot-mapping layouts for scatter tests (test helper, no GPU).

Each layout is a list of int64 slots (page * 16 + offset, -1 for padding) made of segments on
distinct pages, so no slot repeats and the result of a scatter does not depend on write order.
The layouts target the page-segment scatter kernel's ownership rules: several short segments
that add up to 16 tokens right after a page start, a page-start run followed by padding, and
single decode slots at offset 0, mixed with whole pages and runs crossing group boundaries.
"""

from __future__ import annotations

import random

P = 16


def ragged_21_11_40(base_page: int) -> list[int]:
    """Three sequences of 21, 11 and 40 tokens, each from its own page start: after the first
    16 tokens the second group holds 5 + 11 tokens of two segments (a page start, then 16)."""
    out, page = [], base_page
    for n in (21, 11, 40):
        out += [page * P + i for i in range(n)]
        page += (n + P - 1) // P
    return out


def random_layout(seed: int, n_min: int = 1100, n_pages: int = 4096) -> list[int]:
    """Random mix of segment kinds until at least n_min tokens, on pages below n_pages."""
    rng = random.Random(seed)
    pages = list(range(n_pages))
    rng.shuffle(pages)
    nxt = iter(pages)
    out: list[int] = []
    while len(out) < n_min:
        kind = rng.randrange(7)
        if kind == 0:                        # a whole page
            p = next(nxt)
            out += [p * P + i for i in range(P)]
        elif kind == 1:                      # short run from a page start
            p = next(nxt)
            out += [p * P + i for i in range(rng.randint(1, P - 1))]
        elif kind == 2:                      # run from an odd offset, clipped to its page
            p, o = next(nxt), rng.randint(1, P - 1)
            out += [p * P + i for i in range(o, min(P, o + rng.randint(1, P)))]
        elif kind == 3:                      # page-start run, then padding
            p, n = next(nxt), rng.randint(1, P - 1)
            out += [p * P + i for i in range(n)] + [-1] * rng.randint(1, P - n)
        elif kind == 4:                      # decode slots: one token per page, often offset 0
            for _ in range(rng.randint(1, 20)):
                p = next(nxt)
                out.append(p * P + (0 if rng.random() < 0.5 else rng.randrange(P)))
        elif kind == 5:                      # a sequence over several pages from a page start
            n = rng.randint(17, 70)
            first = [next(nxt) for _ in range((n + P - 1) // P)]
            out += [first[i // P] * P + i % P for i in range(n)]
        else:                                # the 21 / 11 / 40 pattern
            base = [next(nxt) for _ in range(6)]
            for n, pp in ((21, base[0:2]), (11, base[2:3]), (40, base[3:6])):
                out += [pp[i // P] * P + i % P for i in range(n)]
    return out
