"""Storage tiers (reference: src/plastic_infer/planning/tiers.py): where a tracked object lives."""

from __future__ import annotations

from enum import Enum, auto


class Tier(Enum):
    GPU = auto()    # HBM
    HOST = auto()   # host RAM (pinned or pageable)
    DISK = auto()   # NVMe / SSD


TIER_ORDER: dict[Tier, int] = {Tier.GPU: 0, Tier.HOST: 1, Tier.DISK: 2}


def tier_colder(a: Tier, b: Tier) -> bool:
    """True if tier a is slower / cheaper than tier b."""
    return TIER_ORDER[a] > TIER_ORDER[b]
