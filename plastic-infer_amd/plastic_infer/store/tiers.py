"""Re-export of the storage tiers for the store package."""

from ..planning.tiers import TIER_ORDER, Tier, tier_colder  # noqa: F401
