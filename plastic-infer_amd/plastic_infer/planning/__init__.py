"""Storage tier vocabulary."""
