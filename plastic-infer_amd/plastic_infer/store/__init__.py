"""Residency bookkeeping and the expert slot pool."""
