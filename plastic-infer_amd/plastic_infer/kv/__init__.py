"""Paged KV: allocator, block tables, chunk keys and the HBM KV store."""
