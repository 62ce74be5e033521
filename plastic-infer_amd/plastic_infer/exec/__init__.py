"""Paged attention and MoE routing ops with the reference's call signatures."""
