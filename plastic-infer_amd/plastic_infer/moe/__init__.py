"""Fused-MoE routing front end and the batched expert slot cache."""
