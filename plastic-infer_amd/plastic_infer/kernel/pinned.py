"""Pinned host-tensor helpers used by the expert caches (the reference's
src/plastic_infer/kernel/pinned.py surface that the slot-cache path needs)."""

from __future__ import annotations

import torch

from .index_copy import device_ptr

__all__ = ["copy_to_pinned_tensor", "create_pinned_tensor_like", "device_ptr"]


def create_pinned_tensor_like(input: torch.Tensor) -> torch.Tensor:
    """A pinned host tensor with the size, stride and dtype of ``input``."""
    return torch.empty_strided(input.shape, input.stride(), dtype=input.dtype, device="cpu",
                               pin_memory=True)


def copy_to_pinned_tensor(input: torch.Tensor) -> torch.Tensor:
    """Copy a host tensor into newly allocated pinned storage."""
    out = create_pinned_tensor_like(input)
    out.copy_(input)
    return out
