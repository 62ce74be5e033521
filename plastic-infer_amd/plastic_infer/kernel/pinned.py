"""Pinned host-tensor helpers used by the expert caches (the reference's
src/plastic_infer/kernel/pinned.py surface that the slot-cache path needs)."""

from __future__ import annotations

import torch

from .index_copy import device_ptr

__all__ = ["alloc_pinned_tensor", "copy_to_pinned_tensor", "create_pinned_tensor_like",
           "device_ptr"]


def create_pinned_tensor_like(input: torch.Tensor) -> torch.Tensor:
    """A pinned host tensor with the size, stride and dtype of ``input``."""
    return torch.empty_strided(input.shape, input.stride(), dtype=input.dtype, device="cpu",
                               pin_memory=True)


def copy_to_pinned_tensor(input: torch.Tensor) -> torch.Tensor:
    """Copy a host tensor into newly allocated pinned storage."""
    out = create_pinned_tensor_like(input)
    out.copy_(input)
    return out


def alloc_pinned_tensor(*shape: int, dtype: torch.dtype) -> torch.Tensor:
    """A pinned host tensor of the given shape (reference src/plastic_infer/kernel/pinned.py:65-67:
    torch's pinned pool, which HIP maps into every device's address space)."""
    return torch.empty(tuple(int(s) for s in shape), dtype=dtype, pin_memory=True)


_INFLIGHT: list = []


def hold_until_done(objs, stream: torch.cuda.Stream) -> None:
    """Keep `objs` (typically pinned host tensors a kernel reads in place through their device
    mapping) alive until the work queued so far on `stream` has finished. torch's pinned pool
    only tracks its own copies, so a block freed while a kernel still reads it could be handed
    out and rewritten; finished entries are released on later calls."""
    while _INFLIGHT and _INFLIGHT[0][0].query():
        _INFLIGHT.pop(0)
    ev = torch.cuda.Event()
    ev.record(stream)
    _INFLIGHT.append((ev, objs))
