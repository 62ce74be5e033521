"""Pinned host-tensor helpers used by the expert caches (the reference's
src/plastic_infer/kernel/pinned.py surface that the slot-cache path needs)."""

from __future__ import annotations

import ctypes
import math
import threading
import weakref

import torch

from .index_copy import device_ptr

__all__ = ["alloc_pinned_exact", "alloc_pinned_tensor", "copy_to_pinned_tensor",
           "create_pinned_tensor_like", "device_ptr"]

_hip_lock = threading.Lock()
_hip_rt: ctypes.CDLL | None = None


def _hip_runtime() -> ctypes.CDLL:
    global _hip_rt
    with _hip_lock:
        if _hip_rt is None:
            rt = ctypes.CDLL("libamdhip64.so")
            rt.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t,
                                         ctypes.c_uint]
            rt.hipHostMalloc.restype = ctypes.c_int
            rt.hipHostFree.argtypes = [ctypes.c_void_p]
            rt.hipHostFree.restype = ctypes.c_int
            _hip_rt = rt
        return _hip_rt


def alloc_pinned_exact(shape, dtype: torch.dtype) -> torch.Tensor:
    """A contiguous host tensor in page-locked memory of exactly its size (hipHostMalloc).
    torch's pinned allocator rounds every block up to a power of two, so tens of GiB of expert
    banks would take up to twice their size; this allocation is freed (hipHostFree) when the
    last tensor viewing it is gone, and left to the process's exit otherwise."""
    shape = tuple(int(s) for s in shape)
    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    if nbytes == 0:
        return torch.empty(shape, dtype=dtype, pin_memory=True)
    rt = _hip_runtime()
    ptr = ctypes.c_void_p()
    rc = rt.hipHostMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes), ctypes.c_uint(0))
    if rc != 0 or not ptr.value:
        raise RuntimeError(f"hipHostMalloc of {nbytes} bytes failed (hipError {rc})")
    buf = (ctypes.c_uint8 * nbytes).from_address(ptr.value)
    fin = weakref.finalize(buf, rt.hipHostFree, ptr.value)
    fin.atexit = False
    return torch.frombuffer(buf, dtype=torch.uint8).view(dtype).view(shape)


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
