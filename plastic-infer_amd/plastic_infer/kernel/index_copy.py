"""Row index-copy entry points (expert slots <- pinned host banks, slot <-> slot moves).

  fast_index_copy        device-planned row copy kernel; same contract as the reference's
                         fast_index_copy_jit (src/plastic_infer/kernel/fast_index_copy.py:124-186):
                         dst[dst_indices[i]] = src[src_indices[i]] for i < n, n optionally read
                         from a device int64 [1] tensor. src may be a pinned host tensor (read
                         by the kernel through the device mapping of pinned memory).
  fast_index_copy_multi  the same rows for several banks in one launch
                         (src/plastic_infer/kernel/fast_index_copy.py:190-243).
  copy_rows_async        host-planned rows moved by the DMA engines with hipMemcpyAsync on a
                         given stream, consecutive runs merged into one transfer.
"""

from __future__ import annotations

import math
from typing import Sequence

import numpy as np
import torch

from .. import _native as N


_DEV_BASE: dict[tuple[int, int], int] = {}


def device_ptr(t: torch.Tensor) -> int:
    """Address at which kernels reach `t`: device tensors as is, pinned host tensors through
    their device mapping (pageable host tensors are rejected). The mapping of a pinned
    allocation is looked up once per (base address, size) and reused for every view of it, so
    a call over hundreds of chunk views of one pinned buffer costs one runtime lookup."""
    import ctypes

    if t.device.type == "cpu":
        st = t.untyped_storage()
        key = (st.data_ptr(), st.nbytes())
        base = _DEV_BASE.get(key)
        if base is None:
            out = ctypes.c_void_p()
            N.call("pia_device_pointer", key[0], ctypes.byref(out))
            base = int(out.value or 0)
            if len(_DEV_BASE) >= 4096:
                _DEV_BASE.clear()
            _DEV_BASE[key] = base
        return base + (t.data_ptr() - key[0])
    out = ctypes.c_void_p()
    N.call("pia_device_pointer", t.data_ptr(), ctypes.byref(out))
    return int(out.value or 0)


def _row_bytes(t: torch.Tensor) -> int:
    return math.prod(t.shape[1:]) * t.element_size()


def _check_rows_tensor(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.type == "cpu":
        if not t.is_pinned():
            raise ValueError(f"{name} is a pageable host tensor; host banks must be pinned")
    else:
        N.require_device(t, names=(name,))


def fast_index_copy(dst: torch.Tensor, dst_indices: torch.Tensor, src: torch.Tensor,
                    src_indices: torch.Tensor, num_indices: torch.Tensor | None = None) -> None:
    """Copy rows src[src_indices] -> dst[dst_indices] on the current stream of dst's device.

    dst/src: [rows, ...] banks with equal per-row bytes; indices int32/int64 device tensors of
    equal shape; num_indices: optional device int64 [1] valid-length override.
    """
    dev = N.require_device(dst, dst_indices, src_indices,
                           names=("dst", "dst_indices", "src_indices"))
    _check_rows_tensor("src", src)
    _check_rows_tensor("dst", dst)
    if _row_bytes(dst) != _row_bytes(src):
        raise ValueError("dst and src rows must have the same byte size")
    if dst_indices.shape != src_indices.shape or dst_indices.dtype != src_indices.dtype:
        raise ValueError("index tensors must share shape and dtype")
    if dst_indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("indices must be int32 or int64")
    if num_indices is not None:
        N.require_device(num_indices, names=("num_indices",))
        if num_indices.dtype != torch.int64 or num_indices.numel() != 1:
            raise ValueError("num_indices must be a device int64 [1] tensor")
    n = dst_indices.numel()
    if n == 0:
        return
    N.call("pia_index_copy_rows", dst.data_ptr(), dst_indices.contiguous().data_ptr(),
           dst.shape[0], src.data_ptr(), src_indices.contiguous().data_ptr(), src.shape[0], n,
           N.ptr(num_indices), _row_bytes(dst), 1 if dst_indices.dtype == torch.int32 else 0,
           N.stream_of(dev))


def fast_index_copy_multi(dst_ptrs: torch.Tensor, src_ptrs: torch.Tensor,
                          feat_bytes: torch.Tensor, dst_indices: torch.Tensor,
                          src_indices: torch.Tensor, num_indices: torch.Tensor | None = None) -> None:
    """One launch copying the same (dst_indices, src_indices) rows for every bank; per-bank
    base addresses and row bytes are device int64 [num_banks] tensors (row bytes % 16 == 0,
    16-byte aligned bases; the caller validates them when building the descriptor)."""
    dev = N.require_device(dst_ptrs, src_ptrs, feat_bytes, dst_indices, src_indices,
                           names=("dst_ptrs", "src_ptrs", "feat_bytes", "dst_indices", "src_indices"))
    for name, t in (("dst_ptrs", dst_ptrs), ("src_ptrs", src_ptrs), ("feat_bytes", feat_bytes)):
        if t.dtype != torch.int64 or t.numel() != dst_ptrs.numel():
            raise ValueError(f"{name} must be int64 [num_banks]")
    if dst_indices.shape != src_indices.shape or dst_indices.dtype != src_indices.dtype:
        raise ValueError("index tensors must share shape and dtype")
    n = dst_indices.numel()
    if n == 0:
        return
    N.call("pia_index_copy_rows_multi", dst_ptrs.data_ptr(), src_ptrs.data_ptr(),
           feat_bytes.data_ptr(), dst_ptrs.numel(), dst_indices.contiguous().data_ptr(),
           src_indices.contiguous().data_ptr(), n, N.ptr(num_indices),
           1 if dst_indices.dtype == torch.int32 else 0, N.stream_of(dev))


def _host_rows(x: Sequence[int] | np.ndarray | torch.Tensor) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        if x.device.type != "cpu":
            raise ValueError("row plans of copy_rows_async are host arrays")
        x = x.numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64))


def copy_rows_async(dst: torch.Tensor, dst_rows, src: torch.Tensor, src_rows,
                    stream: torch.cuda.Stream | None = None) -> int:
    """hipMemcpyAsync rows src[src_rows[i]] -> dst[dst_rows[i]] on `stream` (default: the
    current stream of the device involved); runs of consecutive rows are merged. dst/src are
    device tensors or pinned host tensors with equal row bytes. Returns the number of copies
    issued. The caller orders consumers after the copies (events / stream waits)."""
    _check_rows_tensor("dst", dst)
    _check_rows_tensor("src", src)
    if _row_bytes(dst) != _row_bytes(src):
        raise ValueError("dst and src rows must have the same byte size")
    dr, sr = _host_rows(dst_rows), _host_rows(src_rows)
    if dr.shape != sr.shape or dr.ndim != 1:
        raise ValueError("dst_rows and src_rows must be 1-D of equal length")
    if dr.size and (dr.max() >= dst.shape[0] or sr.max() >= src.shape[0]):
        raise IndexError("row index out of range")
    dev = dst.device if dst.device.type == "cuda" else src.device
    if dev.type != "cuda":
        raise ValueError("copy_rows_async needs a device tensor on one side")
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    issued = np.zeros(1, dtype=np.int64)
    N.call("pia_copy_rows_async", dst.data_ptr(), dr.ctypes.data, src.data_ptr(), sr.ctypes.data,
           dr.size, _row_bytes(dst), issued.ctypes.data, s.cuda_stream)
    return int(issued[0])
