"""The reference's index-copy entry points (src/plastic_infer/kernel/fast_index_copy.py:124-243)
under their own names, on the HIP row-copy kernels of this package. The launch tuning knobs of
the reference's templated CUDA kernels (worker threads, blocks) have no counterpart and are
accepted and ignored; the priority-gated mode belongs to the CPU-executor plumbing, which this
build does not include, and is rejected.
"""

from __future__ import annotations

import math
import os

import torch

from .index_copy import fast_index_copy, fast_index_copy_multi

DEFAULT_NUM_BLOCKS = 4
SKIP_FAST_INDEX_COPY_ENV = "FREETOKEN_SKIP_FAST_INDEX_COPY"
_TRUE_VALUES = {"1", "true", "yes", "on"}


def _skip_fast_index_copy_enabled() -> bool:
    """Ablation switch of the reference: the copies become no-ops (bookkeeping unchanged)."""
    return os.getenv(SKIP_FAST_INDEX_COPY_ENV, "").strip().lower() in _TRUE_VALUES


def _require_feature_alignment(feature_size: int) -> None:
    if feature_size % 128 != 0:
        raise ValueError(
            f"fast_index_copy: feature byte size {feature_size} must be a multiple of 128"
        )


def fast_index_copy_jit(dst: torch.Tensor, dst_indices: torch.Tensor, src: torch.Tensor,
                        src_indices: torch.Tensor, num_indices: torch.Tensor | None = None, *,
                        worker_threads: int | None = None, worker_feature_size: int = 2048,
                        num_block: int | None = None, priority: str | None = None,
                        sync_flag: torch.Tensor | None = None) -> None:
    """Rows src[src_indices] -> dst[dst_indices] of one bank, on the current stream;
    ``num_indices`` (device int64 [1]) optionally caps the count on device."""
    if priority is not None or sync_flag is not None:
        raise NotImplementedError("priority-gated copies are not part of this build")
    if math.prod(src.shape[1:]) != math.prod(dst.shape[1:]):
        raise AssertionError("dst and src rows differ in size")
    if _skip_fast_index_copy_enabled():
        return
    _require_feature_alignment(math.prod(dst.shape[1:]) * dst.element_size())
    if dst_indices.shape != src_indices.shape:
        raise AssertionError("index shape mismatch")
    fast_index_copy(dst, dst_indices, src, src_indices, num_indices)


def fast_index_copy_multi_jit(dst_ptrs: torch.Tensor, src_ptrs: torch.Tensor,
                              feat_bytes: torch.Tensor, dst_indices: torch.Tensor,
                              src_indices: torch.Tensor, num_indices: torch.Tensor | None = None,
                              *, num_threads: int = 1024, blocks_per_bank: int = 8) -> None:
    """The same rows of every bank in one launch; per-bank base addresses and row bytes are
    device int64 [num_banks] tensors (row bytes % 16 == 0, 16-byte aligned bases)."""
    if _skip_fast_index_copy_enabled():
        return
    fast_index_copy_multi(dst_ptrs, src_ptrs, feat_bytes, dst_indices, src_indices, num_indices)
