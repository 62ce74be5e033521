"""Fused-MoE routing front end with the reference's signatures (src/plastic_infer/moe/fused.py).

  fused_topk            :11-45  softmax over all experts -> top-k -> renormalise; fp32 weights,
                                int32 ids; rows >= num_token_non_padded get ids -1
  moe_align_block_size  :48-94  (sorted_token_ids, expert_ids, num_tokens_post_pad)
Both run as HIP kernels. The permute plan orders routes inside an expert by ascending
flattened route index (deterministic; the reference's atomic-based order is not).
"""

from __future__ import annotations

import torch

from .. import _native as N
from ..kernel.moe_ops import moe_align_block_size as _align
from ..kernel.moe_ops import moe_topk


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int,
               renormalize: bool, num_token_non_padded: torch.Tensor | int | None = None
               ) -> tuple[torch.Tensor, torch.Tensor]:
    """(topk_weights fp32 [T, k], topk_ids int32 [T, k])."""
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    N.require_device(gating_output, names=("gating_output",))
    n_np = None
    if num_token_non_padded is not None:
        n_np = int(num_token_non_padded.item()) if isinstance(num_token_non_padded, torch.Tensor) \
            else int(num_token_non_padded)
    return moe_topk(gating_output, topk, renormalize=renormalize, mode=0,
                    num_token_non_padded=n_np)


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int
                         ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Pad each expert's route count to a multiple of block_size and lay routes out
    expert-contiguously. Sentinel = topk_ids.numel(); ids in [0, num_experts] are routed
    (num_experts itself is the extra sentinel expert of the fused-MoE convention)."""
    return _align(topk_ids, block_size, num_experts)


__all__ = ["fused_topk", "moe_align_block_size"]
