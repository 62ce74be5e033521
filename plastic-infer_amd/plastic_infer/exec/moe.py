"""MoE routing and the sparse routed forward with the reference's call signatures.

  topk_route          reference src/plastic_infer/exec/moe.py:19-38 — top-k of the logits,
                      weights = softmax of the selected logits (fp32 math, cast to logits dtype),
                      ids int64. Ties between equal logits go to the lower expert index.
  moe_forward_sparse  reference src/plastic_infer/exec/moe.py:127-160 — per-expert mini-batches
                      and a weighted combine. Here: one HIP permute plan (stable counting sort,
                      within an expert in ascending (token, slot) order, the order nonzero()
                      gives the reference), one permute kernel, one GEMM group per resident
                      expert on its contiguous rows, one unpermute kernel (fp32 accumulation).
  moe_forward_v1      reference src/plastic_infer/exec/moe.py:41-82 — the dense-bank variant
                      (w1 [E, H, I], w2 [E, I, H], one up projection, SiLU): the same permute
                      plan, permute and unpermute, with the two GEMMs per expert in between.
  swiglu_mlp          the expert MLP (plain library GEMMs; expert math is not part of the
                      data path this package accelerates).

The reference's per-token loops (moe_forward_reference, moe_forward_reference_swiglu) are its
tests' ground truth; the tests here restate them next to the cases that use them.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _native as N
from ..kernel.moe_ops import moe_align_block_size, moe_permute, moe_topk, moe_unpermute
from ..store.experts import ExpertWeights


def topk_route(router_logits: torch.Tensor, k: int = 2) -> tuple[torch.Tensor, torch.Tensor]:
    """(expert_ids int64 [T, k], weights [T, k] in the logits' dtype)."""
    w, ids = moe_topk(router_logits, k, renormalize=True, mode=1)
    return ids.to(torch.int64), w.to(router_logits.dtype)


def swiglu_mlp(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
               w3: torch.Tensor) -> torch.Tensor:
    """silu(x @ w1^T) * (x @ w3^T) @ w2^T."""
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w3), w2)


def _route_rows(hidden: torch.Tensor, expert_ids: torch.Tensor, num_experts: int):
    """Permute plan (block 1: each expert's rows exactly contiguous), the permuted rows and each
    expert's row count (one host read of the routed ids; the plan itself stays on the device)."""
    k = expert_ids.shape[1]
    ids32 = expert_ids.to(torch.int32)
    sorted_ids, _, npp, route_pos = moe_align_block_size(ids32, 1, num_experts,
                                                        return_route_pos=True)
    x_perm = moe_permute(hidden, sorted_ids, npp, k, route_pos=route_pos)
    counts = torch.bincount(ids32.view(-1).clamp(min=-1).add(1), minlength=num_experts + 2)
    return x_perm, route_pos, counts[1:num_experts + 2].cpu().tolist()


def moe_forward_v1(hidden: torch.Tensor, expert_w1: torch.Tensor, expert_w2: torch.Tensor,
                   expert_ids: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_s weights[t, s] * silu(hidden[t] @ w1[e]) @ w2[e], e = expert_ids[t, s];
    expert_w1 [E, H, I], expert_w2 [E, I, H] (reference src/plastic_infer/exec/moe.py:41-82)."""
    N.require_device(hidden, expert_w1, expert_w2, expert_ids, weights,
                     names=("hidden", "expert_w1", "expert_w2", "expert_ids", "weights"))
    T, H = hidden.shape
    k = expert_ids.shape[1]
    E = expert_w1.shape[0]
    if expert_w1.dim() != 3 or expert_w2.shape != (E, expert_w1.shape[2], H) or \
            expert_w1.shape[1] != H:
        raise ValueError(f"expert_w1 must be [E, {H}, I] and expert_w2 [E, I, {H}], got "
                         f"{tuple(expert_w1.shape)} and {tuple(expert_w2.shape)}")
    if T == 0:
        return torch.zeros_like(hidden)
    x_perm, route_pos, counts = _route_rows(hidden, expert_ids, E)
    y = torch.zeros_like(x_perm)
    start = 0
    for e in range(E):
        n = counts[e]
        if n:
            y[start:start + n] = F.silu(x_perm[start:start + n] @ expert_w1[e]) @ expert_w2[e]
        start += n
    return moe_unpermute(y, route_pos, weights.to(torch.float32).contiguous(), T, k)


def moe_forward_sparse(hidden: torch.Tensor, experts: dict[int, ExpertWeights],
                       expert_ids: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_s weights[t, s] * expert_{ids[t,s]}(hidden[t]) over the routed experts
    present in `experts` (others contribute nothing)."""
    dev = N.require_device(hidden, expert_ids, weights, names=("hidden", "expert_ids", "weights"))
    T, H = hidden.shape
    k = expert_ids.shape[1]
    if T == 0 or not experts:
        return torch.zeros_like(hidden)
    num_experts = max(experts) + 1
    x_perm, route_pos, counts = _route_rows(hidden, expert_ids, num_experts)
    y = torch.zeros_like(x_perm)
    start = 0
    for e in range(num_experts + 1):
        n = counts[e]
        w = experts.get(e)
        if n and w is not None:
            y[start:start + n] = swiglu_mlp(x_perm[start:start + n], w.w1, w.w2, w.w3)
        start += n
    return moe_unpermute(y, route_pos, weights.to(torch.float32).contiguous(), T, k)


__all__ = ["topk_route", "swiglu_mlp", "moe_forward_v1", "moe_forward_sparse"]
