"""Fused-MoE front end with the reference's signatures (src/plastic_infer/moe/fused.py).

  fused_topk                 :11-45   softmax over all experts -> top-k -> renormalise; fp32
                                      weights, int32 ids; rows >= num_token_non_padded get ids -1
  moe_align_block_size       :48-94   (sorted_token_ids, expert_ids, num_tokens_post_pad)
  fused_experts_impl         :169-273 routed gated-MLP FFN, result written over hidden_states
  fused_experts_decode_impl  :276-359 the same FFN into a new tensor
  FusedMoe                   :362-390 router + experts behind BaseMoeBackend
All run as HIP kernels. The permute plan orders routes inside an expert by ascending flattened
route index (deterministic; the reference's atomic-based order is not). Both FFN entry points
share one plan-driven path: moe_align_block_size, the first expert GEMM with the activation
fused into its epilogue, the second expert GEMM with the routing weight, moe_sum_reduce; the
rounding points are the reference's (first GEMM output, activation output, second GEMM output
and the sum are each rounded to the storage dtype; with fp32 storage there is no rounding).
"""

from __future__ import annotations

import torch

from .. import _native as N
from ..kernel.moe_ops import moe_align_block_size as _align
from ..kernel.moe_ops import moe_expert_gemm, moe_sum_reduce, moe_topk
from .base import BaseMoeBackend

# Plan block of the expert GEMMs: the kernel takes 16 planned routes per work item, so the
# finest block wastes the fewest padded rows when an expert serves only a few routes.
EXPERT_BLOCK_M = 16


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


def _check_ffn_args(hidden_states, w1, w2, topk_weights, topk_ids, activation):
    assert hidden_states.dim() == 2 and w1.dim() == 3 and w2.dim() == 3
    assert hidden_states.shape[1] == w1.shape[2], "Hidden size mismatch"
    assert w1.shape[0] == w2.shape[0], "Expert cache size mismatch"
    assert w1.shape[1] == 2 * w2.shape[2], "Intermediate size mismatch"
    assert w2.shape[1] == hidden_states.shape[1], "Output hidden size mismatch"
    assert topk_weights.shape == topk_ids.shape, "topk shape mismatch"
    assert topk_ids.shape[0] == hidden_states.shape[0], "Number of tokens mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert w2.is_contiguous(), "Expert weights2 must be contiguous"
    if activation not in {"silu", "gelu", "gelu_tanh"}:
        raise ValueError(f"Unsupported activation: {activation}")
    if hidden_states.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise NotImplementedError("expert GEMMs are built for bf16, fp16 and fp32 storage")
    assert w1.dtype == hidden_states.dtype and w2.dtype == hidden_states.dtype
    N.require_device(hidden_states, w1, w2, topk_weights, topk_ids,
                     names=("hidden_states", "w1", "w2", "topk_weights", "topk_ids"))


def routed_ffn_routes(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                      topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                      route_out: torch.Tensor, activation: str = "silu",
                      apply_router_weight_on_input: bool = False,
                      act_buffer: torch.Tensor | None = None) -> torch.Tensor:
    """The routed FFN of every route whose id is in [0, E), into route_out [T, k, H]: row
    (t, s) = w2[id] . act(w1[id] . x_t) times the routing weight, rounded to the storage dtype
    at the reference's points. Routes with id -1 are left untouched, so the routes of one
    token can be computed in several calls (e.g. experts already in HBM first, copied ones
    after their copies land) and summed once with moe_sum_reduce: the result is bit-identical
    to one call over all routes. act_buffer [T * k, I] may be shared between such calls."""
    M, H = hidden_states.shape
    E, two_i, _ = w1.shape
    k = topk_ids.shape[1]
    numel = M * k
    if numel == 0:
        return route_out
    if route_out.shape != (M, k, H) or not route_out.is_contiguous() \
            or route_out.dtype != hidden_states.dtype:
        raise ValueError(f"route_out must be a contiguous [{M}, {k}, {H}] tensor of the "
                         "hidden dtype")
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    weights = topk_weights.to(torch.float32).contiguous()
    sorted_ids, expert_ids, npp = _align(ids, EXPERT_BLOCK_M, E)
    dev = hidden_states.device
    ws = torch.empty(N.query("pia_moe_expert_gemm_workspace_bytes", sorted_ids.numel(),
                             EXPERT_BLOCK_M), dtype=torch.uint8, device=dev)
    if act_buffer is None:
        act_buffer = torch.empty(numel, two_i // 2, dtype=hidden_states.dtype, device=dev)
    moe_expert_gemm(hidden_states, w1, weights, sorted_ids, expert_ids, npp, EXPERT_BLOCK_M,
                    numel, k, activation=activation,
                    mul_routed_weight=apply_router_weight_on_input, out=act_buffer, workspace=ws)
    moe_expert_gemm(act_buffer, w2, weights, sorted_ids, expert_ids, npp, EXPERT_BLOCK_M, numel,
                    1, activation=None, mul_routed_weight=not apply_router_weight_on_input,
                    out=route_out.view(numel, H), workspace=ws)
    return route_out


def _routed_ffn(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                topk_weights: torch.Tensor, topk_ids: torch.Tensor, activation: str,
                apply_router_weight_on_input: bool, out: torch.Tensor) -> torch.Tensor:
    M, H = hidden_states.shape
    k = topk_ids.shape[1]
    if M * k == 0:
        return out
    route_out = torch.empty(M, k, H, dtype=hidden_states.dtype, device=hidden_states.device)
    routed_ffn_routes(hidden_states, w1, w2, topk_weights, topk_ids, route_out, activation,
                      apply_router_weight_on_input)
    moe_sum_reduce(route_out, out)
    return out


def fused_experts_impl(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                       topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                       activation: str = "silu",
                       apply_router_weight_on_input: bool = False) -> torch.Tensor:
    """Returns ``hidden_states`` itself, overwritten with the routed output (the reference's
    contract: a caller that still needs the input must read it first or pass a copy).
    w1 [E, 2I, H] (gate rows then up rows), w2 [E, H, I]; ids in [0, E)."""
    _check_ffn_args(hidden_states, w1, w2, topk_weights, topk_ids, activation)
    return _routed_ffn(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                       apply_router_weight_on_input, hidden_states)


def fused_experts_decode_impl(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                              topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                              activation: str = "silu",
                              apply_router_weight_on_input: bool = False) -> torch.Tensor:
    """The routed FFN into a new tensor (ids are expert or slot indices into w1 / w2)."""
    _check_ffn_args(hidden_states, w1, w2, topk_weights, topk_ids, activation)
    assert topk_weights.dtype == torch.float32
    assert topk_ids.dtype == torch.int32
    out = torch.empty_like(hidden_states)
    return _routed_ffn(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                       apply_router_weight_on_input, out)


class FusedMoe(BaseMoeBackend):
    def forward(self, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                gating_output: torch.Tensor, topk: int, renormalize: bool,
                activation: str = "silu",
                apply_router_weight_on_input: bool = False) -> torch.Tensor:
        topk_weights, topk_ids = fused_topk(hidden_states=hidden_states,
                                            gating_output=gating_output, topk=topk,
                                            renormalize=renormalize)
        return fused_experts_impl(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                                  apply_router_weight_on_input=apply_router_weight_on_input)


__all__ = ["fused_topk", "moe_align_block_size", "fused_experts_impl",
           "fused_experts_decode_impl", "routed_ffn_routes", "FusedMoe", "EXPERT_BLOCK_M"]
