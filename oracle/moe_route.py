"""ORACLE (test infrastructure only): CPU restatement of the reference's MoE routing, permute
plan and combine."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def fused_topk(logits: torch.Tensor, topk: int, renormalize: bool = True
               ) -> tuple[torch.Tensor, torch.Tensor]:
    """reference src/plastic_infer/moe/fused.py:11-30: softmax over fp32 logits, top-k of the
    probabilities, optional renormalisation; ids int32."""
    probs = torch.softmax(logits.float(), dim=-1)
    w, ids = torch.topk(probs, topk, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.contiguous(), ids.to(torch.int32).contiguous()


def topk_route(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """reference src/plastic_infer/exec/moe.py:19-38: top-k of the logits, softmax of the
    selected logits in fp32, cast back to the logits dtype; ids int64."""
    top, ids = torch.topk(logits, k, dim=-1)
    return ids, F.softmax(top.float(), dim=-1).to(logits.dtype)


def max_num_tokens_padded(numel: int, num_experts: int, block_size: int) -> int:
    """reference src/plastic_infer/kernel/triton/moe_align.py:228-232."""
    if numel < num_experts + 1:
        return numel * block_size
    return numel + (num_experts + 1) * (block_size - 1)


def moe_align_block_size(topk_ids, block_size: int, num_experts: int):
    """Permute plan with the semantics of reference src/plastic_infer/kernel/triton/moe_align.py:9-20:
    effective_E = num_experts + 1; count[e]; cumsum padded to multiples of block_size;
    expert_ids[b] = owner of block b; sorted_token_ids[cumsum[e] + r] = r-th route of e;
    all other entries = numel. Within an expert routes are in ascending flattened index — the
    order nonzero() yields in moe_forward_sparse (src/plastic_infer/exec/moe.py:149); the
    reference's GPU kernel leaves that order unspecified. expert_ids past the used blocks are
    -1 (unwritten in the reference). Returns numpy (sorted_ids, expert_ids, npp, route_pos)."""
    ids = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    numel = ids.size
    E_eff = num_experts + 1
    mpad = max_num_tokens_padded(numel, num_experts, block_size)
    valid = (ids >= 0) & (ids < E_eff)
    counts = np.bincount(ids[valid], minlength=E_eff).astype(np.int64)
    padded = (counts + block_size - 1) // block_size * block_size
    cumsum = np.concatenate([[0], np.cumsum(padded)])
    npp = int(cumsum[-1])
    sorted_ids = np.full(mpad, numel, dtype=np.int32)
    expert_ids = np.full((mpad + block_size - 1) // block_size, -1, dtype=np.int32)
    route_pos = np.full(numel, -1, dtype=np.int32)
    for e in range(E_eff):
        routes = np.nonzero(ids == e)[0]            # ascending route index
        base = int(cumsum[e])
        sorted_ids[base:base + routes.size] = routes
        route_pos[routes] = base + np.arange(routes.size)
        expert_ids[base // block_size:(base + int(padded[e])) // block_size] = e
    return sorted_ids, expert_ids, npp, route_pos


def permute(hidden: torch.Tensor, sorted_ids: np.ndarray, npp: int, topk: int) -> torch.Tensor:
    """x_perm[r] = hidden[sorted_ids[r] // topk] for r < npp; sentinel rows are zero.
    The per-expert hidden[rows] gather of reference src/plastic_infer/exec/moe.py:150-153."""
    numel = hidden.shape[0] * topk
    out = torch.zeros(npp, hidden.shape[1], dtype=hidden.dtype)
    r = np.asarray(sorted_ids[:npp], dtype=np.int64)
    real = r < numel
    out[torch.from_numpy(np.nonzero(real)[0])] = hidden[torch.from_numpy(r[real] // topk)]
    return out


def unpermute(y: torch.Tensor, route_pos: np.ndarray, weights, num_tokens: int, topk: int,
              out_dtype: torch.dtype) -> torch.Tensor:
    """out[t] = cast(sum_{s<k} w[t,s] * y[route_pos[t*k+s]]) with fp32 accumulation in slot
    order, multiply and add each rounded to fp32 (moe_sum_reduce with the GEMM2 routing
    weight: reference src/plastic_infer/kernel/triton/fused_moe.py:111-153,292-294; the combine
    of src/plastic_infer/exec/moe.py:155-158). weights None means 1."""
    yf = y.float().numpy()
    H = yf.shape[1]
    w = None if weights is None else np.asarray(weights, dtype=np.float32).reshape(num_tokens, topk)
    acc = np.zeros((num_tokens, H), dtype=np.float32)
    pos = np.asarray(route_pos, dtype=np.int64).reshape(num_tokens, topk)
    for s in range(topk):
        rows = pos[:, s]
        ok = rows >= 0
        contrib = np.zeros((num_tokens, H), dtype=np.float32)
        contrib[ok] = yf[rows[ok]]
        if w is not None:
            contrib = contrib * w[:, s:s + 1]
        acc = np.where(ok[:, None], acc + contrib, acc).astype(np.float32)
    return torch.from_numpy(acc).to(out_dtype)


def sum_reduce(inp: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """reference src/plastic_infer/kernel/triton/fused_moe.py:111-153: out[t] = sum_k in[t,k],
    fp32 accumulation in k order, cast once."""
    T, k, H = inp.shape
    pos = np.arange(T * k, dtype=np.int64)
    return unpermute(inp.reshape(T * k, H), pos, None, T, k, out_dtype)


def moe_forward_sparse(hidden: torch.Tensor, experts: dict, expert_ids: torch.Tensor,
                       weights: torch.Tensor) -> torch.Tensor:
    """reference src/plastic_infer/exec/moe.py:127-160 in the inputs' dtype: for each expert in
    the dict's order, the (token, slot) pairs routed to it in nonzero() order, the SwiGLU MLP
    silu(x w1^T) * (x w3^T) w2^T of their rows, times the weights, index_add_ into the output
    (so with bf16 storage every product and every running sum is rounded to bf16)."""
    out = torch.zeros_like(hidden)
    for eid, w in experts.items():
        pairs = (expert_ids == eid).nonzero()
        if pairs.shape[0] == 0:
            continue
        rows = pairs[:, 0]
        wts = weights[rows, pairs[:, 1]].unsqueeze(1)
        x = hidden[rows]
        inter = F.silu(F.linear(x, w.w1)) * F.linear(x, w.w3)
        out.index_add_(0, rows, F.linear(inter, w.w2) * wts)
    return out
