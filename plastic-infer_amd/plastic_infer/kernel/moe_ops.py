"""MoE routing / permutation entry points over the HIP library.

  moe_topk              softmax-topk-renormalise router (reference: src/plastic_infer/moe/fused.py:11-30)
                        and the topk-then-softmax variant (src/plastic_infer/exec/moe.py:19-38)
  moe_align_block_size  permute plan (src/plastic_infer/moe/fused.py:48-94, semantics of
                        src/plastic_infer/kernel/triton/moe_align.py:9-20,216-239) with a
                        deterministic within-expert order (ascending flattened route index)
  moe_permute           hidden rows -> expert-contiguous rows
  moe_unpermute         weighted combine back to token order, fp32 accumulation
  moe_sum_reduce        out[t] = sum_k in[t, k] (src/plastic_infer/kernel/moe_impl.py:169-197)
"""

from __future__ import annotations

import torch

from .. import _native as N


def max_num_tokens_padded(numel: int, num_experts: int, block_size: int) -> int:
    """Buffer length of sorted_token_ids, sized as the reference sizes it
    (src/plastic_infer/kernel/triton/moe_align.py:228-232)."""
    if numel < num_experts + 1:
        return numel * block_size
    return numel + (num_experts + 1) * (block_size - 1)


def moe_topk(logits: torch.Tensor, topk: int, renormalize: bool = True, mode: int = 0,
             num_token_non_padded: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (weights fp32 [T, k], ids int32 [T, k]).

    mode 0: p = softmax(float(logits)); top-k of p; weights /= their sum when renormalize.
    mode 1: top-k of the logits; weights = softmax over the selected logits.
    Ties between equal logits go to the lower expert index.
    """
    dev = N.require_device(logits, names=("logits",))
    if logits.dim() != 2:
        raise ValueError("logits must be [num_tokens, num_experts]")
    logits = logits.contiguous()
    T, E = logits.shape
    if not 0 < topk <= min(E, 64):
        raise ValueError(f"topk must be in [1, min(num_experts, 64)], got {topk}")
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    if T:
        N.call("pia_moe_topk", w.data_ptr(), ids.data_ptr(), logits.data_ptr(),
               N.dtype_code(logits.dtype), T, E, topk, 1 if renormalize else 0, mode,
               -1 if num_token_non_padded is None else int(num_token_non_padded),
               N.stream_of(dev))
    return w, ids


def moe_topk_align(logits: torch.Tensor, topk: int, block_size: int, renormalize: bool = True,
                   mode: int = 0, num_token_non_padded: int | None = None):
    """moe_topk then moe_align_block_size on its ids, in one call (two launches for large
    plans: the router kernel also counts the plan's per-chunk experts).
    Returns (weights, ids, sorted_token_ids, expert_ids, num_tokens_post_pad, route_pos)."""
    dev = N.require_device(logits, names=("logits",))
    if logits.dim() != 2:
        raise ValueError("logits must be [num_tokens, num_experts]")
    logits = logits.contiguous()
    T, E = logits.shape
    if not 0 < topk <= min(E, 64):
        raise ValueError(f"topk must be in [1, min(num_experts, 64)], got {topk}")
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    numel = T * topk
    mpad = max_num_tokens_padded(numel, E, block_size)
    sorted_ids = torch.empty(mpad, dtype=torch.int32, device=dev)
    expert_ids = torch.empty((mpad + block_size - 1) // block_size, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    route_pos = torch.empty(numel, dtype=torch.int32, device=dev)
    ws_bytes = N.query("pia_moe_align_workspace_bytes", E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    N.call("pia_moe_topk_align", w.data_ptr(), ids.data_ptr(), logits.data_ptr(),
           N.dtype_code(logits.dtype), T, E, topk, 1 if renormalize else 0, mode,
           -1 if num_token_non_padded is None else int(num_token_non_padded),
           sorted_ids.data_ptr(), expert_ids.data_ptr(), npp.data_ptr(), route_pos.data_ptr(),
           block_size, mpad, ws.data_ptr(), ws_bytes, N.stream_of(dev))
    return w, ids, sorted_ids, expert_ids, npp, route_pos


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         return_route_pos: bool = False):
    """(sorted_token_ids, expert_ids, num_tokens_post_pad[, route_pos]).

    topk_ids: int32, any shape (flattened in row-major order; route index i = t*k + s).
    sorted_token_ids: int32 [max_num_tokens_padded], sentinel = numel.
    expert_ids: int32 [ceil(max_num_tokens_padded / block_size)], -1 past the used blocks.
    route_pos: int32 [numel], row of each route in sorted order (-1 if dropped).
    """
    dev = N.require_device(topk_ids, names=("topk_ids",))
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    ids = topk_ids.contiguous().view(-1)
    numel = ids.numel()
    mpad = max_num_tokens_padded(numel, num_experts, block_size)
    sorted_ids = torch.empty(mpad, dtype=torch.int32, device=dev)
    expert_ids = torch.empty((mpad + block_size - 1) // block_size, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    route_pos = torch.empty(numel, dtype=torch.int32, device=dev) if return_route_pos else None
    ws_bytes = N.query("pia_moe_align_workspace_bytes", num_experts)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    N.call("pia_moe_align_block_size", sorted_ids.data_ptr(), expert_ids.data_ptr(),
           npp.data_ptr(), N.ptr(route_pos), ids.data_ptr() if numel else None, numel,
           num_experts, block_size, mpad, ws.data_ptr(), ws_bytes, N.stream_of(dev))
    if return_route_pos:
        return sorted_ids, expert_ids, npp, route_pos
    return sorted_ids, expert_ids, npp


def moe_permute(hidden: torch.Tensor, sorted_token_ids: torch.Tensor,
                num_tokens_post_pad: torch.Tensor, topk: int,
                out: torch.Tensor | None = None,
                route_pos: torch.Tensor | None = None) -> torch.Tensor:
    """x_perm[r] = hidden[sorted_token_ids[r] // topk] for r < num_tokens_post_pad and
    sorted_token_ids[r] < numel. Output has sorted_token_ids.numel() rows; padding rows
    (sentinel ids) and rows past num_tokens_post_pad are left as allocated (consumers skip
    sentinel rows). Bit-exact. With route_pos (moe_align_block_size's inverse map) every token
    row is read once and written to all its routes."""
    dev = N.require_device(hidden, sorted_token_ids, num_tokens_post_pad,
                           names=("hidden", "sorted_token_ids", "num_tokens_post_pad"))
    if route_pos is not None:
        N.require_device(route_pos, names=("route_pos",))
        if route_pos.dtype != torch.int32 or route_pos.numel() != hidden.shape[0] * topk:
            raise ValueError("route_pos must be int32 [num_tokens * topk]")
        route_pos = route_pos.contiguous()
    if hidden.dim() != 2 or hidden.stride(1) != 1:
        raise ValueError("hidden must be [T, H] with contiguous rows")
    T, H = hidden.shape
    rows = sorted_token_ids.numel()
    if out is None:
        out = torch.empty(rows, H, dtype=hidden.dtype, device=dev)
    elif out.shape != (rows, H) or out.dtype != hidden.dtype or not out.is_contiguous():
        raise ValueError("out must be contiguous [len(sorted_token_ids), H] of hidden's dtype")
    eb = hidden.element_size()
    N.call("pia_moe_permute", out.data_ptr(), hidden.data_ptr(), sorted_token_ids.data_ptr(),
           N.ptr(route_pos), num_tokens_post_pad.data_ptr(), rows, T * topk, topk, H * eb,
           hidden.stride(0) * eb, N.stream_of(dev))
    return out


def moe_unpermute(y: torch.Tensor, route_pos: torch.Tensor, topk_weights: torch.Tensor | None,
                  num_tokens: int, topk: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = sum_{s<k} w[t,s] * y[route_pos[t*k+s]] (fp32 accumulation in slot order,
    separately rounded multiply and add; weight 1 when topk_weights is None)."""
    dev = N.require_device(y, route_pos, names=("y", "route_pos"))
    if y.dim() != 2 or not y.is_contiguous():
        raise ValueError("y must be contiguous [rows, H]")
    H = y.shape[1]
    if route_pos.dtype != torch.int32 or route_pos.numel() != num_tokens * topk:
        raise ValueError("route_pos must be int32 [num_tokens * topk]")
    if topk_weights is not None:
        N.require_device(topk_weights, names=("topk_weights",))
        if topk_weights.dtype != torch.float32 or topk_weights.numel() != num_tokens * topk:
            raise ValueError("topk_weights must be float32 [num_tokens, topk]")
        topk_weights = topk_weights.contiguous()
    if out is None:
        out = torch.empty(num_tokens, H, dtype=y.dtype, device=dev)
    N.call("pia_moe_unpermute", out.data_ptr(), y.data_ptr(), y.shape[0],
           route_pos.contiguous().data_ptr(),
           N.ptr(topk_weights), num_tokens, topk, H, N.dtype_code(y.dtype), N.stream_of(dev))
    return out


def moe_sum_reduce(input: torch.Tensor, output: torch.Tensor) -> None:
    """output[t] = sum_k input[t, k] with fp32 accumulation (input [T, k, H], output [T, H])."""
    dev = N.require_device(input, output, names=("input", "output"))
    if not (input.is_contiguous() and output.is_contiguous()):
        raise ValueError("input and output must be contiguous")
    T, k, H = input.shape
    if output.shape != (T, H) or output.dtype != input.dtype:
        raise ValueError("output must be [T, H] of input's dtype")
    N.call("pia_moe_sum_reduce", output.data_ptr(), input.data_ptr(), T, k, H,
           N.dtype_code(input.dtype), N.stream_of(dev))


ACTIVATION_CODES = {"silu": 0, "gelu": 1, "gelu_tanh": 2}


def moe_expert_gemm(a: torch.Tensor, w: torch.Tensor, topk_weights: torch.Tensor | None,
                    sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                    num_tokens_post_pad: torch.Tensor, block_m: int, numel: int, a_div: int,
                    activation: str | None = None, mul_routed_weight: bool = False,
                    out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One GEMM of the fused experts FFN over a permute plan (block_m a multiple of 16).

    For every planned route r < numel of expert e: acc = a[r // a_div] . w[e]^T (fp32), then
    activation None: out[r] = round(acc * w_r); activation X: out[r, n] =
    round(X(round(acc[n] * w_r)) * round(acc[I + n] * w_r)) with I = w.shape[1] // 2.
    w_r = topk_weights.flat[r] when mul_routed_weight, else 1. out is [numel, N or I] unless given
    (a [*, N or I] view with unit column stride). workspace: optional device buffer reused
    across calls (pia_moe_expert_gemm_workspace_bytes of the plan)."""
    dev = N.require_device(a, w, sorted_token_ids, expert_ids, num_tokens_post_pad,
                           names=("a", "w", "sorted_token_ids", "expert_ids",
                                  "num_tokens_post_pad"))
    if a.dim() != 2 or a.stride(1) != 1:
        raise ValueError("a must be [rows, K] with contiguous rows")
    if w.dim() != 3 or not w.is_contiguous():
        raise ValueError("w must be contiguous [E, N, K]")
    if a.dtype != w.dtype:
        raise ValueError("a and w must share a dtype")
    E, n_rows, K = w.shape
    if a.shape[1] != K:
        raise ValueError(f"a has {a.shape[1]} columns, w expects K = {K}")
    if a_div <= 0 or a.shape[0] * a_div < numel:
        raise ValueError(f"a needs ceil(numel / a_div) = {-(-numel // max(a_div, 1))} rows")
    act = -1 if activation is None else ACTIVATION_CODES.get(activation)
    if act is None:
        raise ValueError(f"Unsupported activation: {activation}")
    out_cols = n_rows if act < 0 else n_rows // 2
    if out is None:
        out = torch.empty(numel, out_cols, dtype=a.dtype, device=dev)
    elif out.dim() != 2 or out.stride(1) != 1 or out.shape[1] != out_cols or \
            out.shape[0] < numel or out.dtype != a.dtype:
        raise ValueError(f"out must be [>= {numel}, {out_cols}] of a's dtype with unit column stride")
    if mul_routed_weight:
        if topk_weights is None or topk_weights.dtype != torch.float32 or \
                not topk_weights.is_contiguous() or topk_weights.numel() != numel:
            raise ValueError("topk_weights must be contiguous float32 with one weight per route")
        N.require_device(topk_weights, names=("topk_weights",))
    for name, t in (("sorted_token_ids", sorted_token_ids), ("expert_ids", expert_ids)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous int32")
    mpad = sorted_token_ids.numel()
    ws_bytes = N.query("pia_moe_expert_gemm_workspace_bytes", mpad, block_m)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    N.call("pia_moe_expert_gemm", out.data_ptr(), a.data_ptr(), w.data_ptr(),
           N.ptr(topk_weights) if mul_routed_weight else None, sorted_token_ids.data_ptr(),
           expert_ids.data_ptr(), num_tokens_post_pad.data_ptr(), mpad, block_m, numel, a_div,
           a.stride(0), E, n_rows, K, out.stride(0), act, 1 if mul_routed_weight else 0,
           N.dtype_code(a.dtype), workspace.data_ptr(),
           workspace.numel() * workspace.element_size(), N.stream_of(dev))
    return out
