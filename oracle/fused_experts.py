"""ORACLE (test infrastructure only): CPU restatement of the reference's fused experts FFN
(src/plastic_infer/moe/fused.py:169-359: fused_experts_impl and fused_experts_decode_impl) and of
its *_and_mul activations (src/plastic_infer/kernel/triton/activation.py:63-113).

Per route r = t*k + j, expert e = topk_ids[t, j], weight w = topk_weights[t, j]:
  c1 = round(hidden[t] . w1[e]^T * (w if apply_router_weight_on_input else 1))      [2I]
       (fused_moe.py:260-302 / decode_moe.py:52-75: fp32 accumulator, weight multiply, cast)
  c2 = round(act(c1[:I]) * c1[I:])                                                    [I]
       (activation.py:86-113: halves read back as fp32, result cast)
  c3 = round(c2 . w2[e]^T * (w if not apply_router_weight_on_input else 1))          [H]
  out[t] = round(c3[t, 0] + c3[t, 1] + ... + c3[t, k-1])   fp32 sum in slot order
       (moe_sum_reduce, src/plastic_infer/kernel/triton/fused_moe.py:111-153)
round() is the storage dtype (bf16 / fp16 round to nearest even; identity for fp32). Each dot
product is the float64 sum of exact products rounded once to fp32; the GPU kernels accumulate in
fp32 in their own order, so parity with them is a tolerance, not bit equality.

Pinned by tests/test_oracle_experts.py against transformers' Qwen3MoeSparseMoeBlock (fp32
storage, silu / gelu / gelu-tanh), against a torch.nn.functional.linear pipeline with the same
bf16 rounding points, and against special cases (top_k 1 with weight 1 is the dense gated MLP; a
zero up half gives zero output; apply_router_weight_on_input moves the weight before the
activation).
"""

from __future__ import annotations

import numpy as np
import torch

ACTIVATIONS = ("silu", "gelu", "gelu_tanh")


def round_to(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """fp32 values rounded to `dtype` (nearest even) and widened back to fp32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == torch.float32:
        return x
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).float().numpy()


def act(g: np.ndarray, activation: str) -> np.ndarray:
    """act(g) in fp32: silu g/(1+exp(-g)); gelu 0.5 g (1 + erf(g/sqrt 2));
    gelu_tanh 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))."""
    t = torch.from_numpy(np.asarray(g, dtype=np.float32))
    if activation == "silu":
        y = t / (1.0 + torch.exp(-t))
    elif activation == "gelu":
        y = 0.5 * t * (1.0 + torch.erf(t * 0.7071067811865476))
    elif activation == "gelu_tanh":
        y = 0.5 * t * (1.0 + torch.tanh(0.7978845608028654 * (t + 0.044715 * t * t * t)))
    else:
        raise ValueError(f"Unsupported activation: {activation}")
    return y.numpy()


def act_and_mul(x: torch.Tensor, activation: str = "silu") -> torch.Tensor:
    """y = round(act(x[..., :d]) * x[..., d:]) in x's dtype (activation.py:86-113)."""
    d = x.shape[-1] // 2
    xf = x.float().numpy()
    y = act(xf[..., :d], activation) * xf[..., d:]
    return torch.from_numpy(round_to(y, x.dtype)).to(x.dtype)


def _dot_f32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """a [m, K] . w [N, K]^T as float64 sums rounded once to fp32."""
    return (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


def fused_experts(hidden: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                  activation: str = "silu", apply_router_weight_on_input: bool = False,
                  return_intermediate: bool = False):
    """out [T, H] in hidden's dtype; with return_intermediate also (c2 [T*k, I], c3 [T, k, H]) as
    fp32 arrays of the rounded values."""
    dt = hidden.dtype
    x = hidden.float().numpy()
    W1 = w1.float().numpy()
    W2 = w2.float().numpy()
    T, H = x.shape
    E, two_i, _ = W1.shape
    I = two_i // 2
    tw = topk_weights.float().numpy().astype(np.float32)
    ids = topk_ids.numpy().astype(np.int64)
    k = ids.shape[1]
    c2 = np.zeros((T * k, I), np.float32)
    c3 = np.zeros((T, k, H), np.float32)
    flat = ids.reshape(-1)
    for e in np.unique(flat):
        if e < 0 or e >= E:
            continue
        routes = np.nonzero(flat == e)[0]
        toks, slots = routes // k, routes % k
        wr = tw[toks, slots][:, None]
        one = np.float32(1.0)
        c1 = _dot_f32(x[toks], W1[e])
        c1 = round_to(c1 * (wr if apply_router_weight_on_input else one), dt)
        h = round_to(act(c1[:, :I], activation) * c1[:, I:], dt)
        c2[routes] = h
        y = _dot_f32(h, W2[e])
        c3[toks, slots] = round_to(y * (one if apply_router_weight_on_input else wr), dt)
    acc = c3[:, 0].copy()
    for j in range(1, k):
        acc = (acc + c3[:, j]).astype(np.float32)
    out = torch.from_numpy(round_to(acc, dt)).to(dt)
    if return_intermediate:
        return out, c2, c3
    return out
