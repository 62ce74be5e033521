"""ORACLE (test infrastructure only): CPU restatement of the reference's MoE decode step over
paged KV, one request per call.

Follows decode_step_moe_paged (reference src/plastic_infer/exec/runner_moe_paged.py:101-162)
with its routed FFN _moe_ffn / _decode_routed (src/plastic_infer/exec/runner_moe.py:108-146,
_MOE_RENORMALIZE = True, silu, weight on the output :37-39) and the helpers it calls:
rms_norm and qk_norm (src/plastic_infer/exec/attention.py:77-95), RoPE tables built in the model
dtype and applied in rotate-half form (:23-74), linear = x @ W^T (src/plastic_infer/exec/runner.py
:141-143), the KV write (_write_kv_layer, runner_paged.py:112-129) and paged attention with
causal=False (attention.py:151-190). The expert FFN reads the host banks directly (placement of
experts never changes the result, runner_moe_paged.py:9-11).

Composition only: the attention, routing and expert FFN are the oracle functions of
oracle/paged_kv.py, oracle/moe_route.py and oracle/fused_experts.py. The composition itself is
pinned in tests/test_oracle_decode_step.py against transformers' Qwen3MoeForCausalLM decoding
one token after a prefix, with the same weights (fp32).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import fused_experts as OF
from . import moe_route as OR
from . import paged_kv as OP


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """attention.py:77-80: x / sqrt(mean(x^2) + eps) * w, in x's dtype."""
    return x / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * w


def rope_tables(seq_len: int, head_dim: int, base: float, dtype: torch.dtype):
    """attention.py:52-74: inv_freq, positions and angles in `dtype`; cos/sin of [f, f]."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=dtype) / head_dim))
    t = torch.arange(seq_len, dtype=dtype)
    f = torch.outer(t, inv)
    emb = torch.cat((f, f), dim=-1)
    return emb.cos(), emb.sin()


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: int) -> torch.Tensor:
    """attention.py:23-49 for one position: x [heads, D]."""
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos[pos] + torch.cat([-x2, x1], dim=-1) * sin[pos]


def decode_step(weights: dict, cfg, banks: dict, k_pages: torch.Tensor, v_pages: torch.Tensor,
                tables: list[list[int]], pos: int, token: int, page_size: int,
                route_ids: list | None = None, router_logits: list | None = None
                ) -> torch.Tensor:
    """One decode token of one request at position `pos` (0-based; the request has pos tokens
    before it). tables[l] lists layer l's pages (covering pos + 1 tokens). k_pages / v_pages
    are updated in place with the new token's K / V. Returns logits [vocab] in the model dtype.
    weights: the reference's key names (CPU tensors); banks: per-layer gate_up [E, 2I, H] and
    down [E, H, I]; cfg: n_layers, n_heads, n_kv_heads, head_dim, n_experts_per_tok,
    max_seq_len, rope_base, qk_norm, dtype.
    route_ids[l] (optional, [k] ints): use these experts in layer l instead of this oracle's own
    top-k, with weights from this oracle's probabilities renormalised over them (a caller whose
    routing flipped on a near-tie of two logits follows the same experts).
    router_logits (optional list): receives each layer's router logits [E]."""
    dt = cfg.dtype
    Hq, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    cos, sin = rope_tables(cfg.max_seq_len, D, cfg.rope_base, dt)
    x = weights["embed_tokens.weight"][token].to(dt)[None]            # [1, H]
    for l in range(cfg.n_layers):
        p = f"layers.{l}."
        residual = x
        h = rms_norm(x, weights[p + "input_layernorm.weight"])
        q = F.linear(h, weights[p + "self_attn.q_proj.weight"]).view(Hq, D)
        k = F.linear(h, weights[p + "self_attn.k_proj.weight"]).view(Hkv, D)
        v = F.linear(h, weights[p + "self_attn.v_proj.weight"]).view(Hkv, D)
        if cfg.qk_norm:
            q = rms_norm(q, weights[p + "self_attn.q_norm.weight"])
            k = rms_norm(k, weights[p + "self_attn.k_norm.weight"])
        q, k = rope(q, cos, sin, pos), rope(k, cos, sin, pos)
        OP.write_kv_layer(tables[l], page_size, pos, k[None], v[None], k_pages, v_pages)
        attn = OP.paged_attention(q[None, None], k_pages, v_pages, tables[l], page_size,
                                  kv_num_tokens=pos + 1, causal=False)[0, 0]
        x = residual + F.linear(attn.reshape(1, Hq * D), weights[p + "self_attn.o_proj.weight"])
        residual = x
        h = rms_norm(x, weights[p + "post_attention_layernorm.weight"])
        logits = F.linear(h, weights[p + "mlp.router.weight"])
        if router_logits is not None:
            router_logits.append(logits[0])
        w, ids = OR.fused_topk(logits, cfg.n_experts_per_tok, renormalize=True)
        if route_ids is not None:
            ids = torch.as_tensor(route_ids[l], dtype=torch.int32).view(1, -1)
            probs = torch.softmax(logits.float(), dim=-1).gather(1, ids.long())
            w = probs / probs.sum(dim=-1, keepdim=True)
        routed = OF.fused_experts(h, banks["gate_up"][l], banks["down"][l], w, ids)
        x = residual + routed
    x = rms_norm(x, weights["norm.weight"])
    return F.linear(x, weights["lm_head.weight"])[0]
