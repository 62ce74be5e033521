"""Pins the fused-experts oracle (oracle/fused_experts.py) on the CPU.

1. fp32 storage: the oracle FFN behind the oracle router equals transformers'
   Qwen3MoeSparseMoeBlock (router softmax -> top-k -> renormalise, gate_up_proj [E, 2I, H] with the
   gate rows first, down_proj [E, H, I], weighted sum), for silu, gelu and gelu-tanh.
2. bf16 storage: the rounding points (first GEMM output, activation output, second GEMM output,
   the sum) match a torch.nn.functional.linear pipeline that rounds at the same points. A missing
   or extra rounding step changes about half of the elements; an fp32 summation-order difference
   changes a small fraction, so the bar is < 1 % differing elements, within one bf16 step.
3. Special cases: top_k 1 with weight 1 is the dense gated MLP; a zero up half gives exact zeros;
   apply_router_weight_on_input scales the first GEMM instead of the second.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.fused_experts as OF
import oracle.moe_route as OM

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig  # noqa: E402
from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock  # noqa: E402

HF_ACT = {"silu": "silu", "gelu": "gelu", "gelu_tanh": "gelu_pytorch_tanh"}


@pytest.mark.parametrize("activation", ["silu", "gelu", "gelu_tanh"])
def test_oracle_matches_hf_qwen3_moe_block(activation):
    torch.manual_seed(0)
    cfg = Qwen3MoeConfig(hidden_size=64, moe_intermediate_size=24, num_experts=8,
                         num_experts_per_tok=3, norm_topk_prob=True,
                         hidden_act=HF_ACT[activation])
    block = Qwen3MoeSparseMoeBlock(cfg).float().eval()
    with torch.no_grad():
        for p in block.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
        x = torch.randn(11, 64)
        ref = block(x[None])[0]
        logits = F.linear(x, block.gate.weight)
    w, ids = OM.fused_topk(logits, 3, True)
    out = OF.fused_experts(x, block.experts.gate_up_proj.detach(),
                           block.experts.down_proj.detach(), w, ids, activation)
    assert out.dtype == torch.float32
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5), (out - ref).abs().max()


def _torch_bf16_pipeline(x, w1, w2, tw, ids, activation, on_input):
    """Per route with torch's CPU bf16 linear (fp32 accumulation, one rounding)."""
    T, k = ids.shape
    I = w1.shape[1] // 2
    c2 = torch.zeros(T * k, I, dtype=x.dtype)
    c3 = torch.zeros(T, k, w2.shape[1], dtype=x.dtype)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            wr = float(tw[t, j])
            c1 = F.linear(x[t:t + 1].float(), w1[e].float())
            c1 = (c1 * (wr if on_input else 1.0)).to(x.dtype).float()
            g, u = c1[:, :I], c1[:, I:]
            a = {"silu": F.silu(g), "gelu": F.gelu(g),
                 "gelu_tanh": F.gelu(g, approximate="tanh")}[activation]
            h = (a * u).to(x.dtype)
            c2[t * k + j] = h[0]
            y = F.linear(h.float(), w2[e].float())
            c3[t, j] = (y * (1.0 if on_input else wr)).to(x.dtype)[0]
    acc = c3[:, 0].float()
    for j in range(1, k):
        acc = acc + c3[:, j].float()
    return acc.to(x.dtype), c2, c3


def _assert_mostly_equal(a: torch.Tensor, b: torch.Tensor, what: str):
    a, b = a.float(), b.float()
    diff = a != b
    frac = diff.float().mean().item()
    assert frac < 0.01, f"{what}: {frac:.4f} of elements differ"
    if diff.any():
        # a differing element is off by about one bf16 step of its magnitude
        rel = ((a - b).abs() / b.abs().clamp_min(1e-3))[diff].max().item()
        assert rel <= 2 ** -7 + 1e-6, f"{what}: relative step {rel}"


@pytest.mark.parametrize("activation,on_input", [("silu", False), ("gelu", True),
                                                 ("gelu_tanh", False)])
def test_oracle_bf16_rounding_points(activation, on_input):
    g = torch.Generator().manual_seed(1)
    T, H, I, E, k = 9, 128, 48, 6, 2
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.1).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    tw, ids = OM.fused_topk(logits, k, True)
    out, c2, c3 = OF.fused_experts(x, w1, w2, tw, ids, activation, on_input,
                                   return_intermediate=True)
    rout, rc2, rc3 = _torch_bf16_pipeline(x, w1, w2, tw, ids, activation, on_input)
    _assert_mostly_equal(torch.from_numpy(c2), rc2, "activation output")
    _assert_mostly_equal(torch.from_numpy(c3), rc3, "second GEMM output")
    _assert_mostly_equal(out, rout, "sum")


def test_oracle_topk1_is_dense_gated_mlp():
    g = torch.Generator().manual_seed(2)
    T, H, I = 7, 64, 32
    x = torch.randn(T, H, generator=g)
    gate, up, down = (torch.randn(I, H, generator=g), torch.randn(I, H, generator=g),
                      torch.randn(H, I, generator=g))
    w1 = torch.cat([gate, up], 0)[None]
    ref = F.linear(F.silu(F.linear(x, gate)) * F.linear(x, up), down)
    out = OF.fused_experts(x, w1, down[None], torch.ones(T, 1), torch.zeros(T, 1, dtype=torch.int32))
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-4)


def test_oracle_zero_up_half_gives_zero():
    g = torch.Generator().manual_seed(3)
    T, H, I, E = 5, 32, 16, 3
    w1 = torch.randn(E, 2 * I, H, generator=g).to(torch.bfloat16)
    w1[:, I:] = 0
    out = OF.fused_experts(torch.randn(T, H, generator=g).to(torch.bfloat16), w1,
                           torch.randn(E, H, I, generator=g).to(torch.bfloat16),
                           torch.rand(T, 2, generator=g), torch.randint(0, E, (T, 2), generator=g,
                                                                         dtype=torch.int32))
    assert bool((out == 0).all())


def test_oracle_weight_on_input_moves_the_weight():
    # silu is not linear: weighting the input of the activation changes the result, while for a
    # single route with weight 1 both placements agree exactly.
    g = torch.Generator().manual_seed(4)
    T, H, I, E = 4, 32, 16, 2
    x = torch.randn(T, H, generator=g)
    w1, w2 = torch.randn(E, 2 * I, H, generator=g), torch.randn(E, H, I, generator=g)
    ids = torch.zeros(T, 1, dtype=torch.int32)
    ones = torch.ones(T, 1)
    assert torch.equal(OF.fused_experts(x, w1, w2, ones, ids, "silu", True),
                       OF.fused_experts(x, w1, w2, ones, ids, "silu", False))
    half = ones * 0.5
    a = OF.fused_experts(x, w1, w2, half, ids, "silu", True)
    b = OF.fused_experts(x, w1, w2, half, ids, "silu", False)
    assert not torch.allclose(a, b, rtol=1e-3)
    # on input the weight scales gate and up: silu(0.5 g) * 0.5 u, then the down projection
    gg, uu = F.linear(x, w1[0, :I]), F.linear(x, w1[0, I:])
    ref = F.linear(F.silu(0.5 * gg) * (0.5 * uu), w2[0])
    assert torch.allclose(a, ref, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("activation", ["silu", "gelu", "gelu_tanh"])
def test_oracle_act_and_mul_matches_torch(activation):
    x = torch.randn(33, 2 * 40, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    g, u = x[:, :40].float(), x[:, 40:].float()
    a = {"silu": F.silu(g), "gelu": F.gelu(g), "gelu_tanh": F.gelu(g, approximate="tanh")}
    ref = (a[activation] * u).to(torch.bfloat16)
    _assert_mostly_equal(OF.act_and_mul(x, activation), ref, activation)
    assert np.isfinite(OF.act_and_mul(x, activation).float().numpy()).all()
