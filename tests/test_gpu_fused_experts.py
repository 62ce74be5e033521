"""GPU parity of the grouped expert GEMMs, the *_and_mul activations and the fused experts FFN
against the oracle (oracle/fused_experts.py).

The GPU accumulates in fp32 in its own order (MFMA), so the bar is a tolerance: every rounded
intermediate agrees with the oracle's except for a small fraction of elements near a rounding
boundary (< 1 %, each within a few storage-dtype steps), and the FFN output is within 1e-2 of the
output's largest magnitude (the reference's own GPU-vs-CPU bar is 2e-2,
tests/test_cpu_moe_executor.py:86-119). With fp32 storage nothing is rounded, so every
intermediate and the output are held to 2e-5 of their largest magnitude (fp32 sums of up to
2048 products in two orders, and the activations' exp / erf / tanh to a few fp32 ulps).
"""

from __future__ import annotations

import pytest
import torch

import oracle.fused_experts as OF
import oracle.moe_route as OM
from plastic_infer.kernel import (
    gelu_and_mul,
    gelu_tanh_and_mul,
    moe_align_block_size,
    moe_expert_gemm,
    silu_and_mul,
)
from plastic_infer.moe.fused import (
    FusedMoe,
    fused_experts_decode_impl,
    fused_experts_impl,
    fused_topk,
)

pytestmark = pytest.mark.gpu

ACT = {"silu": silu_and_mul, "gelu": gelu_and_mul, "gelu_tanh": gelu_tanh_and_mul}


def _mostly_equal(got: torch.Tensor, ref: torch.Tensor, what: str, frac_max=0.01, steps=4):
    got, ref = got.float().cpu(), ref.float().cpu()
    diff = got != ref
    frac = diff.float().mean().item()
    assert frac < frac_max, f"{what}: {frac:.4f} of elements differ"
    if diff.any() and steps is not None:
        rel = ((got - ref).abs() / ref.abs().clamp_min(1e-2))[diff].max().item()
        assert rel <= steps * 2 ** -7, f"{what}: relative difference {rel}"


def _close(got: torch.Tensor, ref: torch.Tensor, what: str, tol=1e-2):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-6)
    assert err < tol, f"{what}: max error {err:.3e} of the largest magnitude"


def _problem(seed, T, H, I, E, k, dtype, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(dtype)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * scale).to(dtype)
    w2 = (torch.randn(E, H, I, generator=g) * scale).to(dtype)
    logits = torch.randn(T, E, generator=g)
    tw, ids = OM.fused_topk(logits, k, True)
    return x, w1, w2, tw, ids


F32_TOL = 2e-5


def _agree(got, ref, what, dtype, **kw):
    """The bar of the storage dtype: a tolerance for fp32, mostly-equal for bf16 / fp16."""
    if dtype == torch.float32:
        _close(got, ref, what, tol=F32_TOL)
    else:
        _mostly_equal(got, ref, what, **kw)


@pytest.mark.parametrize("activation", ["silu", "gelu", "gelu_tanh"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,d", [(64, 768), (7, 100), (3, 10)])
def test_act_and_mul(dev, activation, dtype, rows, d):
    x = torch.randn(rows, 2 * d, generator=torch.Generator().manual_seed(rows)).to(dtype) * 3
    got = ACT[activation](x.to(dev))
    _agree(got, OF.act_and_mul(x, activation), f"{activation} {dtype}", dtype, steps=1)


@pytest.mark.parametrize("seed,T,H,I,E,k,dtype,activation,on_input", [
    (0, 64, 2048, 768, 128, 8, torch.bfloat16, "silu", False),   # Qwen3-30B-A3B decode layer
    (1, 5, 200, 40, 7, 3, torch.float16, "gelu", True),          # K, N tails; weight on input
    (2, 100, 128, 64, 4, 2, torch.bfloat16, "gelu_tanh", False), # ~50 routes per expert
    # from 2048 routes per call the LDS-tiled kernel runs (up to 320 routes per expert in one tile)
    (10, 1024, 512, 256, 8, 4, torch.bfloat16, "silu", False),   # 512 routes per expert
    (11, 700, 200, 40, 7, 6, torch.float16, "gelu", True),       # K tail, column tail
    (12, 512, 2048, 768, 128, 8, torch.bfloat16, "silu", False), # Qwen3-30B-A3B prefill chunk
    (13, 2400, 256, 128, 64, 8, torch.bfloat16, "silu", False),  # ~300 routes per expert
    (14, 2100, 136, 72, 3, 2, torch.float16, "gelu", True),      # ~1400 per expert: 5 row tiles
    # second GEMM at K = I in {512, 768, 1024} below 2048 routes: the streaming kernel, here
    # with 8-row column tails on the last expert (read past its rows: zeros, not stored)
    (15, 40, 1000, 768, 9, 3, torch.bfloat16, "silu", True),
    (16, 33, 2040, 1024, 5, 2, torch.float16, "gelu", False),
    (17, 3, 520, 512, 40, 8, torch.bfloat16, "silu", False),     # 24 routes over 40 experts
    # K a multiple of 1024 up to 4096 streams through LDS in K quarters: second GEMMs at
    # K = 2048 and 3072 (no activation, column tails), a first GEMM at K = 3072
    (18, 20, 520, 2048, 6, 2, torch.bfloat16, "silu", False),
    (19, 9, 1000, 3072, 5, 3, torch.float16, "gelu", True),
    (23, 7, 3072, 64, 4, 2, torch.bfloat16, "gelu_tanh", False),
    # fp32 storage (split-K kernel at every size; K a multiple of 4 suffices)
    (20, 64, 2048, 768, 128, 8, torch.float32, "silu", False),
    (21, 5, 100, 36, 7, 3, torch.float32, "gelu", True),         # K = 100 and 36: not / 8
    (22, 700, 204, 44, 7, 6, torch.float32, "gelu_tanh", False), # 4200 routes, column tails
])
def test_expert_gemms_match_oracle_intermediates(dev, seed, T, H, I, E, k, dtype, activation,
                                                 on_input):
    x, w1, w2, tw, ids = _problem(seed, T, H, I, E, k, dtype)
    _, rc2, rc3 = OF.fused_experts(x, w1, w2, tw, ids, activation, on_input,
                                   return_intermediate=True)
    numel = T * k
    s, e, npp = moe_align_block_size(ids.to(dev), 16, E)
    xd, w1d, w2d, twd = x.to(dev), w1.to(dev), w2.to(dev), tw.to(dev)
    c2 = moe_expert_gemm(xd, w1d, twd, s, e, npp, 16, numel, k, activation=activation,
                         mul_routed_weight=on_input)
    _agree(c2, torch.from_numpy(rc2), "first GEMM + activation", dtype)
    # the second GEMM from the oracle's own activation output isolates its error
    c3 = moe_expert_gemm(torch.from_numpy(rc2).to(dtype).to(dev), w2d, twd, s, e, npp, 16,
                         numel, 1, mul_routed_weight=not on_input)
    _agree(c3, torch.from_numpy(rc3).view(numel, H), "second GEMM", dtype)


@pytest.mark.parametrize("seed,T,H,I,E,k,dtype,activation,on_input", [
    (3, 64, 2048, 768, 128, 8, torch.bfloat16, "silu", False),
    (4, 1, 1024, 512, 16, 4, torch.bfloat16, "silu", False),     # one token
    (5, 37, 256, 96, 60, 6, torch.float16, "gelu", True),
    (13, 64, 2048, 768, 128, 8, torch.float32, "silu", False),
    (14, 1, 132, 20, 5, 2, torch.float32, "gelu_tanh", True),
])
def test_fused_experts_decode_matches_oracle(dev, seed, T, H, I, E, k, dtype, activation,
                                             on_input):
    x, w1, w2, tw, ids = _problem(seed, T, H, I, E, k, dtype)
    ref = OF.fused_experts(x, w1, w2, tw, ids, activation, on_input)
    got = fused_experts_decode_impl(x.to(dev), w1.to(dev), w2.to(dev), tw.to(dev),
                                    ids.to(dev), activation, on_input)
    if dtype == torch.float32:
        _close(got, ref, "decode FFN", tol=F32_TOL)
        return
    _close(got, ref, "decode FFN")
    # a flipped last bit in one of the k summed rows can be large relative to a sum that cancels,
    # so the output is held to the fraction of differing elements (the rows themselves are held
    # to a few steps each above)
    _mostly_equal(got, ref, "decode FFN", frac_max=0.02, steps=None)


@pytest.mark.parametrize("T,dtype", [(300, torch.bfloat16), (1100, torch.bfloat16),
                                     (1100, torch.float32)])
def test_fused_experts_impl_overwrites_hidden(dev, T, dtype):
    x, w1, w2, tw, ids = _problem(6, T, 512, 128, 32, 4, dtype)
    ref = OF.fused_experts(x, w1, w2, tw, ids)
    xd = x.to(dev)
    got = fused_experts_impl(xd, w1.to(dev), w2.to(dev), tw.to(dev), ids.to(dev))
    assert got.data_ptr() == xd.data_ptr()
    _close(got, ref, "prefill FFN", tol=F32_TOL if dtype == torch.float32 else 1e-2)


def test_fused_experts_over_slot_ids(dev):
    """Decode over a slot cache: ids are slot indices into 3072 slots (few of them used)."""
    g = torch.Generator().manual_seed(7)
    T, H, I, S, k = 64, 64, 32, 3072, 8
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(S, 2 * I, H, generator=g) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(S, H, I, generator=g) * 0.1).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(S, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    tw = torch.rand(T, k, generator=g)
    ref = OF.fused_experts(x, w1, w2, tw, ids)
    got = fused_experts_decode_impl(x.to(dev), w1.to(dev), w2.to(dev), tw.to(dev), ids.to(dev))
    _close(got, ref, "slot-id FFN")


def test_fused_moe_backend_routes_and_computes(dev):
    x, w1, w2, _, _ = _problem(8, 48, 256, 64, 16, 4, torch.bfloat16)
    logits = torch.randn(48, 16, generator=torch.Generator().manual_seed(9))
    tw, ids = fused_topk(x.to(dev), logits.to(dev), 4, True)
    rtw, rids = OM.fused_topk(logits, 4, True)
    assert torch.equal(ids.cpu(), rids)
    ref = OF.fused_experts(x, w1, w2, rtw, rids)
    got = FusedMoe().forward(x.to(dev).clone(), w1.to(dev), w2.to(dev), logits.to(dev), 4, True)
    _close(got, ref, "FusedMoe")


def test_expert_gemm_rejects_bad_shapes(dev):
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device=dev)      # K = 12 is not a multiple of 8
    w = torch.zeros(2, 8, 12, dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(4, 1, dtype=torch.int32, device=dev)
    s, e, npp = moe_align_block_size(ids, 16, 2)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        moe_expert_gemm(x, w, None, s, e, npp, 16, 4, 1)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        moe_expert_gemm(x[:, :8].contiguous(), w[:, :, :8].contiguous(), None, s, e, npp, 8, 4, 1)
    xf = torch.zeros(4, 6, dtype=torch.float32, device=dev)       # fp32 needs K % 4 == 0
    wf = torch.zeros(2, 8, 6, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="multiples of 4"):
        moe_expert_gemm(xf, wf, None, s, e, npp, 16, 4, 1)
    with pytest.raises(ValueError, match="dtype"):
        moe_expert_gemm(xf.double(), wf.double(), None, s, e, npp, 16, 4, 1)
