"""GPU parity of routing / permute plan / permute / combine against the oracle.

Indices, the permute plan, the permuted rows and the combine (fp32, fixed order, separately
rounded multiply and add) are bit-exact; router weights are compared at 1e-6 relative (exp and
the order of the renormalising sum differ from torch's CPU kernels).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.moe_route as OM
import oracle.workloads as W
from plastic_infer.exec.moe import moe_forward_sparse, swiglu_mlp, topk_route
from plastic_infer.kernel import moe_align_block_size, moe_permute, moe_sum_reduce, moe_unpermute
from plastic_infer.moe.fused import fused_topk
from plastic_infer.store.experts import ExpertWeights

pytestmark = pytest.mark.gpu


def test_router_t4096_e128_indices_bit_exact(dev):
    wl = W.moe_workload()
    w, ids = fused_topk(wl.hidden.to(dev), wl.logits.to(dev), wl.topk, True)
    rw, rids = OM.fused_topk(wl.logits, wl.topk, True)
    assert torch.equal(ids.cpu(), rids)
    assert torch.allclose(w.cpu(), rw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_router_dtypes_and_padding(dev, dtype):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(37, 200, generator=g).to(dtype)
    w, ids = fused_topk(torch.zeros(37, 1), logits.to(dev), 6, False, num_token_non_padded=30)
    p = torch.softmax(logits.float(), -1)
    ref_ids = torch.from_numpy(np.argsort(-logits.float().numpy(), 1, kind="stable")[:, :6].copy())
    assert torch.equal(ids.cpu()[:30].long(), ref_ids[:30])
    assert (ids.cpu()[30:] == -1).all()
    assert torch.allclose(w.cpu(), torch.gather(p, 1, ref_ids), rtol=1e-5, atol=1e-7)


def test_topk_route_kats(dev):
    ids, w = topk_route(torch.tensor([[1.0, 5.0, 3.0, 0.5, 2.0]], device=dev), k=2)
    assert set(ids[0].tolist()) == {1, 2} and torch.allclose(w.sum(-1).cpu(), torch.ones(1))
    ids, w = topk_route(torch.tensor([[1.0, 2.0, 3.0, 4.0]], device=dev), k=2)
    assert ids[0].tolist() == [3, 2] and ids.dtype == torch.int64
    assert torch.allclose(w.cpu(), F.softmax(torch.tensor([[4.0, 3.0]]), -1), atol=1e-6)


def _check_align(dev, ids_np, bs, E):
    s, e, npp, pos = moe_align_block_size(torch.from_numpy(ids_np).to(dev), bs, E,
                                          return_route_pos=True)
    rs, re_, rnpp, rpos = OM.moe_align_block_size(ids_np, bs, E)
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy()[:rnpp // bs], re_[:rnpp // bs])
    assert np.array_equal(pos.cpu().numpy(), rpos)


def test_align_reference_docstring_example(dev):
    _check_align(dev, np.array([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], np.int32), 4, 4)


@pytest.mark.parametrize("seed,T,k,E,bs", [(0, 4096, 8, 128, 64), (1, 1, 8, 128, 16),
                                           (2, 300, 8, 128, 1), (3, 77, 3, 5, 7),
                                           (4, 2000, 2, 1023, 16),
                                           # one-launch path at its limits and just past them
                                           (5, 512, 8, 128, 16), (6, 513, 8, 128, 16),
                                           (7, 64, 8, 3072, 16), (8, 64, 8, 12287, 16),
                                           (9, 64, 8, 12288, 16)])
def test_align_random_bit_exact(dev, seed, T, k, E, bs):
    rng = np.random.default_rng(seed)
    _check_align(dev, rng.integers(-1, E + 2, size=(T, k)).astype(np.int32), bs, E)


@pytest.mark.parametrize("seed,T,k,E,bs,H,dtype", [(5, 300, 8, 16, 16, 100, torch.float32),
                                                   (6, 77, 3, 5, 7, 2048, torch.bfloat16),
                                                   (7, 64, 64, 100, 4, 24, torch.float16)])
def test_permute_token_major_matches_row_major(dev, seed, T, k, E, bs, H, dtype):
    rng = np.random.default_rng(seed)
    ids = torch.tensor(rng.integers(-1, E + 1, size=(T, k)), dtype=torch.int32, device=dev)
    hidden = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).to(dtype).to(dev)
    s, _, npp, pos = moe_align_block_size(ids, bs, E, return_route_pos=True)
    a = torch.full((s.numel(), H), 5.0, dtype=dtype, device=dev)
    moe_permute(hidden, s, npp, k, out=a)
    b = torch.full_like(a, 3.0)
    moe_permute(hidden, s, npp, k, out=b, route_pos=pos)
    rs, _, rnpp, _ = OM.moe_align_block_size(ids.cpu().numpy(), bs, E)
    ref = OM.permute(hidden.cpu(), rs, rnpp, k)
    _check_permuted(a, 5.0, s, npp, T * k, ref)
    _check_permuted(b, 3.0, s, npp, T * k, ref)


def _check_permuted(out, fill, sorted_ids, npp, numel, ref):
    """Rows of real routes equal the oracle's permute bit for bit; padding rows (sentinel ids)
    and rows past npp still hold `fill` (the permute leaves them untouched)."""
    n = int(npp.item())
    real = (sorted_ids[:n] < numel).cpu()
    got = out.cpu()
    assert torch.equal(got[:n][real], ref[real])
    assert bool((got[:n][~real] == fill).all()) and bool((got[n:] == fill).all())


def test_align_empty(dev):
    s, e, npp = moe_align_block_size(torch.empty(0, 8, dtype=torch.int32, device=dev), 16, 128)
    assert int(npp.item()) == 0 and s.numel() == 0


def test_permute_combine_t4096(dev):
    wl = W.moe_workload()
    w, ids = OM.fused_topk(wl.logits, wl.topk, True)
    T, k = ids.shape
    s, e, npp, pos = moe_align_block_size(ids.to(dev), 64, 128, return_route_pos=True)
    hidden = wl.hidden.to(dev)
    xp = torch.full((s.numel(), hidden.shape[1]), 5.0, dtype=hidden.dtype, device=dev)
    moe_permute(hidden, s, npp, k, out=xp)
    rs, _, rnpp, rpos = OM.moe_align_block_size(ids.numpy(), 64, 128)
    ref_xp = OM.permute(wl.hidden, rs, rnpp, k)
    _check_permuted(xp, 5.0, s, npp, T * k, ref_xp)
    # token-major path (each token row read once): the same rows, the rest untouched
    xt = torch.full_like(xp, 7.0)
    moe_permute(hidden, s, npp, k, out=xt, route_pos=pos)
    _check_permuted(xt, 7.0, s, npp, T * k, ref_xp)
    out = moe_unpermute(xp, pos, w.to(dev), T, k)              # identity expert stand-in
    ref = OM.unpermute(ref_xp, rpos, w.numpy(), T, k, torch.bfloat16)
    assert torch.equal(out.cpu(), ref)
    closed = (wl.hidden.double() * w.double().sum(1, keepdim=True)).to(torch.bfloat16)
    assert (out.cpu().float() - closed.float()).abs().max() <= 2e-2


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 2048), (torch.float32, 100), (torch.float16, 12)])
def test_sum_reduce(dev, dtype, H):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(33, 8, H, generator=g).to(dtype)
    out = torch.empty(33, H, dtype=dtype, device=dev)
    moe_sum_reduce(x.to(dev), out)
    assert torch.equal(out.cpu(), OM.sum_reduce(x, dtype))


def _experts(E, H, I, seed=7):
    g = torch.Generator().manual_seed(seed)
    return {e: ExpertWeights(torch.randn(I, H, generator=g) * 0.1, torch.randn(H, I, generator=g) * 0.1,
                             torch.randn(I, H, generator=g) * 0.1) for e in range(E)}


def test_moe_forward_sparse_vs_loop(dev):
    torch.manual_seed(11)
    T, H, I, E, k = 8, 16, 32, 4, 2
    hidden = torch.randn(T, H) * 0.5
    experts = _experts(E, H, I)
    eids, weights = topk_route(torch.randn(T, E).to(dev), k=k)
    routed = {int(x) for x in eids.flatten().tolist()}
    dev_experts = {e: ExpertWeights(*(t.to(dev) for t in (w.w1, w.w2, w.w3)))
                   for e, w in experts.items() if e in routed}
    out = moe_forward_sparse(hidden.to(dev), dev_experts, eids, weights).cpu()
    ref = torch.zeros(T, H)
    for t in range(T):
        for s_ in range(k):
            w = experts[int(eids[t, s_])]
            ref[t] += swiglu_mlp(hidden[t], w.w1, w.w2, w.w3) * weights[t, s_].cpu()
    assert torch.allclose(out, ref, atol=1e-5)


def test_moe_forward_sparse_bf16_vs_reference_composition(dev):
    """bf16: the drop-in (permute, per-expert GEMMs, one fp32 weighted unpermute, one rounding)
    against the reference's composition (per-expert bf16 products and bf16 index_add_ in the
    dict's order, oracle moe_route.moe_forward_sparse). The two round the k weighted terms of a
    token differently: each bf16 running sum is off by at most half a bf16 step of its
    magnitude, and the expert MLPs are bf16 GEMMs on different devices, so the bar is 4 bf16
    steps (4 * 2^-8) of the output's largest magnitude."""
    g = torch.Generator().manual_seed(12)
    T, H, I, E, k = 64, 256, 128, 8, 2
    dt = torch.bfloat16
    hidden = (torch.randn(T, H, generator=g) * 0.5).to(dt)
    experts = {e: ExpertWeights(*((torch.randn(*s, generator=g) * 0.1).to(dt)
                                  for s in ((I, H), (H, I), (I, H)))) for e in range(E)}
    logits = torch.randn(T, E, generator=g).to(dt)
    eids, weights = topk_route(logits.to(dev), k=k)
    dev_experts = {e: ExpertWeights(*(t.to(dev) for t in (w.w1, w.w2, w.w3)))
                   for e, w in experts.items()}
    out = moe_forward_sparse(hidden.to(dev), dev_experts, eids, weights).cpu()
    ref = OM.moe_forward_sparse(hidden, experts, eids.cpu(), weights.cpu())
    assert out.dtype == dt and ref.dtype == dt
    err = (out.float() - ref.float()).abs().max().item()
    assert err <= 4 * 2 ** -8 * ref.float().abs().max().item(), err


def _check_plan(ids, s, e, npp, pos, bs, E):
    rs, re_, rnpp, rpos = OM.moe_align_block_size(ids.cpu().numpy(), bs, E)
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy()[:rnpp // bs], re_[:rnpp // bs])
    assert (e.cpu().numpy()[rnpp // bs:] == -1).all()
    assert np.array_equal(pos.cpu().numpy(), rpos)


@pytest.mark.parametrize("T", [61440, 61441])
def test_topk_align_byte_count_boundary(dev, T):
    """61,440 tokens is the largest call of the fused plan (240-token chunks, so a chunk's count
    of one expert fits the byte the plan stores it in); one token more takes the three-launch
    path. Every token routes to experts 0..7 (a large bias on their logits), so each chunk
    counts 240 routes of each: the byte table at its maximum. Ids against the stable argsort,
    the plan bit-exact against the oracle."""
    from plastic_infer.kernel import moe_topk_align

    k, E, bs = 8, 128, 64
    g = torch.Generator().manual_seed(T)
    logits = torch.randn(T, E, generator=g)
    logits[:, :k] += 100.0
    w, ids, s, e, npp, pos = moe_topk_align(logits.to(dev), k, bs)
    ref_ids = np.argsort(-logits.numpy(), 1, kind="stable")[:, :k]
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    _check_plan(ids, s, e, npp, pos, bs, E)


@pytest.mark.parametrize("T,k,E,bs,dtype,n_np", [
    (4096, 8, 128, 64, torch.float32, None),   # Qwen3-30B-A3B routing (two-launch path)
    (600, 8, 64, 16, torch.float32, None),     # just past the one-block plan
    (5000, 6, 200, 1, torch.bfloat16, 4900),   # 48-token chunks, ties in bf16, padded tokens
    (2048, 8, 509, 16, torch.float16, None),   # the largest expert count of the fused path
    (100, 2, 16, 16, torch.float32, 90),       # small: top-k then the one-block plan
])
def test_topk_align_matches_topk_then_oracle_plan(dev, T, k, E, bs, dtype, n_np):
    """moe_topk_align: weights and ids bit-identical to moe_topk on the same logits (lowest
    index first on ties, the stable argsort of the logits), the plan bit-exact against the
    oracle's stable plan of those ids, route_pos -1 for the padded tokens' routes."""
    from plastic_infer.kernel import moe_topk, moe_topk_align

    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g).to(dtype).to(dev)
    w, ids, s, e, npp, pos = moe_topk_align(logits, k, bs, num_token_non_padded=n_np)
    w1, ids1 = moe_topk(logits, k, True, num_token_non_padded=n_np)
    assert torch.equal(ids, ids1) and torch.equal(w, w1)
    lim = T if n_np is None else n_np
    ref_ids = np.argsort(-logits.float().cpu().numpy(), 1, kind="stable")[:, :k]
    assert np.array_equal(ids.cpu().numpy()[:lim], ref_ids[:lim])
    assert (ids.cpu()[lim:] == -1).all()
    rs, re_, rnpp, rpos = OM.moe_align_block_size(ids.cpu().numpy(), bs, E)
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy()[:rnpp // bs], re_[:rnpp // bs])
    assert (e.cpu().numpy()[rnpp // bs:] == -1).all()
    assert np.array_equal(pos.cpu().numpy(), rpos)
