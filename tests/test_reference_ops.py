"""The reference's hot-path op test cases (reference tests/test_ops.py: paged gather, paged
attention, MoE routing, MoE forward, sparse MoE forward, host-stream attention), one for one, on
this package's HIP path. Same shapes, seeds and tolerances; the reference's ground-truth helpers
(contiguous SDPA, its per-token MoE loops) are restated here next to the cases that use them.
(RMSNorm and RoPE cases are outside the data path.)"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from plastic_infer.exec.attention import (gather_paged_kv, host_stream_attention_v1,
                                          paged_attention_v1)
from plastic_infer.exec.moe import moe_forward_sparse, moe_forward_v1, swiglu_mlp, topk_route
from plastic_infer.store.experts import ExpertWeights

pytestmark = pytest.mark.gpu


def _sdpa_gqa(q, k, v, causal, mask=None):
    """Contiguous SDPA over [B, S, H, D] with kv heads repeated G times (CPU, fp32)."""
    G = q.shape[2] // k.shape[2]
    qt = q.transpose(1, 2)
    kt = k.transpose(1, 2).repeat_interleave(G, dim=1)
    vt = v.transpose(1, 2).repeat_interleave(G, dim=1)
    if mask is not None:
        return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask).transpose(1, 2)
    return F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal).transpose(1, 2)


# ---- TestPagedKvGather (reference :102-147) -----------------------------------------------------

def test_gather_single_page(dev):
    torch.manual_seed(0)
    kp, vp = torch.randn(10, 2, 8, 16), torch.randn(10, 2, 8, 16)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [3], 16)
    assert k.shape == (1, 16, 2, 8)
    assert torch.equal(k[0, 0].cpu(), kp[3, :, :, 0])


def test_gather_multiple_pages_in_order(dev):
    torch.manual_seed(1)
    kp, vp = torch.randn(5, 2, 4, 8), torch.randn(5, 2, 4, 8)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [0, 2, 4], 8)
    assert k.shape == (1, 24, 2, 4)
    for t, p in ((0, 0), (8, 2), (16, 4)):
        assert torch.equal(k[0, t].cpu(), kp[p, :, :, 0])


def test_gather_partial_last_page(dev):
    kp, vp = torch.randn(4, 2, 4, 16), torch.randn(4, 2, 4, 16)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [0, 1], 16, num_tokens=20)
    assert k.shape == (1, 20, 2, 4)


def test_gather_empty_block_table(dev):
    kp, vp = torch.randn(4, 2, 4, 16), torch.randn(4, 2, 4, 16)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [], 16)
    assert k.shape == (1, 0, 2, 4) and v.shape == (1, 0, 2, 4)


# ---- TestPagedAttention (reference :186-291) ----------------------------------------------------

def test_paged_attention_matches_contiguous(dev):
    torch.manual_seed(7)
    B, Sq, H, D, P, n_pages, Hkv = 1, 8, 4, 16, 4, 3, 2
    q = torch.randn(B, Sq, H, D) * 0.1
    kc = torch.randn(B, n_pages * P, Hkv, D) * 0.1
    vc = torch.randn(B, n_pages * P, Hkv, D) * 0.1
    kp = kc[0].view(n_pages, P, Hkv, D).permute(0, 2, 3, 1).contiguous()   # [N, Hkv, D, P]
    vp = vc[0].view(n_pages, P, Hkv, D).permute(0, 2, 3, 1).contiguous()
    out = paged_attention_v1(q.to(dev), kp.to(dev), vp.to(dev), list(range(n_pages)), P,
                             kv_num_tokens=n_pages * P, causal=True).cpu()
    assert torch.allclose(out, _sdpa_gqa(q, kc, vc, True), atol=1e-4)


def test_paged_attention_noncontiguous_pages(dev):
    torch.manual_seed(11)
    q = torch.randn(1, 6, 2, 8) * 0.1
    kp, vp = torch.randn(5, 2, 8, 3) * 0.1, torch.randn(5, 2, 8, 3) * 0.1
    table = [4, 1, 3]
    out = paged_attention_v1(q.to(dev), kp.to(dev), vp.to(dev), table, 3, kv_num_tokens=9,
                             causal=True).cpu()
    kc = torch.cat([kp[p].permute(2, 0, 1) for p in table]).unsqueeze(0)
    vc = torch.cat([vp[p].permute(2, 0, 1) for p in table]).unsqueeze(0)
    assert torch.allclose(out, _sdpa_gqa(q, kc, vc, True), atol=1e-4)


def test_paged_attention_decode_single_token(dev):
    torch.manual_seed(13)
    q = torch.randn(1, 1, 2, 8) * 0.1
    kp, vp = torch.randn(5, 2, 8, 4) * 0.1, torch.randn(5, 2, 8, 4) * 0.1
    out = paged_attention_v1(q.to(dev), kp.to(dev), vp.to(dev), list(range(5)), 4,
                             kv_num_tokens=20, causal=True)
    assert out.shape == (1, 1, 2, 8) and torch.isfinite(out).all()
    # and the value the reference's composition gives: SDPA(is_causal=True) aligns the mask to
    # the top left, so the one query row (position 0) attends key 0 only
    kc = torch.cat([kp[p].permute(2, 0, 1) for p in range(5)]).unsqueeze(0)
    vc = torch.cat([vp[p].permute(2, 0, 1) for p in range(5)]).unsqueeze(0)
    ref = _sdpa_gqa(q, kc, vc, True)
    assert torch.allclose(ref[0, 0], vc[0, 0], atol=1e-6)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)


# ---- TestMoERouting (reference :294-325) --------------------------------------------------------

def test_topk_picks_largest(dev):
    ids, w = topk_route(torch.tensor([[1.0, 5.0, 3.0, 0.5, 2.0]], device=dev), k=2)
    assert ids.shape == (1, 2) and set(ids[0].tolist()) == {1, 2}
    assert torch.allclose(w.sum(-1).cpu(), torch.ones(1))


def test_topk_softmax_correct(dev):
    ids, w = topk_route(torch.tensor([[1.0, 2.0, 3.0, 4.0]], device=dev), k=2)
    assert ids[0].tolist() == [3, 2]
    assert torch.allclose(w.cpu(), F.softmax(torch.tensor([[4.0, 3.0]]), -1), atol=1e-5)


def test_route_batch(dev):
    torch.manual_seed(0)
    ids, w = topk_route(torch.randn(16, 8).to(dev), k=2)
    assert ids.shape == (16, 2) and w.shape == (16, 2)
    assert (w > 0).all() and torch.allclose(w.sum(-1).cpu(), torch.ones(16))


# ---- TestMoEForward (reference :332-377) --------------------------------------------------------

def _moe_v1_loop(hidden, w1, w2, ids, w):
    """The reference's per-token ground truth (src/plastic_infer/exec/moe.py:85-118)."""
    out = torch.zeros_like(hidden)
    for t in range(hidden.shape[0]):
        for s in range(ids.shape[1]):
            e = int(ids[t, s])
            out[t] += (F.silu(hidden[t] @ w1[e]) @ w2[e]) * w[t, s]
    return out


def test_moe_v1_matches_reference(dev):
    torch.manual_seed(99)
    T, H, I, E, k = 8, 16, 32, 4, 2
    hidden = torch.randn(T, H) * 0.5
    w1, w2 = torch.randn(E, H, I) * 0.1, torch.randn(E, I, H) * 0.1
    ids, w = topk_route(torch.randn(T, E).to(dev), k=k)
    out = moe_forward_v1(hidden.to(dev), w1.to(dev), w2.to(dev), ids, w).cpu()
    ref = _moe_v1_loop(hidden, w1, w2, ids.cpu(), w.cpu())
    assert out.shape == ref.shape and torch.allclose(out, ref, atol=1e-4)


def test_moe_v1_single_token_single_expert(dev):
    T, H, I, E, k = 1, 4, 8, 1, 1
    hidden, w1, w2 = torch.randn(T, H), torch.randn(E, H, I), torch.randn(E, I, H)
    out = moe_forward_v1(hidden.to(dev), w1.to(dev), w2.to(dev),
                         torch.zeros(T, k, dtype=torch.long, device=dev),
                         torch.ones(T, k, device=dev)).cpu()
    assert torch.allclose(out, F.silu(hidden @ w1[0]) @ w2[0], atol=1e-5)


def test_moe_v1_output_shape(dev):
    T, H, I, E, k = 10, 32, 64, 8, 2
    w = torch.rand(T, k)
    out = moe_forward_v1(torch.randn(T, H).to(dev), torch.randn(E, H, I).to(dev),
                         torch.randn(E, I, H).to(dev), torch.randint(0, E, (T, k)).to(dev),
                         (w / w.sum(-1, keepdim=True)).to(dev))
    assert out.shape == (T, H)


# ---- TestSparseMoEForward (reference :380-445) --------------------------------------------------

def _experts(E, H, I, seed=7):
    g = torch.Generator().manual_seed(seed)
    return {e: ExpertWeights(w1=torch.randn(I, H, generator=g) * 0.1,
                             w2=torch.randn(H, I, generator=g) * 0.1,
                             w3=torch.randn(I, H, generator=g) * 0.1) for e in range(E)}


def _on(dev, experts):
    return {e: ExpertWeights(w1=x.w1.to(dev), w2=x.w2.to(dev), w3=x.w3.to(dev))
            for e, x in experts.items()}


def _swiglu_loop(hidden, experts, ids, w):
    """The reference's per-token ground truth (src/plastic_infer/exec/moe.py:163-185)."""
    out = torch.zeros_like(hidden)
    for t in range(hidden.shape[0]):
        for s in range(ids.shape[1]):
            x = experts[int(ids[t, s])]
            out[t] += F.linear(F.silu(F.linear(hidden[t], x.w1)) * F.linear(hidden[t], x.w3),
                               x.w2) * w[t, s]
    return out


def test_sparse_matches_reference(dev):
    torch.manual_seed(11)
    T, H, I, E, k = 8, 16, 32, 4, 2
    hidden = torch.randn(T, H) * 0.5
    experts = _experts(E, H, I)
    ids, w = topk_route(torch.randn(T, E).to(dev), k=k)
    routed = {int(e) for e in ids.flatten().tolist()}
    out = moe_forward_sparse(hidden.to(dev), _on(dev, {e: experts[e] for e in routed}), ids, w)
    ref = _swiglu_loop(hidden, experts, ids.cpu(), w.cpu())
    assert out.shape == ref.shape and torch.allclose(out.cpu(), ref, atol=1e-5)


def test_sparse_single_token_single_expert(dev):
    T, H, I, k = 1, 4, 8, 1
    hidden = torch.randn(T, H)
    x = ExpertWeights(w1=torch.randn(I, H), w2=torch.randn(H, I), w3=torch.randn(I, H))
    out = moe_forward_sparse(hidden.to(dev), _on(dev, {0: x}),
                             torch.zeros(T, k, dtype=torch.long, device=dev),
                             torch.ones(T, k, device=dev))
    assert torch.allclose(out.cpu(), swiglu_mlp(hidden, x.w1, x.w2, x.w3), atol=1e-5)


def test_sparse_unrouted_experts_not_needed(dev):
    torch.manual_seed(13)
    T, H, I, E, k = 12, 16, 32, 8, 2
    hidden = torch.randn(T, H) * 0.5
    experts = _experts(E, H, I, seed=3)
    ids, w = topk_route(torch.randn(T, E).to(dev), k=k)
    routed = {int(e) for e in ids.flatten().tolist()}
    sparse = moe_forward_sparse(hidden.to(dev), _on(dev, {e: experts[e] for e in routed}), ids, w)
    full = moe_forward_sparse(hidden.to(dev), _on(dev, experts), ids, w)
    assert torch.allclose(sparse, full, atol=1e-6)


# ---- TestHostStreamAttention (reference :448-544) -----------------------------------------------

def _hs_setup(seed, total_kv, host_len, chunk, Hkv=2, D=16):
    torch.manual_seed(seed)
    kf = torch.randn(1, total_kv, Hkv, D) * 0.1
    vf = torch.randn(1, total_kv, Hkv, D) * 0.1
    chunks = [(kf[0, s:s + chunk][:host_len - s].permute(1, 2, 0).contiguous(),
               vf[0, s:s + chunk][:host_len - s].permute(1, 2, 0).contiguous())
              for s in range(0, host_len, chunk)]
    return kf, vf, chunks, kf[:, host_len:], vf[:, host_len:]


def _hs_reference(q, kf, vf, q_start, causal=True):
    q_len, kv_len = q.shape[1], kf.shape[1]
    if causal and (q_start > 0 or q_len != kv_len):
        qp = torch.arange(q_start, q_start + q_len)
        mask = torch.zeros(q_len, kv_len).masked_fill(
            ~(torch.arange(kv_len)[None, :] <= qp[:, None]), float("-inf"))
        return _sdpa_gqa(q, kf, vf, True, mask=mask[None, None])
    return _sdpa_gqa(q, kf, vf, causal)


def _hs_run(dev, q, chunks, rk, rv, q_start):
    return host_stream_attention_v1(q.to(dev), [(k.to(dev), v.to(dev)) for k, v in chunks],
                                    rk.to(dev), rv.to(dev), q_start_pos=q_start).cpu()


@pytest.mark.parametrize("seed,total,host,chunk,q_len,q_start", [
    (1, 10, 6, 3, 2, 10),   # test_full_tail_prefill_matches_contiguous
    (2, 8, 5, 4, 1, 8),     # test_decode_step_matches_contiguous
    (3, 8, 4, 2, 2, 5),     # test_offset_query_attends_suffix
])
def test_host_stream_matches_contiguous(dev, seed, total, host, chunk, q_len, q_start):
    kf, vf, chunks, rk, rv = _hs_setup(seed, total, host, chunk)
    q = torch.randn(1, q_len, 4, 16) * 0.1
    out = _hs_run(dev, q, chunks, rk, rv, q_start)
    assert torch.allclose(out, _hs_reference(q, kf, vf, q_start), atol=1e-4)


def test_host_stream_all_resident_no_chunks(dev):
    kf, vf, _, _, _ = _hs_setup(4, 6, 6, 3)
    q = kf.clone().repeat_interleave(2, dim=2)   # q_len == kv_len, q_start_pos 0
    out = _hs_run(dev, q, [], kf, vf, 0)
    assert torch.allclose(out, _hs_reference(q, kf, vf, 0), atol=1e-4)
