"""Pins the MoE routing / permute oracle (CPU, no GPU).

  * router: the reference's known answers (reference tests/test_ops.py:294-325) and the closed
    form w_i = exp(x_i) / sum_{j in top-k} exp(x_j) computed in float64;
  * permute plan: the worked example of the reference's moe_align_block_size docstring
    (reference src/plastic_infer/moe/fused.py:71-86) and structural invariants;
  * permute / unpermute: identity experts give out[t] = (sum_s w[t,s]) * hidden[t];
  * planted mistakes (unpadded regions, descending within-expert order, dropped weight) fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.moe_route as OM


class TestRouterKATs:
    def test_topk_route_picks_largest(self):
        ids, w = OM.topk_route(torch.tensor([[1.0, 5.0, 3.0, 0.5, 2.0]]), 2)
        assert set(ids[0].tolist()) == {1, 2}
        assert torch.allclose(w.sum(-1), torch.ones(1))

    def test_topk_route_softmax(self):
        ids, w = OM.topk_route(torch.tensor([[1.0, 2.0, 3.0, 4.0]]), 2)
        assert ids[0].tolist() == [3, 2]
        assert torch.allclose(w, torch.softmax(torch.tensor([[4.0, 3.0]]), -1), atol=1e-6)

    @pytest.mark.parametrize("renorm", [True, False])
    def test_fused_topk_closed_form(self, renorm):
        g = torch.Generator().manual_seed(0)
        x = torch.randn(64, 16, generator=g)
        w, ids = OM.fused_topk(x, 4, renorm)
        xd = x.double().numpy()
        order = np.argsort(-xd, axis=1, kind="stable")[:, :4]
        assert np.array_equal(ids.numpy(), order)
        e = np.exp(xd - xd.max(1, keepdims=True))
        sel = np.take_along_axis(e, order, 1)
        ref = sel / (sel.sum(1, keepdims=True) if renorm else e.sum(1, keepdims=True))
        np.testing.assert_allclose(w.numpy(), ref, rtol=1e-6)

    def test_variants_agree_on_ids_and_renormalised_weights(self):
        g = torch.Generator().manual_seed(1)
        x = torch.randn(32, 128, generator=g)
        w0, i0 = OM.fused_topk(x, 8, True)
        i1, w1 = OM.topk_route(x, 8)
        assert torch.equal(i0.long(), i1)
        assert torch.allclose(w0, w1.float(), atol=1e-6)


DOC_IDS = [[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]]
DOC_SORTED = [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]


class TestAlign:
    def test_reference_docstring_example(self):
        s, e, npp, pos = OM.moe_align_block_size(DOC_IDS, 4, 4)
        assert npp == 16
        assert s[:16].tolist() == DOC_SORTED
        assert (s[16:] == 12).all() and s.size == OM.max_num_tokens_padded(12, 4, 4) == 27
        assert e[:4].tolist() == [1, 2, 3, 4] and (e[4:] == -1).all()
        for r in range(12):
            assert s[pos[r]] == r

    @pytest.mark.parametrize("seed,T,k,E,bs", [(0, 50, 2, 8, 4), (1, 1, 8, 128, 64),
                                               (2, 300, 8, 128, 16), (3, 7, 3, 5, 1)])
    def test_invariants(self, seed, T, k, E, bs):
        rng = np.random.default_rng(seed)
        ids = rng.integers(-1, E + 2, size=(T, k)).astype(np.int32)   # includes dropped ids
        s, e, npp, pos = OM.moe_align_block_size(ids, bs, E)
        flat = ids.reshape(-1)
        numel = flat.size
        valid = (flat >= 0) & (flat <= E)
        assert npp % bs == 0
        real = s[:npp][s[:npp] < numel]
        assert sorted(real.tolist()) == np.nonzero(valid)[0].tolist()   # every valid route once
        for b in range(npp // bs):
            blk = s[b * bs:(b + 1) * bs]
            assert all(flat[r] == e[b] for r in blk if r < numel)
        for ex in range(E + 1):
            rows = [r for r in s[:npp] if r < numel and flat[r] == ex]
            assert rows == sorted(rows)                                 # ascending in expert
        assert (pos[~valid] == -1).all()
        assert all(s[pos[r]] == r for r in np.nonzero(valid)[0])

    def test_planted_unpadded_plan_fails_kat(self):
        ids = np.asarray(DOC_IDS).reshape(-1)
        wrong = np.concatenate([np.nonzero(ids == ex)[0] for ex in range(5)])   # no padding
        assert wrong.tolist() != DOC_SORTED[:len(wrong)]

    def test_planted_descending_order_fails_invariant(self):
        s, _, npp, _ = OM.moe_align_block_size(DOC_IDS, 4, 4)
        bad = s.copy()
        bad[0:3] = bad[0:3][::-1]
        assert bad[:16].tolist() != DOC_SORTED


class TestPermuteCombine:
    def test_identity_experts_closed_form(self):
        g = torch.Generator().manual_seed(3)
        T, H, E, k = 40, 32, 16, 4
        hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
        logits = torch.randn(T, E, generator=g)
        w, ids = OM.fused_topk(logits, k, True)
        s, _, npp, pos = OM.moe_align_block_size(ids.numpy(), 8, E)
        xp = OM.permute(hidden, s, npp, k)
        for r in range(npp):
            if s[r] < T * k:
                assert torch.equal(xp[r], hidden[s[r] // k])
            else:
                assert not xp[r].any()
        out = OM.unpermute(xp, pos, w.numpy(), T, k, torch.float32)
        ref = hidden.double() * w.double().sum(1, keepdim=True)
        assert torch.allclose(out.double(), ref, atol=1e-5)

    def test_unpermute_sequential_fp32(self):
        g = torch.Generator().manual_seed(4)
        y = torch.randn(12, 5, generator=g)
        w = torch.rand(3, 4, generator=g)
        pos = np.arange(12, dtype=np.int32)[::-1].copy()
        out = OM.unpermute(y, pos, w.numpy(), 3, 4, torch.float32)
        for t in range(3):
            acc = np.zeros(5, np.float32)
            for s_ in range(4):
                acc = (acc + np.float32(w[t, s_]) * y[pos[t * 4 + s_]].numpy()).astype(np.float32)
            assert np.array_equal(out[t].numpy(), acc)

    def test_planted_dropped_weight_is_caught(self):
        g = torch.Generator().manual_seed(5)
        hidden = torch.randn(6, 8, generator=g)
        w = torch.rand(6, 2, generator=g)
        pos = np.arange(12, dtype=np.int32)
        y = hidden.repeat_interleave(2, 0)
        wrong = OM.unpermute(y, pos, None, 6, 2, torch.float32)          # weight dropped
        ref = hidden * w.sum(1, keepdim=True)
        assert not torch.allclose(wrong, ref, atol=1e-4)

    def test_sum_reduce(self):
        g = torch.Generator().manual_seed(6)
        x = torch.randn(5, 3, 7, generator=g).to(torch.bfloat16)
        out = OM.sum_reduce(x, torch.bfloat16)
        ref = ((x[:, 0].float() + x[:, 1].float()) + x[:, 2].float()).to(torch.bfloat16)
        assert torch.equal(out, ref)


def test_oracle_moe_forward_sparse_equals_per_token_loop():
    """fp32: the oracle's per-expert composition equals the per-token definition
    out[t] = sum_s w[t, s] * mlp_{ids[t, s]}(x[t]) (the reference tests' ground truth); an
    expert missing from the dict contributes nothing; dropping the weights breaks it."""
    import types

    import torch.nn.functional as F

    g = torch.Generator().manual_seed(3)
    T, H, I, E, k = 12, 16, 24, 5, 2
    x = torch.randn(T, H, generator=g)
    ex = {e: types.SimpleNamespace(w1=torch.randn(I, H, generator=g) * 0.3,
                                   w2=torch.randn(H, I, generator=g) * 0.3,
                                   w3=torch.randn(I, H, generator=g) * 0.3) for e in range(E)}
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g)

    def mlp(e, v):
        return F.linear(F.silu(F.linear(v, ex[e].w1)) * F.linear(v, ex[e].w3), ex[e].w2)

    ref = torch.stack([sum(w[t, s] * mlp(int(ids[t, s]), x[t]) for s in range(k))
                       for t in range(T)])
    assert torch.allclose(OM.moe_forward_sparse(x, ex, ids, w), ref, atol=1e-5)
    part = {e: v for e, v in ex.items() if e != 2}
    ref2 = torch.stack([sum((w[t, s] * mlp(int(ids[t, s]), x[t]) if int(ids[t, s]) != 2
                             else torch.zeros(H)) for s in range(k)) for t in range(T)])
    assert torch.allclose(OM.moe_forward_sparse(x, part, ids, w), ref2, atol=1e-5)
    assert not torch.allclose(OM.moe_forward_sparse(x, ex, ids, torch.ones_like(w)), ref,
                              atol=1e-3)
