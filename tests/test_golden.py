"""The reference's known answers (tests/golden/reference_kats.json) against the oracle (CPU) and
the HIP path (GPU, through the C-ABI)."""

from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest
import torch

import oracle.moe_route as OM
import oracle.paged_kv as OP

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _check_route(case, ids, w):
    ids, w = ids.cpu(), w.cpu().float()
    if "ids_as_set" in case:
        assert [sorted(r) for r in ids.tolist()] == [sorted(r) for r in case["ids_as_set"]]
    if "ids" in case:
        assert ids.tolist() == case["ids"]
    if "weights" in case:
        assert torch.allclose(w, torch.tensor(case["weights"]), atol=case["atol"])
    if "weight_row_sums" in case:
        assert torch.allclose(w.sum(-1), torch.tensor(case["weight_row_sums"]), atol=1e-6)


def _gather_pools(case):
    g = torch.Generator().manual_seed(0)
    shape = (case["num_pages"], case["num_heads"], case["head_dim"], case["page_size"])
    return torch.randn(shape, generator=g), torch.randn(shape, generator=g)


def _check_gather(case, k, v, kp, vp):
    assert tuple(k.shape) == tuple(case["out_shape"]) and tuple(v.shape) == tuple(case["out_shape"])
    for t, p, o in case["token_page_offset"]:
        assert torch.equal(k[0, t].cpu(), kp[p, :, :, o]) and torch.equal(v[0, t].cpu(), vp[p, :, :, o])


def _check_align(case, sorted_ids, expert_ids, npp):
    assert int(npp) == case["num_tokens_post_pad"]
    assert len(sorted_ids) == case["max_num_tokens_padded"]
    assert list(map(int, sorted_ids)) == case["sorted_token_ids"]
    used = case["num_tokens_post_pad"] // case["block_size"]
    assert list(map(int, expert_ids[:used])) == case["expert_ids_used"]


# ---- oracle (CPU) -------------------------------------------------------------------------------

@pytest.mark.parametrize("case", KATS["topk_route"], ids=lambda c: c["source"])
def test_oracle_topk_route(case):
    ids, w = OM.topk_route(torch.tensor(case["logits"]), case["k"])
    _check_route(case, ids, w)


@pytest.mark.parametrize("case", KATS["gather_paged_kv"], ids=lambda c: c["source"])
def test_oracle_gather(case):
    kp, vp = _gather_pools(case)
    k, v = OP.gather_paged_kv(kp, vp, case["block_table"], case["page_size"], case["num_tokens"])
    _check_gather(case, k, v, kp, vp)


@pytest.mark.parametrize("case", KATS["append_token_placement"], ids=lambda c: c["source"])
def test_oracle_append_placement(case):
    P = case["page_size"]
    kp, vp = torch.zeros(8, 2, 4, P), torch.zeros(8, 2, 4, P)
    k, v = torch.randn(1, 2, 4), torch.randn(1, 2, 4)
    assert case["physical_page"] * P + case["position"] % P == case["slot"]
    OP.scatter_slots(k, v, kp, vp, [case["slot"]])
    assert torch.equal(kp[case["physical_page"], :, :, case["position"] % P], k[0])
    assert torch.equal(vp[case["physical_page"], :, :, case["position"] % P], v[0])


@pytest.mark.parametrize("case", KATS["moe_align_block_size"], ids=lambda c: c["source"][:40])
def test_oracle_align(case):
    ids = np.array(case["topk_ids"])
    assert np.bincount(ids.ravel(), minlength=case["num_experts"] + 1).tolist() == case["counts"]
    assert OM.max_num_tokens_padded(ids.size, case["num_experts"], case["block_size"]) == \
        case["max_num_tokens_padded"]
    s, e, npp, _ = OM.moe_align_block_size(ids, case["block_size"], case["num_experts"])
    _check_align(case, s, e, npp)


# ---- HIP path (GPU) -----------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("case", KATS["topk_route"], ids=lambda c: c["source"])
def test_hip_topk_route(dev, case):
    from plastic_infer.exec.moe import topk_route
    ids, w = topk_route(torch.tensor(case["logits"], device=dev), k=case["k"])
    _check_route(case, ids, w)


@pytest.mark.gpu
@pytest.mark.parametrize("case", KATS["gather_paged_kv"], ids=lambda c: c["source"])
def test_hip_gather(dev, case):
    from plastic_infer.exec.attention import gather_paged_kv
    kp, vp = _gather_pools(case)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), case["block_table"], case["page_size"],
                           case["num_tokens"])
    _check_gather(case, k, v, kp, vp)


@pytest.mark.gpu
@pytest.mark.parametrize("case", KATS["append_token_placement"], ids=lambda c: c["source"])
def test_hip_append_placement(dev, case):
    from plastic_infer.kernel import kv_scatter
    P = case["page_size"]
    kp, vp = torch.zeros(8, 2, 4, P, device=dev), torch.zeros(8, 2, 4, P, device=dev)
    k, v = torch.randn(1, 2, 4), torch.randn(1, 2, 4)
    kv_scatter(k.to(dev), v.to(dev), kp, vp, torch.tensor([case["slot"]], device=dev))
    off = case["position"] % P
    assert torch.equal(kp[case["physical_page"], :, :, off].cpu(), k[0])
    assert torch.equal(vp[case["physical_page"], :, :, off].cpu(), v[0])
    assert int((kp != 0).sum()) == int((k != 0).sum())


@pytest.mark.gpu
@pytest.mark.parametrize("case", KATS["moe_align_block_size"], ids=lambda c: c["source"][:40])
def test_hip_align(dev, case):
    from plastic_infer.moe.fused import moe_align_block_size
    s, e, npp = moe_align_block_size(torch.tensor(case["topk_ids"], dtype=torch.int32, device=dev),
                                     case["block_size"], case["num_experts"])
    _check_align(case, s.cpu().numpy(), e.cpu().numpy(), npp.cpu().reshape(-1)[0])
