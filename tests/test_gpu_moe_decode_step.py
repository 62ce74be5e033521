"""GPU parity of the batched MoE-paged decode step (plastic_infer.exec.runner_moe_paged).

1. A small model end to end: logits of one decode step for 6 rows with their own context
   lengths and block tables against the oracle's decode step (the reference's per-request
   decode_step_moe_paged restated, oracle/moe_decode_step.py) run row by row on the same pool
   contents in the model dtype. Both residency policies ("lru", "static") with the overlapped
   FFN and the reference's order must give bit-identical logits (expert placement and the
   two-pass FFN do not change a single bit), within 3e-2 of the oracle's largest logit (bf16
   everywhere: both sides round the same ~30 intermediates per layer in different orders).
   Routing is an argmax over bf16 logits that the two sides compute in different orders, so
   the oracle follows the GPU's experts; where its own top-k differs, the k-th and (k+1)-th
   logits must be within 4 bf16 steps of each other (a near-tie, not a routing bug).
2. The Qwen3-30B-A3B per-layer shape over 2 layers: 64 rows x 4096 context, 32 q / 4 kv heads,
   128 experts top-8, expert slots for 50 % of the layers' experts. Checks of each part inside
   the composed step: every routed expert's slot rows equal the host banks bit for bit; the
   attention of sampled rows equals the oracle's (2e-2, the bf16 attention bar); the routed
   FFN of sampled tokens equals the oracle's within 1e-2 of its largest magnitude; both
   policies give bit-identical logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.fused_experts as OF
import oracle.moe_decode_step as OD
import oracle.paged_kv as OP
from plastic_infer.exec.runner_moe_paged import (
    DecodeBatch,
    MoeModelConfig,
    MoePagedDecoder,
    random_dense_weights,
    random_expert_banks,
)
from plastic_infer.moe.offload_cache import OffloadMoeCache

pytestmark = pytest.mark.gpu

P = 16


def _batch(dev, cfg, lens, n_pages, seed):
    """Block tables (distinct random pages per row and layer), slots of the new tokens."""
    g = torch.Generator().manual_seed(seed)
    L, B = cfg.n_layers, len(lens)
    per = [(n + P - 1) // P for n in lens]
    perm = torch.randperm(n_pages, generator=g).tolist()
    width = max(per)
    bt = torch.full((L, B, width), -1, dtype=torch.int32)
    tables = [[None] * L for _ in range(B)]
    off = 0
    for l in range(L):
        for b in range(B):
            row = perm[off:off + per[b]]
            off += per[b]
            bt[l, b, :per[b]] = torch.tensor(row, dtype=torch.int32)
            tables[b][l] = row
    assert off <= n_pages
    lens_t = torch.tensor(lens, dtype=torch.int32)
    pos = lens_t.long() - 1
    slots = torch.stack([bt[l, torch.arange(B), pos // P].long() * P + pos % P
                         for l in range(L)])
    return DecodeBatch(bt.to(dev), lens_t.to(dev), slots.to(dev), pos.to(dev)), tables


def _pools(dev, n_pages, Hkv, D, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    kp = torch.randn(n_pages, Hkv, D, P, generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn(n_pages, Hkv, D, P, generator=g, device=dev).to(torch.bfloat16)
    return kp, vp


def _cache(dev, cfg, banks, policy):
    L, E = cfg.n_layers, cfg.n_experts
    if policy == "static":
        c = OffloadMoeCache(L, E, L * (E // 2) + E // 2, dev, cache_policy="static")
    else:
        c = OffloadMoeCache(L, E, L * E // 2, dev)
    c.set_bank_sources(banks)
    return c


def test_small_model_step_matches_oracle_all_policies(dev):
    cfg = MoeModelConfig(n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, hidden_dim=256,
                         vocab_size=96, max_seq_len=512, n_experts=16, n_experts_per_tok=4,
                         moe_intermediate_dim=64, rope_base=10000.0)
    lens = [1, 17, 300, 64, 129, 5]
    n_pages = 200
    w = random_dense_weights(cfg, dev, seed=3, std=0.1)
    banks = random_expert_banks(cfg, dev, seed=4, std=0.1)
    kp0, vp0 = _pools(dev, n_pages, cfg.n_kv_heads, cfg.head_dim, 5)
    batch, tables = _batch(dev, cfg, lens, n_pages, 6)
    tokens = torch.tensor([3, 90, 17, 0, 55, 42], device=dev)
    results = {}
    routed = {}
    for policy in ("lru", "static"):
        for overlap in (True, False):
            kp, vp = kp0.clone(), vp0.clone()
            dec = MoePagedDecoder(w, cfg, _cache(dev, cfg, banks, policy), kp, vp,
                                  max_batch=len(lens), overlap=overlap)
            dec.layer_hook = lambda l, d: routed.__setitem__(l, d["topk_ids"].cpu())
            results[(policy, overlap)] = dec.step(tokens, batch).cpu()
    ref0 = results[("lru", False)]
    for key, got in results.items():
        assert torch.equal(got, ref0), f"{key} differs from the reference order"
    wc = {k: v.cpu() for k, v in w.items()}
    kp, vp = kp0.cpu(), vp0.cpu()
    k = cfg.n_experts_per_tok
    rows = []
    for b in range(len(lens)):
        logits = []
        gpu_ids = [routed[l][b] for l in range(cfg.n_layers)]
        rows.append(OD.decode_step(wc, cfg, banks, kp, vp, tables[b], lens[b] - 1,
                                   int(tokens[b]), P, route_ids=gpu_ids, router_logits=logits))
        for l in range(cfg.n_layers):
            own = torch.topk(logits[l].float(), k + 1)
            if set(own.indices[:k].tolist()) != set(gpu_ids[l].tolist()):
                gap = (own.values[k - 1] - own.values[k]).item()
                assert gap <= 4 * 2 ** -8 * own.values[k - 1].abs().item(), (b, l, gap)
    ref = torch.stack(rows)
    err = (ref0.float() - ref.float()).abs().max().item() / ref.float().abs().max().item()
    assert err <= 3e-2, err


def test_qwen3_30b_a3b_layer_shape_two_layers(dev):
    cfg = MoeModelConfig(n_layers=2, n_heads=32, n_kv_heads=4, head_dim=128, hidden_dim=2048,
                         vocab_size=4096, max_seq_len=4096, n_experts=128, n_experts_per_tok=8,
                         moe_intermediate_dim=768)
    B, ctx = 64, 4096
    n_pages = 2 * B * ctx // P + 8
    w = random_dense_weights(cfg, dev, seed=11)
    banks = random_expert_banks(cfg, dev, seed=12)
    kp0, vp0 = _pools(dev, n_pages, cfg.n_kv_heads, cfg.head_dim, 13)
    batch, tables = _batch(dev, cfg, [ctx] * B, n_pages, 14)
    tokens = torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(15))
    tokens = tokens.to(dev)
    logits = {}
    for policy in ("static", "lru"):
        kp, vp = kp0.clone(), vp0.clone()
        cache = _cache(dev, cfg, banks, policy)
        dec = MoePagedDecoder(w, cfg, cache, kp, vp, max_batch=B, overlap=True)
        seen = {}

        def hook(l, d, cache=cache):
            seen[l] = {k: v for k, v in d.items() if k != "events"}
            # slot rows of every routed expert, bit-exact, compared on the device before the
            # next layer's copies reuse the staging slots
            torch.cuda.synchronize(dev)
            u, first = np.unique(d["topk_ids"].cpu().numpy().reshape(-1), return_index=True)
            su = d["slots"].reshape(-1)[torch.from_numpy(first).to(dev)].long()
            for name, bank in banks.items():
                host = bank[l][torch.from_numpy(u)].to(dev)
                assert torch.equal(cache.bank_caches[name][su], host), (policy, l, name)

        dec.layer_hook = hook
        logits[policy] = dec.step(tokens, batch)
        torch.cuda.synchronize(dev)
        if policy != "static":
            continue
        picks = [0, 17, 40, 63]
        for l in range(cfg.n_layers):
            d = seen[l]
            ids = d["topk_ids"]
            # attention of sampled rows against the oracle, from the pool after this layer
            ids_sel = torch.tensor(picks)
            pages = sorted({p for b in picks for p in tables[b][l]})
            remap = {p: i for i, p in enumerate(pages)}
            sel = torch.tensor(pages, device=dev)
            kl, vl = kp.index_select(0, sel).cpu(), vp.index_select(0, sel).cpu()
            bt = torch.tensor([[remap[p] for p in tables[b][l]] for b in picks], dtype=torch.int32)
            ref_attn = OP.decode_batch(d["q"][ids_sel.to(dev)].cpu(), kl, vl, bt,
                                       [ctx] * len(picks), P)
            err = (d["attn"][ids_sel.to(dev)].cpu().float() - ref_attn.float()).abs().max().item()
            assert err <= 2e-2, (l, err)
            # routed FFN of sampled tokens against the oracle (host banks, routed expert ids)
            x = d["moe_in"][ids_sel.to(dev)].cpu()
            tw = d["topk_weights"][ids_sel.to(dev)].cpu()
            ti = ids[ids_sel.to(dev)].cpu()
            used = torch.unique(ti)
            remap_e = torch.full((cfg.n_experts,), -1, dtype=torch.int64)
            remap_e[used] = torch.arange(used.numel())
            ref_ffn = OF.fused_experts(x, banks["gate_up"][l][used], banks["down"][l][used], tw,
                                       remap_e[ti.long()].to(torch.int32))
            got = d["routed"][ids_sel.to(dev)].cpu().float()
            rel = (got - ref_ffn.float()).abs().max().item() / ref_ffn.float().abs().max().item()
            assert rel < 1e-2, (l, rel)
    assert torch.equal(logits["static"].cpu(), logits["lru"].cpu())
    assert torch.isfinite(logits["static"].float()).all()


def test_qwen3_30b_a3b_full_depth_step(dev):
    """Config 5 at full depth, in the order the product runs: one MoePagedDecoder.step over the
    48-layer Qwen3-30B-A3B (64 rows x 4096 context, 32 q / 4 kv heads, 128 experts top-8,
    expert slots for 50 % of the 6144 experts) under both residency policies, with the
    overlapped FFN. The layer hook only keeps tensors (device gathers of the routed experts'
    slot rows, enqueued on the compute stream; no synchronisation), so layers run as they do
    in the product. After the step: the slot rows every route of layers 0, 23 and 47 read equal
    the host banks bit for bit; the attention (2e-2) and routed FFN (1e-2 of its largest
    magnitude) of sampled rows of those layers equal the oracle's; both policies give
    bit-identical finite logits; the global LRU over 3072 slots admits every expert it is
    routed to (hit rate 0: the 48 layers route ~6000 distinct experts per step), the static
    policy serves the resident half from HBM (hit rate ~0.5)."""
    from plastic_infer.exec.runner_moe_paged import qwen3_30b_a3b_config

    cfg = qwen3_30b_a3b_config(n_layers=48, max_seq_len=4096)
    cfg.vocab_size = 4096             # the LM head's size does not touch the path under test
    L, E = cfg.n_layers, cfg.n_experts
    B, ctx = 64, 4096
    n_pages = L * B * ctx // P
    w = random_dense_weights(cfg, dev, seed=51)
    banks = random_expert_banks(cfg, dev, seed=52)
    kp0, vp0 = _pools(dev, n_pages, cfg.n_kv_heads, cfg.head_dim, 53)
    batch, tables = _batch(dev, cfg, [ctx] * B, n_pages, 54)
    tokens = torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(55))
    tokens = tokens.to(dev)
    checked = (0, 23, 47)
    picks = [0, 21, 42, 63]
    logits, rates = {}, {}
    for policy in ("static", "lru"):
        kp, vp = kp0.clone(), vp0.clone()
        cache = _cache(dev, cfg, banks, policy)
        cache.collect_stats = True
        dec = MoePagedDecoder(w, cfg, cache, kp, vp, max_batch=B, overlap=True)
        seen = {}

        def hook(l, d, cache=cache):
            if l not in checked:
                return
            # clamped so that the gather stays in bounds whatever the slots hold; every slot is
            # checked to be a real one after the step
            rows = d["slots"].reshape(-1).long().clamp(0, cache.cache_size - 1)
            seen[l] = {k: d[k] for k in ("q", "attn", "moe_in", "topk_weights", "topk_ids",
                                           "routed", "slots")}
            seen[l]["rows"] = {n: cache.bank_caches[n].index_select(0, rows)
                               for n in ("gate_up", "down")}

        dec.layer_hook = hook
        logits[policy] = dec.step(tokens, batch)
        torch.cuda.synchronize(dev)
        rates[policy] = cache.decode_miss_stats()
        assert rates[policy]["layer_calls"] == L
        for l in checked:
            d = seen[l]
            assert bool((d["slots"] >= 0).all()), (policy, l)
            ids = d["topk_ids"].reshape(-1).long().cpu()
            for name in ("gate_up", "down"):
                host = banks[name][l].index_select(0, ids).to(dev)
                assert torch.equal(d["rows"][name], host), (policy, l, name)
            del d["rows"]
            if policy != "static":
                continue
            sel = torch.tensor(picks, device=dev)
            pages = sorted({p for b in picks for p in tables[b][l]})
            remap = {p: i for i, p in enumerate(pages)}
            psel = torch.tensor(pages, device=dev)
            kl, vl = kp.index_select(0, psel).cpu(), vp.index_select(0, psel).cpu()
            bt = torch.tensor([[remap[p] for p in tables[b][l]] for b in picks], dtype=torch.int32)
            ref_attn = OP.decode_batch(d["q"][sel].cpu(), kl, vl, bt, [ctx] * len(picks), P)
            err = (d["attn"][sel].cpu().float() - ref_attn.float()).abs().max().item()
            assert err <= 2e-2, (l, err)
            x, tw, ti = d["moe_in"][sel].cpu(), d["topk_weights"][sel].cpu(), \
                d["topk_ids"][sel].cpu()
            used = torch.unique(ti)
            remap_e = torch.full((E,), -1, dtype=torch.int64)
            remap_e[used] = torch.arange(used.numel())
            ref_ffn = OF.fused_experts(x, banks["gate_up"][l][used], banks["down"][l][used], tw,
                                       remap_e[ti.long()].to(torch.int32))
            got = d["routed"][sel].cpu().float()
            rel = (got - ref_ffn.float()).abs().max().item() / ref_ffn.float().abs().max().item()
            assert rel < 1e-2, (l, rel)
        del dec, cache, kp, vp, seen
        torch.cuda.empty_cache()
    assert torch.equal(logits["static"].cpu(), logits["lru"].cpu())
    assert torch.isfinite(logits["static"].float()).all()
    assert rates["lru"]["hit_rate"] == 0.0, rates["lru"]
    assert 0.4 < rates["static"]["hit_rate"] < 0.6, rates["static"]
