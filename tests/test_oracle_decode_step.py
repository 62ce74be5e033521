"""Pins the decode-step oracle (oracle/moe_decode_step.py) on the CPU against transformers'
Qwen3MoeForCausalLM with the same fp32 weights: a prompt decoded one token at a time through
the paged oracle (each step writes its K / V into pages of a shuffled block table and attends
every earlier position) gives the logits HF's full causal forward gives at every position.

Planted mistakes (each must break the agreement): RoPE left out, q rotated one position ahead
of k (a shift of both is invisible: RoPE scores see only relative positions), the q / k norm
skipped, the experts' weights not renormalised, attention restricted to the previous tokens.
"""

from __future__ import annotations

import types

import pytest
import torch

import oracle.moe_decode_step as OD

transformers = pytest.importorskip("transformers")
from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM  # noqa: E402

L, H, HQ, HKV, D, E, K, I, V, P = 2, 64, 4, 2, 16, 8, 2, 24, 50, 4


def _model(seed: int):
    torch.manual_seed(seed)
    cfg = Qwen3MoeConfig(vocab_size=V, hidden_size=H, intermediate_size=96, num_hidden_layers=L,
                         num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
                         max_position_embeddings=64, rms_norm_eps=1e-5, num_experts=E,
                         num_experts_per_tok=K, moe_intermediate_size=I, norm_topk_prob=True,
                         decoder_sparse_step=1, mlp_only_layers=[], tie_word_embeddings=False,
                         rope_parameters={"rope_theta": 10000.0, "rope_type": "default"},
                         attn_implementation="eager")
    m = Qwen3MoeForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.3 * torch.randn_like(p))
            else:
                p.copy_(0.3 * torch.randn_like(p))
    sd = {k: v.detach() for k, v in m.state_dict().items()}
    w = {"embed_tokens.weight": sd["model.embed_tokens.weight"],
         "norm.weight": sd["model.norm.weight"], "lm_head.weight": sd["lm_head.weight"]}
    banks = {"gate_up": [], "down": []}
    for l in range(L):
        src, dst = f"model.layers.{l}.", f"layers.{l}."
        for n in ("input_layernorm", "post_attention_layernorm"):
            w[dst + n + ".weight"] = sd[src + n + ".weight"]
        for n in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
            w[dst + "self_attn." + n + ".weight"] = sd[src + "self_attn." + n + ".weight"]
        w[dst + "mlp.router.weight"] = sd[src + "mlp.gate.weight"]
        banks["gate_up"].append(sd[src + "mlp.experts.gate_up_proj"])
        banks["down"].append(sd[src + "mlp.experts.down_proj"])
    ocfg = types.SimpleNamespace(n_layers=L, n_heads=HQ, n_kv_heads=HKV, head_dim=D,
                                 n_experts_per_tok=K, max_seq_len=64, rope_base=10000.0,
                                 qk_norm=True, dtype=torch.float32)
    return m, w, banks, ocfg


def _oracle_logits(w, banks, ocfg, tokens, seed):
    g = torch.Generator().manual_seed(seed)
    n_pages = L * ((len(tokens) + P - 1) // P)
    perm = torch.randperm(n_pages + 3, generator=g).tolist()
    per = (len(tokens) + P - 1) // P
    tables = [perm[l * per:(l + 1) * per] for l in range(L)]
    kp = torch.zeros(n_pages + 3, HKV, D, P)
    vp = torch.zeros_like(kp)
    return torch.stack([OD.decode_step(w, ocfg, banks, kp, vp, tables, pos, int(t), P)
                        for pos, t in enumerate(tokens)])


@pytest.mark.parametrize("seed", [0, 1])
def test_decode_oracle_matches_hf_qwen3_moe(seed):
    m, w, banks, ocfg = _model(seed)
    tokens = torch.randint(0, V, (11,), generator=torch.Generator().manual_seed(seed + 10))
    with torch.no_grad():
        ref = m(tokens[None]).logits[0]
    got = _oracle_logits(w, banks, ocfg, tokens, seed)
    assert torch.allclose(got, ref, rtol=1e-4, atol=1e-4), (got - ref).abs().max()


def test_planted_mistakes_break_the_agreement(monkeypatch):
    m, w, banks, ocfg = _model(3)
    tokens = torch.randint(0, V, (9,), generator=torch.Generator().manual_seed(13))
    with torch.no_grad():
        ref = m(tokens[None]).logits[0]

    def far(**kw):
        got = _oracle_logits(w, banks, ocfg, tokens, 3)
        return (got - ref).abs().max().item()

    assert far() < 1e-4
    rope = OD.rope
    monkeypatch.setattr(OD, "rope", lambda x, c, s, pos: x)
    assert far() > 1e-2
    monkeypatch.setattr(OD, "rope",
                        lambda x, c, s, pos: rope(x, c, s, pos + (1 if x.shape[0] == HQ else 0)))
    assert far() > 1e-2
    monkeypatch.setattr(OD, "rope", rope)
    monkeypatch.setattr(ocfg, "qk_norm", False)
    assert far() > 1e-2
    monkeypatch.setattr(ocfg, "qk_norm", True)
    topk = OD.OR.fused_topk
    monkeypatch.setattr(OD.OR, "fused_topk", lambda lg, k, renormalize=True: topk(lg, k, False))
    assert far() > 1e-2
    monkeypatch.setattr(OD.OR, "fused_topk", topk)
    attn = OD.OP.paged_attention
    monkeypatch.setattr(OD.OP, "paged_attention",
                        lambda q, kp, vp, t, ps, kv_num_tokens=None, causal=True:
                        attn(q, kp, vp, t, ps, kv_num_tokens=max(1, kv_num_tokens - 1),
                             causal=causal))
    assert far() > 1e-2
