"""Batched MoE decode step over the paged KV pool and the expert slot cache.

Per-request semantics of the reference's decode_step_moe_paged
(src/plastic_infer/exec/runner_moe_paged.py:101-162) with its routed FFN _moe_ffn /
_decode_routed (src/plastic_infer/exec/runner_moe.py:108-146), run for a batch of B sequences
at once. Every layer of a step does, for all B rows:

  input RMSNorm -> q / k / v projections -> per-head q / k RMSNorm -> RoPE at each row's own
  position -> slot scatter of the new K / V rows (one launch) -> GQA paged decode attention
  over each row's block table (one launch) -> o projection + residual -> post-attention
  RMSNorm -> router logits -> softmax top-k with renormalised weights -> routed expert FFN
  over the slot cache -> residual;

then the final RMSNorm and the LM head give [B, vocab] logits. The projections, norms and RoPE
are plain torch ops in the model dtype with the reference's formulas (RoPE tables built in the
model dtype, as the reference builds them); the KV, attention, routing and expert data path is
this package's HIP kernels.

Routed experts, overlapped (overlap=True): the cache plans the layer's misses on the host and
copies them with the DMA engines on its copy stream (OffloadMoeCache.stage_layer); the FFN of
the routes whose experts are already in HBM runs on the compute stream meanwhile, then the
compute stream waits on the copies' event and runs the copied routes; one sum over the k
routes of each token gives a result bit-identical to a single FFN over all routes.
overlap=False is the reference's order: ensure_experts, copy_missing, one FFN.

The reference writes a zero K / V row for every layer before the real one
(decode_step_moe_paged's dummy append, :119-122); each position is written once here, by the
scatter, before attention reads it, so the zero writes are skipped.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from ..kernel.moe_ops import moe_sum_reduce
from ..kernel.paged_kv import decode_workspace_bytes, paged_decode_append_attention
from ..kernel.pinned import alloc_pinned_exact
from ..moe.fused import fused_experts_decode_impl, fused_topk, routed_ffn_routes
from ..moe.offload_cache import OffloadMoeCache
from .attention import build_rope_cache, rms_norm


@dataclass
class MoeModelConfig:
    """The model fields the decode step needs (names of the reference's ModelConfig,
    src/plastic_infer/exec/runner.py:36-51)."""
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    hidden_dim: int
    vocab_size: int
    max_seq_len: int
    n_experts: int
    n_experts_per_tok: int
    moe_intermediate_dim: int
    rope_base: float = 1_000_000.0
    qk_norm: bool = True
    dtype: torch.dtype = torch.bfloat16


def qwen3_30b_a3b_config(n_layers: int = 48, max_seq_len: int = 8192) -> MoeModelConfig:
    """Qwen3-30B-A3B: 48 layers, hidden 2048, 32 q / 4 kv heads of 128, 128 experts top-8 with
    an intermediate size of 768, vocabulary 151936."""
    return MoeModelConfig(n_layers=n_layers, n_heads=32, n_kv_heads=4, head_dim=128,
                          hidden_dim=2048, vocab_size=151936, max_seq_len=max_seq_len,
                          n_experts=128, n_experts_per_tok=8, moe_intermediate_dim=768)


def random_dense_weights(cfg: MoeModelConfig, device: torch.device, seed: int = 0,
                         std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init non-expert weights under the reference's key names, N(0, std) projections
    and unit norms, drawn on the device."""
    g = torch.Generator(device=device).manual_seed(seed)
    H, D, dt = cfg.hidden_dim, cfg.head_dim, cfg.dtype

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=device) * std).to(dt)

    w = {"embed_tokens.weight": rnd(cfg.vocab_size, H), "norm.weight": torch.ones(H, dtype=dt,
                                                                                  device=device),
         "lm_head.weight": rnd(cfg.vocab_size, H)}
    for l in range(cfg.n_layers):
        p = f"layers.{l}."
        w[p + "input_layernorm.weight"] = torch.ones(H, dtype=dt, device=device)
        w[p + "post_attention_layernorm.weight"] = torch.ones(H, dtype=dt, device=device)
        w[p + "self_attn.q_proj.weight"] = rnd(cfg.n_heads * D, H)
        w[p + "self_attn.k_proj.weight"] = rnd(cfg.n_kv_heads * D, H)
        w[p + "self_attn.v_proj.weight"] = rnd(cfg.n_kv_heads * D, H)
        w[p + "self_attn.o_proj.weight"] = rnd(H, cfg.n_heads * D)
        w[p + "self_attn.q_norm.weight"] = torch.ones(D, dtype=dt, device=device)
        w[p + "self_attn.k_norm.weight"] = torch.ones(D, dtype=dt, device=device)
        w[p + "mlp.router.weight"] = rnd(cfg.n_experts, H)
    return w


def random_expert_banks(cfg: MoeModelConfig, device: torch.device, seed: int = 0,
                        std: float = 0.02, pin=None) -> dict[str, list[torch.Tensor]]:
    """Random-init expert banks in pinned host memory: per layer gate_up [E, 2I, H] (gate rows
    then up rows) and down [E, H, I], drawn on the device one layer at a time and copied out.
    pin(shape) allocates a pinned host tensor (default: page-locked memory of exactly the
    bank's size, kernel.pinned.alloc_pinned_exact)."""
    g = torch.Generator(device=device).manual_seed(seed)
    E, H, I = cfg.n_experts, cfg.hidden_dim, cfg.moe_intermediate_dim
    alloc = pin or (lambda shape: alloc_pinned_exact(shape, cfg.dtype))
    banks: dict[str, list[torch.Tensor]] = {"gate_up": [], "down": []}
    for _ in range(cfg.n_layers):
        for name, shape in (("gate_up", (E, 2 * I, H)), ("down", (E, H, I))):
            host = alloc(shape)
            host.copy_((torch.randn(*shape, generator=g, device=device) * std).to(cfg.dtype))
            banks[name].append(host)
    return banks


@dataclass
class DecodeBatch:
    """Where a decode step's new tokens go and what each row attends.

    block_tables int32 [L, B, max_pages]: layer l's pages of every row; context_lens int32 [B]:
    tokens including the new one; slot_mapping int64 [L, B]: the new token's slot per layer
    (the block table's slot of position context_lens - 1, which is where the step writes it);
    positions int64 [B]: its position (context_lens - 1). All on the device."""
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    slot_mapping: torch.Tensor
    positions: torch.Tensor

    @classmethod
    def from_requests(cls, store, caches) -> "DecodeBatch":
        """Reserve the new token's position in every request (a page when one is needed, the
        reference's append order) and build the batch tensors from their block tables."""
        cfg = store.config
        P, L = cfg.page_size, cfg.n_layers
        for c in caches:
            c._ensure_pages(c.length + 1)
            c._length += 1
        lens = [c.length for c in caches]
        width = max(1, max((n + P - 1) // P for n in lens))
        bt = torch.full((L, len(caches), width), -1, dtype=torch.int32)
        slots = torch.empty(L, len(caches), dtype=torch.int64)
        for b, c in enumerate(caches):
            pos = c.length - 1
            for l in range(L):
                row = c.block_table.pages[l]
                bt[l, b, :len(row)] = torch.tensor(row, dtype=torch.int32)
                slots[l, b] = row[pos // P] * P + pos % P
        dev = store.gpu.device
        lens_t = torch.tensor(lens, dtype=torch.int32)
        return cls(bt.to(dev), lens_t.to(dev), slots.to(dev), (lens_t - 1).long().to(dev))


class MoePagedDecoder:
    """Batched decode of a random-init or loaded MoE model over one KV pool shared by all
    layers (each layer's pages are distinct page ids, as KVStore lays them out) and an
    OffloadMoeCache holding the routed experts."""

    def __init__(self, weights: dict[str, torch.Tensor], cfg: MoeModelConfig,
                 moe_cache: OffloadMoeCache, k_pages: torch.Tensor, v_pages: torch.Tensor,
                 max_batch: int, overlap: bool = True) -> None:
        self.w, self.cfg, self.cache = weights, cfg, moe_cache
        self.k_pages, self.v_pages = k_pages, v_pages
        self.overlap = overlap
        dev = k_pages.device
        self.device = dev
        self.cos, self.sin = build_rope_cache(cfg.max_seq_len, cfg.head_dim, base=cfg.rope_base,
                                              device=dev, dtype=cfg.dtype)
        P = k_pages.shape[3]
        self._ws = torch.empty(max(1, decode_workspace_bytes(
            max_batch, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, P,
            math.ceil(cfg.max_seq_len / P))), dtype=torch.uint8, device=dev)
        self.layer_hook = None   # called as hook(layer, dict of the layer's tensors)

    # ---- pieces --------------------------------------------------------------------------------

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """RoPE of x [B, heads, D], row b at position pos[b] (rotate-half form)."""
        c = self.cos[pos][:, None, :]
        s = self.sin[pos][:, None, :]
        x1, x2 = x.chunk(2, dim=-1)
        return x * c + torch.cat([-x2, x1], dim=-1) * s

    def _routed(self, layer: int, h: torch.Tensor, topk_w: torch.Tensor,
                topk_ids: torch.Tensor) -> tuple[torch.Tensor, dict]:
        gate_up, down = self.cache.bank_views()
        if not self.overlap:
            slots = topk_ids.clone()
            self.cache.ensure_experts(layer, slots)
            self.cache.copy_missing()
            return fused_experts_decode_impl(h, gate_up, down, topk_w, slots), {"slots": slots}
        routes = self.cache.stage_layer(layer, topk_ids)
        B, k = topk_ids.shape
        route_out = torch.empty(B, k, h.shape[1], dtype=h.dtype, device=h.device)
        act = torch.empty(B * k, down.shape[2], dtype=h.dtype, device=h.device)
        compute = torch.cuda.current_stream(h.device)
        ev = {}
        if routes.issued is not None:
            ev["a0"] = torch.cuda.Event(enable_timing=True)
            ev["a0"].record(compute)
        routed_ffn_routes(h, gate_up, down, topk_w, routes.in_hbm, route_out, act_buffer=act)
        if routes.issued is not None:
            ev["a1"] = torch.cuda.Event(enable_timing=True)
            ev["a1"].record(compute)
        compute.wait_event(routes.ready)
        routed_ffn_routes(h, gate_up, down, topk_w, routes.copied, route_out, act_buffer=act)
        out = torch.empty_like(h)
        moe_sum_reduce(route_out, out)
        return out, {"routes": routes, "events": ev,
                     "slots": torch.maximum(routes.in_hbm, routes.copied)}

    # ---- one step ------------------------------------------------------------------------------

    def step(self, input_ids: torch.Tensor, batch: DecodeBatch) -> torch.Tensor:
        """One decode token for every row: [B] token ids -> [B, vocab] logits."""
        cfg, w = self.cfg, self.w
        B = input_ids.shape[0]
        Hq, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        x = w["embed_tokens.weight"][input_ids].to(cfg.dtype)
        for l in range(cfg.n_layers):
            x = self.layer(l, x, batch)
        x = rms_norm(x, w["norm.weight"])
        return F.linear(x, w["lm_head.weight"])

    def layer(self, l: int, x: torch.Tensor, batch: DecodeBatch) -> torch.Tensor:
        """One decoder layer for all rows: x [B, hidden] -> [B, hidden]."""
        cfg, w = self.cfg, self.w
        B = x.shape[0]
        Hq, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        p = f"layers.{l}."
        residual = x
        h = rms_norm(x, w[p + "input_layernorm.weight"])
        q = F.linear(h, w[p + "self_attn.q_proj.weight"]).view(B, Hq, D)
        k = F.linear(h, w[p + "self_attn.k_proj.weight"]).view(B, Hkv, D)
        v = F.linear(h, w[p + "self_attn.v_proj.weight"]).view(B, Hkv, D)
        if cfg.qk_norm:
            q = rms_norm(q, w[p + "self_attn.q_norm.weight"])
            k = rms_norm(k, w[p + "self_attn.k_norm.weight"])
        q = self._rope(q, batch.positions).contiguous()
        k = self._rope(k, batch.positions).contiguous()
        v = v.contiguous()
        # the reference's _write_kv_layer then _attn_paged, as one call: the new token goes to
        # its slot and the attention takes it from k / v directly
        attn = paged_decode_append_attention(q, self.k_pages, self.v_pages,
                                             batch.block_tables[l], batch.context_lens, k, v,
                                             workspace=self._ws)
        x = residual + F.linear(attn.view(B, Hq * D), w[p + "self_attn.o_proj.weight"])
        residual = x
        h = rms_norm(x, w[p + "post_attention_layernorm.weight"])
        logits = F.linear(h, w[p + "mlp.router.weight"])
        topk_w, topk_ids = fused_topk(h, logits, cfg.n_experts_per_tok, True)
        routed, info = self._routed(l, h, topk_w, topk_ids)
        if self.layer_hook is not None:
            self.layer_hook(l, {"q": q, "k": k, "v": v, "attn": attn, "moe_in": h,
                                "topk_weights": topk_w, "topk_ids": topk_ids, "routed": routed,
                                **info})
        return residual + routed


__all__ = ["MoeModelConfig", "qwen3_30b_a3b_config", "random_dense_weights",
           "random_expert_banks", "DecodeBatch", "MoePagedDecoder"]
