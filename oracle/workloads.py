"""ORACLE (test infrastructure only): seeded synthetic inputs of the benchmark workloads.

Generation rule: one torch.Generator("cpu") per workload with a fixed seed of its own; draws in the
order lengths -> block permutation -> pools -> new K/V -> q, each drawn as fp32 N(0,1) and cast
to bf16. Block tables are consecutive slices of one permutation of the pool's pages. Context
lengths include the token written by this step.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DecodeWorkload:
    k_pages: torch.Tensor        # [N, Hkv, D, P] bf16
    v_pages: torch.Tensor
    block_tables: torch.Tensor   # int32 [B, max_pages]
    context_lens: torch.Tensor   # int32 [B] (including the new token)
    slot_mapping: torch.Tensor   # int64 [B] slot of the new token
    k_new: torch.Tensor          # [B, Hkv, D] bf16
    v_new: torch.Tensor
    q: torch.Tensor              # [B, Hq, D] bf16
    page_size: int


def _randn_bf16(g: torch.Generator, *shape: int) -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(torch.bfloat16)


def decode_workload(seed: int, num_pages: int, batch: int, len_lo: int, len_hi: int, n_heads: int,
                    n_kv_heads: int, head_dim: int = 128, page_size: int = 16,
                    max_len: int | None = None) -> DecodeWorkload:
    """Decode step: one new K/V row per sequence scattered at its slot, then attention.
    Lengths ~ U{len_lo..len_hi}; max_len (default len_hi) sizes the block-table rows."""
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(len_lo, len_hi + 1, (batch,), generator=g, dtype=torch.int64)
    perm = torch.randperm(num_pages, generator=g)
    max_pages = ((max_len or len_hi) + page_size - 1) // page_size
    n_pages = (lens + page_size - 1) // page_size
    if int(n_pages.sum()) > num_pages:
        raise ValueError("pool too small for the drawn lengths")
    bt = torch.zeros(batch, max_pages, dtype=torch.int32)
    off = 0
    for b in range(batch):
        n = int(n_pages[b])
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    k_pages = _randn_bf16(g, num_pages, n_kv_heads, head_dim, page_size)
    v_pages = _randn_bf16(g, num_pages, n_kv_heads, head_dim, page_size)
    k_new = _randn_bf16(g, batch, n_kv_heads, head_dim)
    v_new = _randn_bf16(g, batch, n_kv_heads, head_dim)
    q = _randn_bf16(g, batch, n_heads, head_dim)
    last = lens - 1
    slots = bt[torch.arange(batch), (last // page_size)].to(torch.int64) * page_size + last % page_size
    return DecodeWorkload(k_pages, v_pages, bt, lens.to(torch.int32), slots, k_new, v_new, q,
                          page_size)


def decode_b32_small() -> DecodeWorkload:
    """4096-block pool, 32 sequences of 1..2048 tokens, 16 q heads / 8 kv heads, D 128."""
    return decode_workload(1, 4096, 32, 1, 2048, 16, 8)


@dataclass
class PrefillWriteWorkload:
    k: torch.Tensor              # packed [sum S, Hkv, D] bf16
    v: torch.Tensor
    cu_seqlens: torch.Tensor     # int64 [B + 1]
    block_tables: torch.Tensor   # int32 [B, max_pages]
    slot_mapping: torch.Tensor   # int64 [sum S]
    num_pages: int
    max_len: int
    page_size: int


def prefill_write_workload(seed: int = 3, batch: int = 8, len_lo: int = 256, len_hi: int = 4096,
                           n_kv_heads: int = 8, head_dim: int = 128, page_size: int = 16,
                           spare_pages: int = 1024) -> PrefillWriteWorkload:
    """Ragged chunked-prefill write: packed rows, cu_seqlens, slots from a seeded random page
    allocation (each sequence's last page is partially filled unless S % P == 0)."""
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(len_lo, len_hi + 1, (batch,), generator=g, dtype=torch.int64)
    n_pages = (lens + page_size - 1) // page_size
    num_pages = int(n_pages.sum()) + spare_pages
    perm = torch.randperm(num_pages, generator=g)
    max_pages = (len_hi + page_size - 1) // page_size
    bt = torch.zeros(batch, max_pages, dtype=torch.int32)
    slots = []
    off = 0
    for b in range(batch):
        n = int(n_pages[b])
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
        pos = torch.arange(int(lens[b]))
        slots.append(bt[b, pos // page_size].to(torch.int64) * page_size + pos % page_size)
    total = int(lens.sum())
    k = _randn_bf16(g, total, n_kv_heads, head_dim)
    v = _randn_bf16(g, total, n_kv_heads, head_dim)
    cu = torch.zeros(batch + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(lens, 0)
    return PrefillWriteWorkload(k, v, cu, bt, torch.cat(slots), num_pages, len_hi, page_size)


@dataclass
class MoeWorkload:
    hidden: torch.Tensor   # [T, H] bf16
    logits: torch.Tensor   # [T, E] fp32
    topk: int


def moe_workload(seed: int = 4, tokens: int = 4096, hidden: int = 2048, experts: int = 128,
                 topk: int = 8) -> MoeWorkload:
    """Qwen3-30B-A3B-shaped routing: hidden ~ N(0,1) bf16, router logits ~ N(0,1) fp32."""
    g = torch.Generator("cpu").manual_seed(seed)
    h = _randn_bf16(g, tokens, hidden)
    logits = torch.randn(tokens, experts, generator=g, dtype=torch.float32)
    return MoeWorkload(h, logits, topk)
