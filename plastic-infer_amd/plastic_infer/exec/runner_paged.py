"""KV write / paged attention call sites of the paged runner (reference
src/plastic_infer/exec/runner_paged.py:36-129), batched over the HIP kernels.

Only the data-path helpers live here; the model forward of the reference runner is not part of
this package.
  _write_kv_layer   writes a run of tokens of one layer with ONE slot-mapped scatter launch
                    (reference: one advanced-index store per token, :112-129)
  _attn_paged       paged attention of one layer; q_start_pos > 0 with causal uses the offset
                    rule "key j is visible to row i iff j <= q_start_pos + i" (:61-95)
  _allocate_pages_for_tokens  reserves pages for n new tokens (reference: appends zero tokens
                    through append_token, :98-109; here only pages are allocated and the
                    length advanced — the zero writes are not needed because every position is
                    written by _write_kv_layer before it is read)
"""

from __future__ import annotations

import torch

from ..kernel.paged_kv import kv_scatter, paged_attention
from ..kv.kv_store import KVRequestCache, KVStore
from .attention import _table_tensor, paged_attention_v1


def _write_kv_layer(cache: KVRequestCache, store: KVStore, layer_idx: int, start_pos: int,
                    k: torch.Tensor, v: torch.Tensor) -> None:
    """k, v: [1, S, n_kv_heads, head_dim] for positions start_pos..start_pos+S-1."""
    S = k.shape[1]
    if S == 0:
        return
    slots = cache.slot_mapping(layer_idx, start_pos, S)
    gpu = store.gpu
    slot_t = torch.tensor(slots, dtype=torch.int64).to(gpu.device, non_blocking=True)
    kv_scatter(k[0], v[0], gpu.k_pages, gpu.v_pages, slot_t)


def _allocate_pages_for_tokens(cache: KVRequestCache, store: KVStore, n_tokens: int) -> None:
    cache._ensure_pages(cache.length + n_tokens)
    cache._length += n_tokens


def _attn_paged(q: torch.Tensor, cache: KVRequestCache, layer_idx: int, store: KVStore,
                kv_num_tokens: int | None = None, causal: bool = True,
                q_start_pos: int = 0) -> torch.Tensor:
    cfg = store.config
    block_table = cache.get_block_table_for_layer(layer_idx)
    if not causal or q_start_pos == 0:
        return paged_attention_v1(q, store.gpu.k_pages, store.gpu.v_pages, block_table,
                                  cfg.page_size, kv_num_tokens=kv_num_tokens, causal=causal)
    dev = store.gpu.device
    q_len = q.shape[1]
    kv_len = kv_num_tokens or len(block_table) * cfg.page_size
    bt = _table_tensor(block_table, dev, store.gpu.k_pages.shape[0])
    lens = torch.tensor([kv_len], dtype=torch.int32).to(dev, non_blocking=True)
    cu = torch.tensor([0, q_len], dtype=torch.int32).to(dev, non_blocking=True)
    offs = torch.tensor([q_start_pos], dtype=torch.int32).to(dev, non_blocking=True)
    out = paged_attention(q[0], store.gpu.k_pages, store.gpu.v_pages, bt, lens, cu_q=cu,
                          q_pos_offsets=offs)
    return out.unsqueeze(0)
