"""Paged attention ops with the reference's call signatures, executed by the HIP library.

  gather_paged_kv          reference src/plastic_infer/exec/attention.py:103-148
  paged_attention_v1       reference src/plastic_infer/exec/attention.py:151-190
  host_stream_attention_v1 reference src/plastic_infer/exec/attention.py:193-250

Semantics kept from the reference:
  * K/V pools are [num_pages, n_kv_heads, head_dim, page_size]; block_table is the request's
    list of physical pages in logical order; num_tokens / kv_num_tokens trims the last page.
  * GQA: query head h reads kv head h // (H / H_kv).
  * causal=True follows torch SDPA is_causal: query row i attends keys j <= i (top-left
    alignment, so a single decode row with causal=True sees key 0 only). Decode callers pass
    causal=False, as the reference runner does (src/plastic_infer/exec/runner_paged.py:253-255).
  * host_stream_attention_v1: row i of q sits at position q_start_pos + i and, when causal,
    attends keys j <= q_start_pos + i.
Unlike the reference there is no gather-then-SDPA: the kernels read pages in place (the
gather_paged_kv entry point itself is the one op that materialises contiguous K/V).

RoPE / RMSNorm helpers are re-exported for import compatibility of this module; they are plain
torch elementwise code and not part of the paged data path.
"""

from __future__ import annotations

import torch

from .. import _native as N
from ..kernel.host_stream import host_stream_attention
from ..kernel.paged_kv import kv_gather, paged_attention, paged_decode_attention


def _table_tensor(block_table: list[int], device: torch.device, num_pages: int) -> torch.Tensor:
    """The table as an int32 [1, n] device row. Every listed id must name a pool page: the
    reference index_selects the whole list (src/plastic_infer/exec/attention.py:134-136), which
    raises IndexError for an id < 0 or >= num_pages."""
    ids = [int(x) for x in block_table]
    if ids and (min(ids) < 0 or max(ids) >= num_pages):
        raise IndexError("index out of range in self")
    return torch.tensor([ids], dtype=torch.int32).to(device, non_blocking=True)


def gather_paged_kv(k_pages: torch.Tensor, v_pages: torch.Tensor, block_table: list[int],
                    page_size: int, num_tokens: int | None = None
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """Contiguous K, V [1, T, n_kv_heads, head_dim] of the pages in block_table (logical order),
    T = min(num_tokens, len(block_table) * page_size) (all pages when num_tokens is None)."""
    dev = N.require_device(k_pages, v_pages, names=("k_pages", "v_pages"))
    if k_pages.shape[3] != page_size:
        raise ValueError(f"page_size {page_size} does not match the pool's {k_pages.shape[3]}")
    _, H, D, P = k_pages.shape
    cap = len(block_table) * P
    T = cap if num_tokens is None else max(0, min(int(num_tokens), cap))
    bt = _table_tensor(block_table, dev, k_pages.shape[0])
    if T == 0:
        empty = torch.empty(1, 0, H, D, dtype=k_pages.dtype, device=dev)
        return empty, empty.clone()
    cu = torch.tensor([0, T], dtype=torch.int64).to(dev, non_blocking=True)
    k, v = kv_gather(k_pages, v_pages, bt, cu, T,
                     out=(torch.empty(T, H, D, dtype=k_pages.dtype, device=dev),
                          torch.empty(T, H, D, dtype=k_pages.dtype, device=dev)))
    return k.unsqueeze(0), v.unsqueeze(0)


def paged_attention_v1(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                       block_table: list[int], page_size: int, kv_num_tokens: int | None = None,
                       causal: bool = True) -> torch.Tensor:
    """Attention of q [1, Sq, H, D] over the request's paged KV. Returns [1, Sq, H, D]."""
    dev = N.require_device(q, k_pages, v_pages, names=("q", "k_pages", "v_pages"))
    if k_pages.shape[3] != page_size:
        raise ValueError(f"page_size {page_size} does not match the pool's {k_pages.shape[3]}")
    if q.dim() != 4 or q.shape[0] != 1:
        raise ValueError("q must be [1, q_len, n_heads, head_dim]")
    _, Sq, Hq, D = q.shape
    P = k_pages.shape[3]
    cap = len(block_table) * P
    kv_len = cap if kv_num_tokens is None else max(0, min(int(kv_num_tokens), cap))
    if Hq % k_pages.shape[1]:
        raise AssertionError("n_heads must be a multiple of n_kv_heads")
    if Sq == 0:
        return torch.empty_like(q)
    if not block_table:
        return torch.zeros_like(q)
    bt = _table_tensor(block_table, dev, k_pages.shape[0])
    lens = torch.tensor([kv_len], dtype=torch.int32).to(dev, non_blocking=True)
    q3 = q[0]
    if Sq == 1 and not causal:
        out = paged_decode_attention(q3, k_pages, v_pages, bt, lens)
    else:
        cu = torch.tensor([0, Sq], dtype=torch.int32).to(dev, non_blocking=True)
        offs = torch.zeros(1, dtype=torch.int32, device=dev) if causal else None
        out = paged_attention(q3, k_pages, v_pages, bt, lens, cu_q=cu, q_pos_offsets=offs)
    return out.unsqueeze(0)


def host_stream_attention_v1(q: torch.Tensor,
                             host_chunks: list[tuple[torch.Tensor, torch.Tensor]],
                             resident_k: torch.Tensor, resident_v: torch.Tensor,
                             q_start_pos: int = 0, causal: bool = True) -> torch.Tensor:
    """Attention over KV split into host chunks ([H_kv, D, C] each, oldest first) and a device
    resident tail [1, R, H_kv, D]; q [1, q_len, H, D] at positions q_start_pos.. (reference
    src/plastic_infer/exec/attention.py:193-250, same mask rule). The chunks are not
    concatenated: the HIP kernel reads pinned host chunks in place over the host link (decode
    shapes) and device chunks where they are, merging per-split online-softmax partials."""
    N.require_device(q, resident_k, resident_v, names=("q", "resident_k", "resident_v"))
    if q.dim() != 4 or q.shape[0] != 1 or resident_k.dim() != 4 or resident_k.shape[0] != 1:
        raise ValueError("q must be [1, q_len, n_heads, head_dim] and the resident tail "
                         "[1, R, n_kv_heads, head_dim]")
    out = host_stream_attention(q[0], list(host_chunks), resident_k[0], resident_v[0],
                                q_start_pos=q_start_pos, causal=causal)
    return out.unsqueeze(0)


# ---------------------------------------------------------------------------------------------
# Elementwise model helpers (import compatibility; not part of the paged data path)
# ---------------------------------------------------------------------------------------------

def rope_positions(cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                   x: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [B, S, H, D] at `positions` with cos/sin tables [seq, D]."""
    c = cos[positions][None, :, None, :]
    s = sin[positions][None, :, None, :]
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * c + rot * s


def build_rope_cache(seq_len: int, head_dim: int, base: float = 10000.0,
                     device: torch.device | None = None,
                     dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [seq_len, head_dim] with the frequency list repeated over both halves."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=dtype, device=device) / head_dim))
    ang = torch.outer(torch.arange(seq_len, dtype=dtype, device=device), inv)
    ang = torch.cat((ang, ang), dim=-1)
    return ang.cos(), ang.sin()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    return x / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * weight


def qk_norm(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
            head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    return (rms_norm(q.reshape(-1, head_dim), q_weight).view(q.shape),
            rms_norm(k.reshape(-1, head_dim), k_weight).view(k.shape))


__all__ = [
    "gather_paged_kv", "paged_attention_v1", "host_stream_attention_v1",
    "rope_positions", "build_rope_cache", "rms_norm", "qk_norm",
]
