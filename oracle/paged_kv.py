"""ORACLE (test infrastructure only): CPU restatement of the reference's paged-KV torch path.

Layout: k_pages / v_pages [num_pages, n_kv_heads, head_dim, page_size] (token innermost),
reference src/plastic_infer/kv/kv_store.py:18-22,86-88.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def scatter_slots(k: torch.Tensor, v: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                  slot_mapping) -> None:
    """In place: k_pages[s // P, :, :, s % P] = k[i] for s = slot_mapping[i] (s < 0 skipped).

    Restates the per-token advanced-index store of _write_kv_layer
    (reference src/plastic_infer/exec/runner_paged.py:123-129) and of
    KVRequestCache.append_token (src/plastic_infer/kv/kv_store.py:140-143), with the slot
    s = page * P + offset. Tokens are applied in order, so a repeated slot keeps the last write.
    """
    P = k_pages.shape[3]
    slots = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    for i, s in enumerate(slots.tolist()):
        if s < 0:
            continue
        k_pages[s // P, :, :, s % P] = k[i]
        v_pages[s // P, :, :, s % P] = v[i]


def write_kv_layer(block_table_row: list[int], page_size: int, start_pos: int,
                   k: torch.Tensor, v: torch.Tensor, k_pages: torch.Tensor,
                   v_pages: torch.Tensor) -> None:
    """reference src/plastic_infer/exec/runner_paged.py:112-129 for one layer:
    token t of k [S, H, D] goes to page block_table_row[(start_pos+t)//P], offset (start_pos+t)%P."""
    for t in range(k.shape[0]):
        g = start_pos + t
        phys = block_table_row[g // page_size]
        k_pages[phys, :, :, g % page_size] = k[t]
        v_pages[phys, :, :, g % page_size] = v[t]


def gather_paged_kv(k_pages: torch.Tensor, v_pages: torch.Tensor, block_table: list[int],
                    page_size: int, num_tokens: int | None = None
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """reference src/plastic_infer/exec/attention.py:103-148: index_select of the table's pages,
    permute [n, H, D, P] -> [n, P, H, D], reshape to tokens, trim to num_tokens, batch dim."""
    if not block_table:
        H, D = k_pages.shape[1], k_pages.shape[2]
        e = torch.empty(1, 0, H, D, dtype=k_pages.dtype)
        return e, e.clone()
    ids = torch.tensor(block_table, dtype=torch.long)
    kg = k_pages.index_select(0, ids)
    vg = v_pages.index_select(0, ids)
    n, H, D, _ = kg.shape
    k = kg.permute(0, 3, 1, 2).reshape(n * page_size, H, D)
    v = vg.permute(0, 3, 1, 2).reshape(n * page_size, H, D)
    if num_tokens is not None:
        k, v = k[:num_tokens], v[:num_tokens]
    return k.unsqueeze(0), v.unsqueeze(0)


def paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                    block_table: list[int], page_size: int, kv_num_tokens: int | None = None,
                    causal: bool = True, q_start_pos: int = 0) -> torch.Tensor:
    """reference src/plastic_infer/exec/attention.py:151-190 (gather, GQA repeat_interleave,
    SDPA with is_causal) and, for q_start_pos > 0 with causal, the explicit offset mask of
    src/plastic_infer/exec/runner_paged.py:61-95. q [1, Sq, H, D] -> [1, Sq, H, D]."""
    k, v = gather_paged_kv(k_pages, v_pages, block_table, page_size, kv_num_tokens)
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    H, Hkv = qt.shape[1], kt.shape[1]
    if H != Hkv:
        kt = kt.repeat_interleave(H // Hkv, dim=1)
        vt = vt.repeat_interleave(H // Hkv, dim=1)
    if causal and q_start_pos > 0:
        q_len, kv_len = qt.shape[2], kt.shape[2]
        qp = torch.arange(q_start_pos, q_start_pos + q_len)
        kp = torch.arange(kv_len)
        mask = torch.zeros(q_len, kv_len, dtype=q.dtype).masked_fill(
            ~(kp[None, :] <= qp[:, None]), float("-inf"))
        out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask[None, None])
    else:
        out = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)
    return out.transpose(1, 2)


def decode_batch(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                 block_tables: torch.Tensor, context_lens, page_size: int) -> torch.Tensor:
    """Batched decode as the reference runs it: one paged_attention_v1 call per sequence with
    kv_num_tokens = L_b and causal=False (src/plastic_infer/exec/runner_paged.py:253-255).
    q [B, Hq, D] -> [B, Hq, D] (q's dtype)."""
    B = q.shape[0]
    out = torch.empty_like(q)
    lens = [int(x) for x in np.asarray(context_lens).reshape(-1)]
    bt = np.asarray(block_tables)
    for b in range(B):
        L = lens[b]
        n = (L + page_size - 1) // page_size
        table = [int(x) for x in bt[b, :n]]
        out[b] = paged_attention(q[b][None, None], k_pages, v_pages, table, page_size,
                                 kv_num_tokens=L, causal=False)[0, 0]
    return out


def host_stream_attention(q: torch.Tensor, host_chunks, resident_k: torch.Tensor,
                          resident_v: torch.Tensor, q_start_pos: int = 0,
                          causal: bool = True) -> torch.Tensor:
    """reference src/plastic_infer/exec/attention.py:193-250: concatenate host chunks
    ([H, D, C] -> [C, H, D]) and the resident tail, GQA expand, offset-causal SDPA."""
    k_full = torch.cat([k.permute(2, 0, 1) for k, _ in host_chunks] + [resident_k[0]]).unsqueeze(0)
    v_full = torch.cat([v.permute(2, 0, 1) for _, v in host_chunks] + [resident_v[0]]).unsqueeze(0)
    qt, kt, vt = q.transpose(1, 2), k_full.transpose(1, 2), v_full.transpose(1, 2)
    H, Hkv = qt.shape[1], kt.shape[1]
    if H != Hkv:
        kt = kt.repeat_interleave(H // Hkv, dim=1)
        vt = vt.repeat_interleave(H // Hkv, dim=1)
    q_len, kv_len = qt.shape[2], kt.shape[2]
    if causal and (q_start_pos > 0 or q_len != kv_len):
        qp = torch.arange(q_start_pos, q_start_pos + q_len)
        kp = torch.arange(kv_len)
        mask = torch.zeros(q_len, kv_len, dtype=q.dtype).masked_fill(
            ~(kp[None, :] <= qp[:, None]), float("-inf"))
        out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask[None, None])
    else:
        out = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)
    return out.transpose(1, 2)


def pages_to_chunk(pages: torch.Tensor, page_ids: list[int], n_layers: int,
                   pages_per_chunk: int) -> torch.Tensor:
    """reference src/plastic_infer/kv/kv_store.py:249-266: chunk[l, :, :, p*P:(p+1)*P] =
    pages[page_ids[l*ppc + p]] (absent pages, id < 0, stay zero)."""
    N_, H, D, P = pages.shape
    out = torch.zeros(n_layers, H, D, pages_per_chunk * P, dtype=pages.dtype)
    for l in range(n_layers):
        for p in range(pages_per_chunk):
            pid = page_ids[l * pages_per_chunk + p]
            if pid >= 0:
                out[l, :, :, p * P:(p + 1) * P] = pages[pid]
    return out
