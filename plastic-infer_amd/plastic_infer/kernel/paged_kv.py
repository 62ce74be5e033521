"""Batched paged-KV entry points over the HIP library.

These are the batched forms of the reference's per-request ops; each row's result equals the
reference op applied to that row alone:
  kv_scatter              == the advanced-index store of _write_kv_layer / append_token
                             (reference: src/plastic_infer/exec/runner_paged.py:112-129,
                             src/plastic_infer/kv/kv_store.py:124-143)
  kv_gather               == gather_paged_kv (reference: src/plastic_infer/exec/attention.py:103-148)
  paged_decode_attention  == paged_attention_v1(q[b][None,None], ..., kv_num_tokens=L_b,
                             causal=False) (reference: src/plastic_infer/exec/attention.py:151-190,
                             src/plastic_infer/exec/runner_paged.py:253-255)
  paged_attention         == paged_attention_v1 / _attn_paged with several query rows and the
                             causal offset rule (reference: src/plastic_infer/exec/runner_paged.py:36-95)
KV pools are [num_pages, num_kv_heads, head_dim, page_size]; all tensors live on one HIP device.
"""

from __future__ import annotations

import math

import torch

from .. import _native as N


def _check_pool(k_pages: torch.Tensor, v_pages: torch.Tensor) -> None:
    if k_pages.dim() != 4 or k_pages.shape != v_pages.shape:
        raise ValueError(
            f"k_pages/v_pages must be matching [num_pages, H, D, P] tensors, got "
            f"{tuple(k_pages.shape)} / {tuple(v_pages.shape)}")
    if k_pages.dtype != v_pages.dtype:
        raise ValueError("k_pages and v_pages must share a dtype")
    if not (k_pages.is_contiguous() and v_pages.is_contiguous()):
        raise ValueError("KV pools must be contiguous")


def kv_scatter(k: torch.Tensor, v: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
               slot_mapping: torch.Tensor) -> None:
    """k_pages[s // P, :, :, s % P] = k[i] for s = slot_mapping[i] (same for v).

    k, v: [N, H, D] (token rows may be strided; a row whose [H, D] is not contiguous is copied
    first); slot_mapping: int64 [N].
    Negative slots are padding and skipped. Bit-exact.
    """
    dev = N.require_device(k, v, k_pages, v_pages, slot_mapping,
                           names=("k", "v", "k_pages", "v_pages", "slot_mapping"))
    _check_pool(k_pages, v_pages)
    num_pages, H, D, P = k_pages.shape
    if k.dim() != 3 or k.shape != v.shape or tuple(k.shape[1:]) != (H, D):
        raise ValueError(f"k/v must be [N, {H}, {D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if k.dtype != k_pages.dtype or v.dtype != k_pages.dtype:
        raise ValueError("k/v dtype must match the pool dtype")
    # The kernels read token i's row at base + i * stride(0) with heads D apart and elements
    # adjacent; any other layout (for any N, including a single strided token) is copied first.
    if not (k.stride(2) == 1 and k.stride(1) == D):
        k = k.contiguous()
    if not (v.stride(2) == 1 and v.stride(1) == D):
        v = v.contiguous()
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.numel() != k.shape[0]:
        raise ValueError("slot_mapping must be int64 [N]")
    slot_mapping = slot_mapping.contiguous()
    n = k.shape[0]
    if n == 0:
        return
    # a single token's stride(0) is never used to step (and torch may report any value for a
    # size-1 dimension): pass the packed row size
    N.call("pia_kv_scatter", k.data_ptr(), v.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(),
           slot_mapping.data_ptr(), n, k.stride(0) if n > 1 else H * D,
           v.stride(0) if n > 1 else H * D, H, D, P, num_pages, k.element_size(),
           N.stream_of(dev))


def kv_gather(k_pages: torch.Tensor, v_pages: torch.Tensor, block_tables: torch.Tensor,
              cu_seqlens: torch.Tensor, max_seq_len: int,
              out: tuple[torch.Tensor, torch.Tensor] | None = None
              ) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed gather: rows cu_seqlens[b]..cu_seqlens[b+1] of the outputs hold sequence b's
    tokens in logical order, read through block_tables[b] (int32 [B, max_pages]).

    max_seq_len must bound every sequence length (host-known, sizes the launch).
    Returns (k, v), each [total_tokens, H, D] where total_tokens = int(cu_seqlens[-1])
    unless `out` buffers are given (then their first dimension is used).
    """
    dev = N.require_device(k_pages, v_pages, block_tables, cu_seqlens,
                           names=("k_pages", "v_pages", "block_tables", "cu_seqlens"))
    _check_pool(k_pages, v_pages)
    num_pages, H, D, P = k_pages.shape
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables must be int32 [B, max_pages]")
    block_tables = block_tables.contiguous()
    cu = cu_seqlens.to(torch.int64).contiguous()
    B = block_tables.shape[0]
    if cu.numel() != B + 1:
        raise ValueError("cu_seqlens must have B + 1 entries")
    if out is None:
        total = int(cu[-1].item())
        k_out = torch.empty(total, H, D, dtype=k_pages.dtype, device=dev)
        v_out = torch.empty_like(k_out)
    else:
        k_out, v_out = out
        N.require_device(k_out, v_out, names=("k_out", "v_out"))
        if not (k_out.is_contiguous() and v_out.is_contiguous()) or k_out.shape != v_out.shape:
            raise ValueError("out buffers must be contiguous and of equal shape")
    if B and max_seq_len > 0 and block_tables.shape[1] > 0:
        N.call("pia_kv_gather", k_out.data_ptr(), v_out.data_ptr(), k_pages.data_ptr(),
               v_pages.data_ptr(), block_tables.data_ptr(), block_tables.shape[1], cu.data_ptr(),
               B, int(max_seq_len), H, D, P, num_pages, k_pages.element_size(), N.stream_of(dev))
    return k_out, v_out


def decode_workspace_bytes(num_seqs: int, num_heads: int, num_kv_heads: int, head_dim: int,
                           page_size: int, max_pages_per_seq: int) -> int:
    """Scratch bytes paged_decode_attention needs for these shapes (0 if none)."""
    return N.query("pia_paged_decode_workspace_bytes", num_seqs, num_heads, num_kv_heads,
                   head_dim, page_size, max_pages_per_seq)


def paged_decode_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor,
                           scale: float | None = None, out: torch.Tensor | None = None,
                           workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode query row per sequence. q: [B, Hq, D]; block_tables int32 [B, max_pages];
    context_lens int32 [B] (tokens including the newest). Returns [B, Hq, D] in q's dtype.
    Head hq reads kv head hq // (Hq // Hkv); scale defaults to 1/sqrt(D)."""
    dev = N.require_device(q, k_pages, v_pages, block_tables, context_lens,
                           names=("q", "k_pages", "v_pages", "block_tables", "context_lens"))
    _check_pool(k_pages, v_pages)
    num_pages, Hkv, D, P = k_pages.shape
    if q.dim() != 3 or q.shape[2] != D or q.shape[1] % Hkv:
        raise ValueError(f"q must be [B, Hq, {D}] with Hq a multiple of {Hkv}, got {tuple(q.shape)}")
    if q.dtype != k_pages.dtype:
        raise ValueError("q dtype must match the KV pool dtype")
    if not (q.stride(2) == 1 and q.stride(1) == D):
        q = q.contiguous()
    B, Hq, _ = q.shape
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError("block_tables must be int32 [B, max_pages]")
    if context_lens.dtype != torch.int32 or context_lens.shape != (B,):
        raise ValueError("context_lens must be int32 [B]")
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    elif out.shape != (B, Hq, D) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B, Hq, D] tensor of q's dtype")
    if B == 0:
        return out
    need = decode_workspace_bytes(B, Hq, Hkv, D, P, block_tables.shape[1])
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    scale = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    N.call("pia_paged_decode_attention", out.data_ptr(), q.data_ptr(), q.stride(0),
           k_pages.data_ptr(), v_pages.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
           context_lens.data_ptr(), B, Hq, Hkv, D, P, num_pages, scale, N.dtype_code(q.dtype),
           N.ptr(workspace) if need else None,
           (workspace.numel() * workspace.element_size()) if need else 0, N.stream_of(dev))
    return out


def paged_decode_append_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                                  block_tables: torch.Tensor, context_lens: torch.Tensor,
                                  k_new: torch.Tensor, v_new: torch.Tensor,
                                  scale: float | None = None, out: torch.Tensor | None = None,
                                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """A decode step's KV write and attention in one call (the reference's _write_kv_layer then
    _attn_paged, src/plastic_infer/exec/runner_paged.py:251-255): row b's new token is position
    context_lens[b] - 1, whose K / V are k_new[b] / v_new[b] ([B, Hkv, D]); they are written to
    that position's slot of block_tables[b], and the result is paged_decode_attention over the
    updated pools. The fast kernel reads the new token from k_new / v_new and writes the slot
    itself, so no write launch precedes the attention."""
    dev = N.require_device(q, k_pages, v_pages, block_tables, context_lens, k_new, v_new,
                           names=("q", "k_pages", "v_pages", "block_tables", "context_lens",
                                  "k_new", "v_new"))
    _check_pool(k_pages, v_pages)
    num_pages, Hkv, D, P = k_pages.shape
    if q.dim() != 3 or q.shape[2] != D or q.shape[1] % Hkv:
        raise ValueError(f"q must be [B, Hq, {D}] with Hq a multiple of {Hkv}, got {tuple(q.shape)}")
    if q.dtype != k_pages.dtype or k_new.dtype != k_pages.dtype or v_new.dtype != k_pages.dtype:
        raise ValueError("q, k_new and v_new dtypes must match the KV pool dtype")
    if not (q.stride(2) == 1 and q.stride(1) == D):
        q = q.contiguous()
    B, Hq, _ = q.shape
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if t.shape != (B, Hkv, D):
            raise ValueError(f"{name} must be [{B}, {Hkv}, {D}], got {tuple(t.shape)}")
    if k_new.stride() != v_new.stride() or k_new.stride(2) != 1 or k_new.stride(1) != D:
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError("block_tables must be int32 [B, max_pages]")
    if context_lens.dtype != torch.int32 or context_lens.shape != (B,):
        raise ValueError("context_lens must be int32 [B]")
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=dev)
    elif out.shape != (B, Hq, D) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B, Hq, D] tensor of q's dtype")
    if B == 0:
        return out
    need = decode_workspace_bytes(B, Hq, Hkv, D, P, block_tables.shape[1])
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    scale = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    N.call("pia_paged_decode_append_attention", out.data_ptr(), q.data_ptr(), q.stride(0),
           k_pages.data_ptr(), v_pages.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
           context_lens.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), B, Hq,
           Hkv, D, P, num_pages, scale, N.dtype_code(q.dtype),
           N.ptr(workspace) if need else None,
           (workspace.numel() * workspace.element_size()) if need else 0, N.stream_of(dev))
    return out


def paged_decode_attention_noalloc(q: torch.Tensor, k_pages: torch.Tensor,
                                   v_pages: torch.Tensor, block_tables: torch.Tensor,
                                   context_lens: torch.Tensor, out: torch.Tensor,
                                   scale: float | None = None) -> torch.Tensor:
    """paged_decode_attention for callers that cannot allocate (graph capture, serving loops):
    the caller passes every tensor, already in the layout the kernels read, and the library
    keeps its partials in a static per-GPU scratch array instead of a workspace. Nothing here
    allocates; a tensor in another layout raises instead of being copied. Calls that overlap
    on one GPU (two streams) race on the shared scratch; calls on one stream are ordered."""
    dev = N.require_device(q, k_pages, v_pages, block_tables, context_lens, out,
                           names=("q", "k_pages", "v_pages", "block_tables", "context_lens",
                                  "out"))
    _check_pool(k_pages, v_pages)
    num_pages, Hkv, D, P = k_pages.shape
    if q.dim() != 3 or q.shape[2] != D or q.shape[1] % Hkv or q.dtype != k_pages.dtype:
        raise ValueError(f"q must be [B, Hq, {D}] of the pool dtype with Hq a multiple of {Hkv}")
    if not (q.stride(2) == 1 and q.stride(1) == D):
        raise ValueError("q rows [Hq, D] must be contiguous")
    B, Hq, _ = q.shape
    if (block_tables.dtype != torch.int32 or block_tables.dim() != 2
            or block_tables.shape[0] != B or not block_tables.is_contiguous()):
        raise ValueError("block_tables must be a contiguous int32 [B, max_pages] tensor")
    if (context_lens.dtype != torch.int32 or context_lens.shape != (B,)
            or not context_lens.is_contiguous()):
        raise ValueError("context_lens must be a contiguous int32 [B] tensor")
    if out.shape != (B, Hq, D) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B, Hq, D] tensor of q's dtype")
    if B == 0:
        return out
    scale = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    N.call("pia_paged_decode_attention_noalloc", out.data_ptr(), q.data_ptr(), q.stride(0),
           k_pages.data_ptr(), v_pages.data_ptr(), block_tables.data_ptr(),
           block_tables.shape[1], context_lens.data_ptr(), B, Hq, Hkv, D, P, num_pages, scale,
           N.dtype_code(q.dtype), N.stream_of(dev))
    return out


def paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                    block_tables: torch.Tensor, kv_lens: torch.Tensor,
                    cu_q: torch.Tensor | None = None, q_pos_offsets: torch.Tensor | None = None,
                    scale: float | None = None) -> torch.Tensor:
    """General paged attention. q: [rows, Hq, D], rows of sequence b = cu_q[b]..cu_q[b+1]
    (cu_q None: one row per sequence). Row s of b attends keys j < kv_lens[b] and, when
    q_pos_offsets is given, j <= q_pos_offsets[b] + s. Returns [rows, Hq, D]."""
    dev = N.require_device(q, k_pages, v_pages, block_tables, kv_lens,
                           names=("q", "k_pages", "v_pages", "block_tables", "kv_lens"))
    _check_pool(k_pages, v_pages)
    num_pages, Hkv, D, P = k_pages.shape
    if q.dim() != 3 or q.shape[2] != D or q.shape[1] % Hkv:
        raise ValueError(f"q must be [rows, Hq, {D}] with Hq a multiple of {Hkv}")
    if q.dtype != k_pages.dtype:
        raise ValueError("q dtype must match the KV pool dtype")
    q = q.contiguous()
    rows, Hq, _ = q.shape
    B = block_tables.shape[0]
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables must be int32 [B, max_pages]")
    if kv_lens.dtype != torch.int32 or kv_lens.shape != (B,):
        raise ValueError("kv_lens must be int32 [B]")
    for name, t in (("cu_q", cu_q), ("q_pos_offsets", q_pos_offsets)):
        if t is not None:
            N.require_device(t, names=(name,))
            if t.dtype != torch.int32:
                raise ValueError(f"{name} must be int32")
    if cu_q is not None and cu_q.numel() != B + 1:
        raise ValueError("cu_q must have B + 1 entries")
    if q_pos_offsets is not None and q_pos_offsets.shape != (B,):
        raise ValueError("q_pos_offsets must be int32 [B]")
    if cu_q is None and rows != B:
        raise ValueError("without cu_q there must be exactly one query row per sequence")
    out = torch.empty(rows, Hq, D, dtype=q.dtype, device=dev)
    if rows == 0 or B == 0:
        return out
    bt = block_tables.contiguous()
    if bt.shape[1] == 0:  # no pages: every row has no admissible key
        out.zero_()
        return out
    scale = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    N.call("pia_paged_attention", out.data_ptr(), q.data_ptr(), k_pages.data_ptr(),
           v_pages.data_ptr(), bt.data_ptr(), bt.shape[1], kv_lens.contiguous().data_ptr(),
           N.ptr(None if cu_q is None else cu_q.contiguous()),
           N.ptr(None if q_pos_offsets is None else q_pos_offsets.contiguous()),
           B, rows, Hq, Hkv, D, P, num_pages, scale, N.dtype_code(q.dtype), N.stream_of(dev))
    return out


def pages_chunk_copy(chunk: torch.Tensor, pages: torch.Tensor, page_ids: torch.Tensor,
                     to_chunk: bool) -> None:
    """Copy between a chunk buffer [L, H, D, ppc*P] and pool pages listed layer-major in
    page_ids (int64 [L*ppc], -1 = absent). to_chunk: pages -> chunk, else chunk -> pages."""
    dev = N.require_device(chunk, pages, page_ids, names=("chunk", "pages", "page_ids"))
    num_pages, H, D, P = pages.shape
    L = chunk.shape[0]
    if chunk.dim() != 4 or tuple(chunk.shape[1:3]) != (H, D) or chunk.shape[3] % P:
        raise ValueError(f"chunk must be [L, {H}, {D}, ppc*{P}], got {tuple(chunk.shape)}")
    ppc = chunk.shape[3] // P
    if page_ids.dtype != torch.int64 or page_ids.numel() != L * ppc:
        raise ValueError(f"page_ids must be int64 [{L * ppc}]")
    if chunk.dtype != pages.dtype or not chunk.is_contiguous() or not pages.is_contiguous():
        raise ValueError("chunk and pages must be contiguous and share a dtype")
    N.call("pia_kv_pages_chunk_copy", chunk.data_ptr(), pages.data_ptr(),
           page_ids.contiguous().data_ptr(), L, ppc, H, D, P, num_pages, pages.element_size(),
           1 if to_chunk else 0, N.stream_of(dev))


def pages_chunks_copy(chunks: list[torch.Tensor], pages: torch.Tensor, page_ids: torch.Tensor,
                      to_chunk: bool) -> None:
    """pages_chunk_copy for many chunks in one launch. chunks: [L, H, D, ppc*P] contiguous
    tensors of the pool's dtype, each on the pool's device or pinned on the host (reached
    through its device mapping, so a sink writes host memory directly and a prefix load reads
    it, with no device staging); page_ids int64 [len(chunks) * L * ppc] on the pool's device,
    chunk-major then layer-major, -1 = absent. Asynchronous on the current stream: host chunks
    hold the result only after that stream is synchronized."""
    from .index_copy import device_ptr

    dev = N.require_device(pages, page_ids, names=("pages", "page_ids"))
    num_pages, H, D, P = pages.shape
    if not chunks:
        return
    L, _, _, T = chunks[0].shape if chunks[0].dim() == 4 else (0, 0, 0, 0)
    if T % P or T == 0:
        raise ValueError(f"chunks must be [L, {H}, {D}, ppc*{P}], got {tuple(chunks[0].shape)}")
    ptrs = []
    for i, c in enumerate(chunks):
        if c.dim() != 4 or tuple(c.shape) != (L, H, D, T):
            raise ValueError(f"chunk {i} must be [{L}, {H}, {D}, {T}], got {tuple(c.shape)}")
        if c.dtype != pages.dtype or not c.is_contiguous():
            raise ValueError(f"chunk {i} must be contiguous {pages.dtype}")
        if c.device.type == "cpu":
            if not c.is_pinned():
                raise ValueError(f"chunk {i} is a pageable host tensor; host chunks must be pinned")
        elif c.device != dev:
            raise ValueError(f"chunk {i} is on {c.device}, the pool on {dev}")
        ptr = device_ptr(c)
        if ptr % 16:
            raise ValueError(f"chunk {i} is not 16-byte aligned")
        ptrs.append(ptr)
    ppc = T // P
    if page_ids.dtype != torch.int64 or page_ids.numel() != len(chunks) * L * ppc:
        raise ValueError(f"page_ids must be int64 [{len(chunks) * L * ppc}]")
    if not pages.is_contiguous():
        raise ValueError("pages must be contiguous")
    table = torch.tensor(ptrs, dtype=torch.int64).to(dev)
    N.call("pia_kv_pages_chunks_copy", table.data_ptr(), len(chunks), pages.data_ptr(),
           page_ids.contiguous().data_ptr(), L, ppc, H, D, P, num_pages, pages.element_size(),
           1 if to_chunk else 0, N.stream_of(dev))
    # The table is read by the launch: keep it alive until the stream has passed it.
    table.record_stream(torch.cuda.current_stream(dev))
