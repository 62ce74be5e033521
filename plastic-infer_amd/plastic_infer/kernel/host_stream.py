"""Host-stream attention over the HIP library: query rows against KV split into host chunks and
a device-resident tail, with the chunks read in place (reference
src/plastic_infer/exec/attention.py:193-250 concatenates them on the device before SDPA).

Chunks are [n_kv_heads, head_dim, len_c] tensors, all of length chunk_tokens except a shorter
last one. Pinned host chunks are streamed by the kernel over the host link through their device
mapping when every KV byte is read once (q_len * n_heads / n_kv_heads <= 32 query rows per kv
head, the decode case); with more rows, and for pageable host chunks, they are first copied to
HBM. Device chunks are read where they are.
"""

from __future__ import annotations

import math

import torch

from .. import _native as N
from .index_copy import device_ptr
from .pinned import hold_until_done

ROWS_PER_TILE = 32   # query rows one workgroup carries (rows per kv head beyond it re-read KV)


def host_stream_attention(q: torch.Tensor, chunks: list[tuple[torch.Tensor, torch.Tensor]],
                          resident_k: torch.Tensor, resident_v: torch.Tensor,
                          q_start_pos: int = 0, causal: bool = True,
                          scale: float | None = None) -> torch.Tensor:
    """q [q_len, H, D] (device), chunks [(k_c, v_c)] each [H_kv, D, len_c] oldest first,
    resident_k / resident_v [R, H_kv, D] (device, R may be 0). Returns [q_len, H, D]."""
    dev = N.require_device(q, resident_k, resident_v, names=("q", "resident_k", "resident_v"))
    if q.dim() != 3 or resident_k.dim() != 3 or resident_k.shape != resident_v.shape:
        raise ValueError("q must be [q_len, H, D] and resident_k / resident_v matching "
                         "[R, H_kv, D]")
    Sq, Hq, D = q.shape
    R, Hkv, Dk = resident_k.shape
    if Dk != D or Hkv <= 0 or Hq % Hkv:
        raise ValueError(f"heads / head_dim mismatch: q {tuple(q.shape)}, resident "
                         f"{tuple(resident_k.shape)}")
    dt = q.dtype
    for t in (resident_k, resident_v):
        if t.dtype != dt:
            raise ValueError("q, chunks and the resident tail must share a dtype")
    lens = []
    for i, (k_c, v_c) in enumerate(chunks):
        if k_c.dim() != 3 or k_c.shape != v_c.shape or tuple(k_c.shape[:2]) != (Hkv, D):
            raise ValueError(f"chunk {i} must be a matching pair of [{Hkv}, {D}, C] tensors")
        if k_c.dtype != dt or v_c.dtype != dt:
            raise ValueError(f"chunk {i} has dtype {k_c.dtype}, q {dt}")
        lens.append(int(k_c.shape[2]))
    out = torch.empty(Sq, Hq, D, dtype=dt, device=dev)
    if Sq == 0:
        return out
    # Empty chunks carry no keys; a list whose lengths are not (C, ..., C, last <= C) is laid out
    # as one device tail ahead of the resident rows.
    pairs = [(k, v) for (k, v), n in zip(chunks, lens) if n > 0]
    lens = [n for n in lens if n > 0]
    C = lens[0] if lens else 0
    if lens and (any(n != C for n in lens[:-1]) or lens[-1] > C):
        rk_all = torch.cat([k.to(dev).permute(2, 0, 1) for k, _ in pairs] + [resident_k])
        rv_all = torch.cat([v.to(dev).permute(2, 0, 1) for _, v in pairs] + [resident_v])
        return host_stream_attention(q, [], rk_all.contiguous(), rv_all.contiguous(),
                                     q_start_pos, causal, scale)
    G = Hq // Hkv
    in_place = math.ceil(Sq * G / ROWS_PER_TILE) <= 1
    keep, kp, vp = [], [], []
    for k_c, v_c in pairs:
        for t, ptrs in ((k_c, kp), (v_c, vp)):
            if not t.is_contiguous():
                t = t.contiguous()
            if t.device.type == "cpu":
                if not (in_place and t.is_pinned()):
                    t = t.to(dev, non_blocking=t.is_pinned())
            elif t.device != dev:
                t = t.to(dev)
            ptr = device_ptr(t) if t.device.type == "cpu" else t.data_ptr()
            if ptr % 16:
                t = t.to(dev, copy=True)
                ptr = t.data_ptr()
            keep.append(t)
            ptrs.append(ptr)
    host_len = sum(lens)
    rk, rv = resident_k, resident_v
    if R > 0 and not (rk.stride(2) == 1 and rk.stride(1) == D and rv.stride() == rk.stride()):
        rk, rv = rk.contiguous(), rv.contiguous()
    tok_stride = rk.stride(0) if R > 0 else Hkv * D
    n = len(pairs)
    ws_bytes = N.query("pia_host_stream_attention_workspace_bytes", Sq, Hq, Hkv, D, n, C,
                       host_len, R)
    if ws_bytes < 0:
        why = N.load().pia_last_error().decode(errors="replace")
        raise ValueError(f"host_stream_attention: unsupported shape ({why})")
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    tables = torch.tensor([kp + vp], dtype=torch.int64).pin_memory().to(
        dev, non_blocking=True) if n else None
    kt = tables[0, :n].data_ptr() if n else 0
    vt = tables[0, n:].data_ptr() if n else 0
    qc = q.contiguous()
    N.call("pia_host_stream_attention", out.data_ptr(), qc.data_ptr(), Sq, Hq, kt, vt, n, C,
           host_len, rk.data_ptr() if R else 0, rv.data_ptr() if R else 0, R, tok_stride, Hkv, D,
           int(q_start_pos), 1 if causal else 0,
           float(scale if scale is not None else 1.0 / math.sqrt(D)), N.dtype_code(dt),
           ws.data_ptr(), ws.numel(), N.stream_of(dev))
    stream = torch.cuda.current_stream(dev)
    if any(t.device.type == "cpu" for t in keep):
        hold_until_done(keep, stream)
    return out
