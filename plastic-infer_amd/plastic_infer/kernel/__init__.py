"""HIP kernel layer: batched entry points over libplastic_infer_amd.so (gfx950)."""

from .activation import gelu_and_mul, gelu_tanh_and_mul, silu_and_mul
from .index_copy import copy_rows_async, fast_index_copy, fast_index_copy_multi
from .lru_ensure import lru_ensure
from .moe_ops import (
    max_num_tokens_padded,
    moe_align_block_size,
    moe_expert_gemm,
    moe_permute,
    moe_sum_reduce,
    moe_topk,
    moe_topk_align,
    moe_unpermute,
)
from .paged_kv import (
    decode_workspace_bytes,
    kv_gather,
    kv_scatter,
    paged_attention,
    paged_decode_attention,
    paged_decode_append_attention,
    paged_decode_attention_noalloc,
    pages_chunk_copy,
    pages_chunks_copy,
)

__all__ = [
    "gelu_and_mul", "gelu_tanh_and_mul", "silu_and_mul",
    "copy_rows_async", "fast_index_copy", "fast_index_copy_multi", "lru_ensure",
    "max_num_tokens_padded", "moe_align_block_size", "moe_expert_gemm", "moe_permute", "moe_sum_reduce",
    "moe_topk", "moe_topk_align", "moe_unpermute",
    "decode_workspace_bytes", "kv_gather", "kv_scatter", "paged_attention",
    "paged_decode_attention", "paged_decode_append_attention", "paged_decode_attention_noalloc", "pages_chunk_copy",
    "pages_chunks_copy",
]
