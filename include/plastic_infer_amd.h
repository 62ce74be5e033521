/*
 * plastic_infer_amd.h — C-ABI of the MI355X (gfx950) paged-KV and expert-cache data path.
 *
 * One shared library, libplastic_infer_amd.so, built with hipcc for gfx950. Every entry point
 * takes plain device/host pointers, sizes and a HIP stream handle (hipStream_t passed as void*;
 * NULL = the legacy default stream), enqueues its kernels asynchronously on that stream and
 * returns an int status:
 *     0                 success
 *     PIA_EINVAL (-1)   invalid argument (shape, dtype, alignment, size limit); nothing enqueued
 *     PIA_EUNSUPPORTED  (-2) a valid combination this build does not implement; nothing enqueued
 *     > 0               a hipError_t returned by the HIP runtime
 * pia_last_error() returns a NUL-terminated, thread-local description of the last failure.
 *
 * Ownership: the caller owns every buffer. The library never allocates or frees device memory;
 * scratch space is passed in as a caller-owned workspace whose size a *_workspace_bytes query
 * reports. Index/slot arguments that point outside the pool are skipped by the kernels (never
 * dereferenced), mirroring a bounds-checked store rather than faulting.
 *
 * Layouts (row-major, innermost last):
 *   KV pool   k_pages / v_pages : [num_pages, num_kv_heads, head_dim, page_size]   (token innermost)
 *   new rows  k / v             : [num_tokens, num_kv_heads, head_dim] with a token stride
 *   queries   q / out           : [rows, num_heads, head_dim]
 *   block tables                : int32 [num_seqs, bt_stride]  (logical page -> physical page)
 *
 * This is the boundary that replaces the reference's torch data path and its nvcc-JIT ctypes
 * shims (reference: src/plastic_infer/kernel/jit.py:87-124, kernel/fast_index_copy.py:78-243).
 */
#ifndef PLASTIC_INFER_AMD_H
#define PLASTIC_INFER_AMD_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PIA_EINVAL (-1)
#define PIA_EUNSUPPORTED (-2)

/* Element type codes (dtype arguments). */
#define PIA_DTYPE_F32 0
#define PIA_DTYPE_F16 1
#define PIA_DTYPE_BF16 2

/* ---------------------------------------------------------------------------------------------
 * Library
 * ------------------------------------------------------------------------------------------- */

/* Thread-local message of the last non-zero status returned on this thread. */
const char* pia_last_error(void);

/* ABI version of this build (bumped on any signature change). */
int pia_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * Slot-mapped KV scatter.
 * Replaces the per-token advanced-index store of _write_kv_layer
 * (reference: src/plastic_infer/exec/runner_paged.py:112-129) and of KVRequestCache.append_token
 * (src/plastic_infer/kv/kv_store.py:124-143):  for i < num_tokens with slot = slot_mapping[i],
 *     k_pages[slot / page_size, h, d, slot % page_size] = k[i, h, d]   (same for v)
 * Slots < 0 (padding) or >= num_pages*page_size are skipped. Bit-exact byte copy;
 * elem_bytes is 2 or 4; page_size <= 1024. k_token_stride / v_token_stride are in elements.
 * Tokens sharing a slot land in unspecified order (the reference writes them in token order).
 * ------------------------------------------------------------------------------------------- */
int pia_kv_scatter(const void* k, const void* v, void* k_pages, void* v_pages,
                   const int64_t* slot_mapping, int64_t num_tokens,
                   int64_t k_token_stride, int64_t v_token_stride,
                   int num_kv_heads, int head_dim, int page_size, int64_t num_pages,
                   int elem_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Block-table gather into contiguous rows, batched over sequences.
 * Replaces gather_paged_kv (reference: src/plastic_infer/exec/attention.py:103-148):
 *     k_out[cu_seqlens[b] + t, h, d] = k_pages[block_tables[b, t / P], h, d, t % P]
 * for t < cu_seqlens[b+1] - cu_seqlens[b]. max_seq_len bounds the grid (tokens beyond a row's
 * table capacity bt_stride*P are not read). Bit-exact.
 * ------------------------------------------------------------------------------------------- */
int pia_kv_gather(void* k_out, void* v_out, const void* k_pages, const void* v_pages,
                  const int32_t* block_tables, int64_t bt_stride, const int64_t* cu_seqlens,
                  int num_seqs, int64_t max_seq_len,
                  int num_kv_heads, int head_dim, int page_size, int64_t num_pages,
                  int elem_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Page <-> chunk copies for KV chunk sinking / prefix loading
 * (reference: src/plastic_infer/kv/kv_store.py:230-276 sink, :282-334 load_prefix).
 * A chunk buffer is [num_layers, num_kv_heads, head_dim, pages_per_chunk * page_size];
 * page_ids is int64 [num_layers * pages_per_chunk] (layer-major), -1 = absent page (skipped).
 *   to_chunk != 0 : chunk[l, h, d, p*P + t] = pages[page_ids[l*ppc + p], h, d, t]
 *   to_chunk == 0 : pages[page_ids[l*ppc + p], h, d, t] = chunk[l, h, d, p*P + t]
 * ------------------------------------------------------------------------------------------- */
int pia_kv_pages_chunk_copy(void* chunk, void* pages, const int64_t* page_ids,
                            int num_layers, int pages_per_chunk,
                            int num_kv_heads, int head_dim, int page_size, int64_t num_pages,
                            int elem_bytes, int to_chunk, void* stream);

/* The same copy for num_chunks chunks in one launch, in 16-byte words where page_size *
 * elem_bytes allows: chunks is a device-readable array of num_chunks chunk base addresses
 * (device memory, or pinned host memory through its device mapping, pia_device_pointer;
 * 16-byte aligned), page_ids int64
 * [num_chunks * num_layers * pages_per_chunk] (chunk-major, then layer-major). Batches the
 * per-page .to() loops of KVStore.sink_completed_chunks / load_prefix (reference
 * src/plastic_infer/kv/kv_store.py:230-334) into one transfer over the host link. */
int pia_kv_pages_chunks_copy(void* const* chunks, int num_chunks, void* pages,
                             const int64_t* page_ids, int num_layers, int pages_per_chunk,
                             int num_kv_heads, int head_dim, int page_size, int64_t num_pages,
                             int elem_bytes, int to_chunk, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Paged GQA decode attention, batched: one query row per sequence.
 * Per-row semantics of paged_attention_v1(q[b][None,None], ..., kv_num_tokens=L_b, causal=False)
 * (reference: src/plastic_infer/exec/attention.py:151-190, decode call
 * src/plastic_infer/exec/runner_paged.py:253-255): head hq reads kv head hq / (H / Hkv),
 *     out[b, hq, :] = softmax(scale * q[b, hq, :] . K_b^T) V_b   over the L_b = context_lens[b]
 * tokens of block_tables[b, :ceil(L_b / P)]. fp32 accumulation and online softmax.
 * q row stride between sequences is q_seq_stride elements; heads are contiguous [H, D].
 * out is contiguous [num_seqs, num_heads, head_dim]; L_b == 0 writes zeros.
 * A block-table id outside [0, num_pages) inside the first ceil(L_b / P) entries is not
 * dereferenced: the tokens of that page are not keys (the reference's index_select would raise
 * instead; its drop-in wrappers, which see host lists, raise IndexError before launching).
 * A row left with no key writes zeros.
 * workspace: caller-owned device scratch of at least
 *     pia_paged_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_dim, page_size,
 *                                      bt_stride)
 * bytes, 4-byte aligned (may be NULL when that query returns 0). Calls that share a workspace
 * must be ordered (same stream): a launch keeps its partials and arrival counters in it.
 * bf16 or fp16 with head_dim 128 and page_size 16 and Hq/Hkv in 1..8 or 16 takes the fast
 * kernel (the batch's KV steps split over persistent waves, XCD-aware; the probabilities enter
 * the P.V products rounded to the pools' dtype); every other supported combination
 * (f32/f16/bf16, head_dim <= 512, any page_size) takes the general kernel.
 * ------------------------------------------------------------------------------------------- */
int64_t pia_paged_decode_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads,
                                         int head_dim, int page_size, int64_t bt_stride);

/* Layout of the fast decode kernel's scratch for `waves` persistent waves (2 <= waves <= 4096;
 * the workspace above is this layout at 4096 waves, the no-alloc entry point's static array at
 * the waves of its launch). No counterpart in the reference: a host-only query, callable without
 * a GPU, for callers and tests that size or check a scratch buffer. Bytes [0, *partials_offset)
 * hold one 64-bit arrival counter per wave (from the first 8-byte boundary of a 4-byte aligned
 * buffer); bytes [*partials_offset, *total_bytes) hold two partial slots per wave of
 * (num_heads / num_kv_heads) rows of head_dim + 2 fp32. Returns 0, or PIA_EINVAL /
 * PIA_EUNSUPPORTED (Hq / Hkv outside 1..8 and 16). */
int pia_paged_decode_scratch_layout(int num_heads, int num_kv_heads, int waves,
                                    int64_t* partials_offset, int64_t* total_bytes);

int pia_paged_decode_attention(void* out, const void* q, int64_t q_seq_stride,
                               const void* k_pages, const void* v_pages,
                               const int32_t* block_tables, int64_t bt_stride,
                               const int32_t* context_lens, int num_seqs,
                               int num_heads, int num_kv_heads, int head_dim, int page_size,
                               int64_t num_pages, float scale, int dtype,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * The decode step's KV write and attention in one call: the reference's _write_kv_layer of the
 * new token at position pos (page block_table[pos / P], offset pos % P) followed by
 * _attn_paged(..., kv_num_tokens=pos + 1, causal=False)
 * (src/plastic_infer/exec/runner_paged.py:112-129 and :251-255,
 * src/plastic_infer/exec/runner_moe_paged.py:144-147).
 * Row b's new token is position L_b - 1 (L_b = context_lens[b], counting it): k_new / v_new hold
 * its K and V, [num_kv_heads, head_dim] per row, new_seq_stride elements between rows (heads
 * contiguous). Results: the pools hold k_new / v_new at that slot, and out is what
 * pia_paged_decode_attention gives over the updated pools (same arguments, workspace and
 * rules). A row whose L_b is 0 or exceeds bt_stride * page_size writes no slot; a slot whose
 * page id is outside [0, num_pages) is not written and the new token is then no key.
 * The fast kernel (the same shapes as pia_paged_decode_attention's) takes the new token's K / V
 * from k_new / v_new and stores them into the slot itself, so the step has no separate write
 * launch ahead of the attention; other shapes write the slots with a small kernel first.
 * A slot must belong to one row only (a row's new-token page is not read by another row of the
 * call), as with any slot that a decode step writes.
 * ------------------------------------------------------------------------------------------- */
int pia_paged_decode_append_attention(void* out, const void* q, int64_t q_seq_stride,
                                      void* k_pages, void* v_pages,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      const int32_t* context_lens, const void* k_new,
                                      const void* v_new, int64_t new_seq_stride, int num_seqs,
                                      int num_heads, int num_kv_heads, int head_dim,
                                      int page_size, int64_t num_pages, float scale, int dtype,
                                      void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Paged GQA decode attention that allocates nothing and takes no workspace.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as pia_paged_decode_attention without the workspace: the fast
 * kernel keeps its partials in a static device array of the library (32 MiB per GPU, held
 * until the process ends; its address on each device is resolved on the first call there).
 * No hipMalloc / hipFree / allocating library routine is called. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, or unordered host
 * threads) race and must not be issued; calls ordered on one stream are safe. The array needs
 * no clearing (each launch writes what it reads). Returns PIA_EUNSUPPORTED when the partials
 * of the launch would not fit (pia_paged_decode_noalloc_scratch_bytes > 32 MiB).
 * ------------------------------------------------------------------------------------------- */
int64_t pia_paged_decode_noalloc_scratch_bytes(int num_heads, int num_kv_heads);

int pia_paged_decode_attention_noalloc(void* out, const void* q, int64_t q_seq_stride,
                                       const void* k_pages, const void* v_pages,
                                       const int32_t* block_tables, int64_t bt_stride,
                                       const int32_t* context_lens, int num_seqs,
                                       int num_heads, int num_kv_heads, int head_dim,
                                       int page_size, int64_t num_pages, float scale, int dtype,
                                       void* stream);

/* ---------------------------------------------------------------------------------------------
 * General paged attention over several query rows per sequence (prefill / chunked
 * prefill / the drop-in paged_attention_v1 and _attn_paged paths).
 * Rows of sequence b are q[cu_q[b] .. cu_q[b+1]) (cu_q NULL: one row per sequence). Row s of b
 * attends keys j < kv_lens[b]; when q_pos_offsets != NULL additionally j <= q_pos_offsets[b] + s
 * (offset 0 = torch SDPA is_causal=True top-left alignment, reference
 * src/plastic_infer/exec/attention.py:189; offset q_start_pos = the explicit mask of
 * src/plastic_infer/exec/runner_paged.py:61-95). Pages whose block-table id is outside
 * [0, num_pages) hold no keys, as in pia_paged_decode_attention. A row with no admissible key
 * writes zeros. Non-finite inputs: a NaN in q or in an admissible key of a row makes that row's
 * output NaN (IEEE semantics throughout); keys a row may not see are excluded by selection, so
 * a NaN there does not reach it (the reference's additive offset mask lets it through).
 * ------------------------------------------------------------------------------------------- */
int pia_paged_attention(void* out, const void* q, const void* k_pages, const void* v_pages,
                        const int32_t* block_tables, int64_t bt_stride,
                        const int32_t* kv_lens, const int32_t* cu_q, const int32_t* q_pos_offsets,
                        int num_seqs, int64_t total_q_rows,
                        int num_heads, int num_kv_heads, int head_dim, int page_size,
                        int64_t num_pages, float scale, int dtype, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Host-stream attention: q rows over KV split into host chunks and a device-resident tail,
 * read in place (reference host_stream_attention_v1, src/plastic_infer/exec/attention.py:193-250,
 * which concatenates both on the device before SDPA).
 * q, out: [q_len, num_heads, head_dim] contiguous. Chunk c covers KV positions
 * [c*chunk_tokens, ...) and is [num_kv_heads, head_dim, len_c] (token innermost) with
 * len_c = chunk_tokens except the last, len = host_len - (num_chunks-1)*chunk_tokens in
 * [1, chunk_tokens]. chunk_k / chunk_v: device-readable arrays of num_chunks 16-byte-aligned chunk
 * addresses: HBM, or pinned host memory through its device mapping (pia_device_pointer), which
 * the kernel then streams over the host link without staging. The tail (positions host_len ..
 * host_len + resident_len) is token-major: row t at resident_k + t*resident_token_stride elements
 * holds [num_kv_heads, head_dim]. Query row i sits at position q_start_pos + i; causal != 0 lets it
 * see keys at positions <= q_start_pos + i (the reference's mask, and SDPA is_causal when
 * q_start_pos == 0 and q_len == kv_len), causal == 0 sees all keys. Softmax in fp32; a row that
 * sees no key writes zeros. head_dim <= 256. workspace: at least
 * pia_host_stream_attention_workspace_bytes(...) bytes of device memory (4-byte aligned).
 * ------------------------------------------------------------------------------------------- */
int64_t pia_host_stream_attention_workspace_bytes(int64_t q_len, int num_heads, int num_kv_heads,
                                                  int head_dim, int num_chunks,
                                                  int64_t chunk_tokens, int64_t host_len,
                                                  int64_t resident_len);
int pia_host_stream_attention(void* out, const void* q, int64_t q_len, int num_heads,
                              const void* const* chunk_k, const void* const* chunk_v,
                              int num_chunks, int64_t chunk_tokens, int64_t host_len,
                              const void* resident_k, const void* resident_v,
                              int64_t resident_len, int64_t resident_token_stride,
                              int num_kv_heads, int head_dim, int64_t q_start_pos, int causal,
                              float scale, int dtype, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* ---------------------------------------------------------------------------------------------
 * Router: top-k expert selection per token.
 * mode 0 = _torch_fused_topk (reference: src/plastic_infer/moe/fused.py:11-30):
 *     p = softmax(float(logits)); (w, ids) = topk(p, k); w /= sum(w) if renormalize.
 * mode 1 = topk_route (reference: src/plastic_infer/exec/moe.py:19-38):
 *     (x, ids) = topk(logits, k); w = softmax(float(x)).
 * Selection order: descending logit, lowest expert index first on exact ties. Weights are
 * written as fp32 [T, k], ids as int32 [T, k]. logits_dtype: PIA_DTYPE_*; num_experts <= 1024.
 * Rows t >= num_token_non_padded (when >= 0) get ids = -1, as the reference's padding rule.
 * ------------------------------------------------------------------------------------------- */
int pia_moe_topk(float* topk_weights, int32_t* topk_ids, const void* logits, int logits_dtype,
                 int64_t num_tokens, int num_experts, int topk, int renormalize, int mode,
                 int64_t num_token_non_padded, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Permute plan (moe_align_block_size, reference: src/plastic_infer/moe/fused.py:48-94,
 * semantics src/plastic_infer/kernel/triton/moe_align.py:9-20,216-239).
 * effective_E = num_experts + 1 (ids in [0, num_experts] are routed, others dropped).
 *   count[e], padded cumsum in multiples of block_size, num_tokens_post_pad = cumsum[E+1],
 *   expert_ids[blk] = owning expert for blk < npp/block (-1 beyond),
 *   sorted_token_ids[cumsum[e] + r] = r-th route (flattened index t*k+s) of expert e in
 *   ASCENDING route order (the deterministic order moe_forward_sparse's nonzero() yields,
 *   reference src/plastic_infer/exec/moe.py:149); every other entry = numel (sentinel).
 *   route_pos (optional, may be NULL): route_pos[i] = row of route i in sorted order, -1 if dropped.
 * Sizes: sorted_token_ids [max_num_tokens_padded], expert_ids [ceil(max_num_tokens_padded/block)]
 * with max_num_tokens_padded as the reference computes it. workspace >= pia_moe_align_workspace_bytes.
 * ------------------------------------------------------------------------------------------- */
int64_t pia_moe_align_workspace_bytes(int num_experts);

int pia_moe_align_block_size(int32_t* sorted_token_ids, int32_t* expert_ids,
                             int32_t* num_tokens_post_pad, int32_t* route_pos,
                             const int32_t* topk_ids, int64_t numel, int num_experts,
                             int block_size, int64_t max_num_tokens_padded,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Router top-k and the permute plan in one call: the results of pia_moe_topk followed by
 * pia_moe_align_block_size on its ids (reference: fused_topk then moe_align_block_size,
 * src/plastic_infer/moe/fused.py:11-94; the batched moe_route_permute of the port's entry
 * points). Plans of more than 4096 routes with num_experts <= 510 take two launches: the top-k
 * kernel also writes the plan's per-chunk expert histogram (chunk = its block of tokens), then
 * one placement kernel builds the plan from it. Other shapes run the two calls above.
 * Arguments are those of the two calls; route_pos may be NULL.
 * ------------------------------------------------------------------------------------------- */
int pia_moe_topk_align(float* topk_weights, int32_t* topk_ids, const void* logits,
                       int logits_dtype, int64_t num_tokens, int num_experts, int topk,
                       int renormalize, int mode, int64_t num_token_non_padded,
                       int32_t* sorted_token_ids, int32_t* expert_ids,
                       int32_t* num_tokens_post_pad, int32_t* route_pos, int block_size,
                       int64_t max_num_tokens_padded, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* ---------------------------------------------------------------------------------------------
 * Permute: x_perm[r, :] = hidden[sorted_token_ids[r] / topk, :] for r < *num_tokens_post_pad
 * and sorted_token_ids[r] < numel. Padding rows (sentinel: sorted_token_ids[r] >= numel) and rows
 * at or beyond *num_tokens_post_pad are left untouched: a consumer skips sentinel rows, as the
 * reference's grouped GEMM masks them (src/plastic_infer/kernel/triton/fused_moe.py:156-302).
 * Bit-exact row copy (row_bytes multiple of 4).
 * route_pos (optional, the inverse map pia_moe_align_block_size writes): when given, each token
 * row is read once and written to its routes' rows (same result, a quarter of the reads for
 * top-8); NULL walks the destination rows in order.
 * (reference: the per-expert hidden[rows] gather of src/plastic_infer/exec/moe.py:150-153,
 * and the sorted_token_ids / topk A-row read of src/plastic_infer/kernel/triton/fused_moe.py:156-302)
 * ------------------------------------------------------------------------------------------- */
int pia_moe_permute(void* x_perm, const void* hidden, const int32_t* sorted_token_ids,
                    const int32_t* route_pos, const int32_t* num_tokens_post_pad,
                    int64_t max_rows, int64_t numel, int topk, int64_t row_bytes,
                    int64_t hidden_row_stride_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Unpermute / combine: out[t, :] = cast( sum_{s<k} w[t,s] * y[route_pos[t*k+s], :] )
 * accumulated in fp32 in slot order s = 0..k-1 (each step a separately rounded multiply and add),
 * routes with route_pos < 0 or >= y_rows contribute nothing; topk_weights NULL means weight 1
 * (moe_sum_reduce, reference src/plastic_infer/kernel/triton/fused_moe.py:111-153 with the
 * weight of fused_moe.py:292-294; combine of src/plastic_infer/exec/moe.py:155-158).
 * y rows: [*, hidden_dim] of dtype; out [num_tokens, hidden_dim] of dtype.
 * ------------------------------------------------------------------------------------------- */
int pia_moe_unpermute(void* out, const void* y, int64_t y_rows, const int32_t* route_pos,
                      const float* topk_weights, int64_t num_tokens, int topk, int hidden_dim,
                      int dtype, void* stream);

/* Plain sum over the top-k axis: out[t, :] = cast(sum_s in[t, s, :]) with fp32 accumulation
 * (moe_sum_reduce_triton, reference src/plastic_infer/kernel/moe_impl.py:169-197). */
int pia_moe_sum_reduce(void* out, const void* in, int64_t num_tokens, int topk, int hidden_dim,
                       int dtype, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Grouped expert GEMM over a permute plan, one of the two GEMMs of the fused experts FFN
 * (fused_experts_impl / fused_experts_decode_impl, reference src/plastic_infer/moe/fused.py:
 * 169-359; kernels src/plastic_infer/kernel/triton/fused_moe.py:156-302 and
 * src/plastic_infer/kernel/triton/decode_moe.py:6-75; the activation of
 * src/plastic_infer/kernel/triton/activation.py:63-113 fused into the first GEMM).
 * For every plan row p < min(*num_tokens_post_pad, max_num_tokens_padded) holding a route
 * r = sorted_token_ids[p] < numel, with e = expert_ids[p / block_m] in [0, num_experts):
 *     acc[n] = sum_k a[(r / a_div) * lda + k] * w[(e * n_rows + n) * k_dim + k]   (fp32)
 *     activation PIA_ACT_NONE:  out[r * ldo + n] = round(acc[n] * w_r)          n < n_rows
 *     activation X:             g = round(acc[n] * w_r), u = round(acc[n_rows/2 + n] * w_r),
 *                               out[r * ldo + n] = round(X(g) * u)              n < n_rows / 2
 * w_r = topk_weights[r] when mul_routed_weight != 0, else 1; round() is the storage dtype.
 * Routes of a block whose expert is outside [0, num_experts) get zero rows. Storage: a, w, out
 * bf16, fp16 or fp32 (dtype; for fp32 round() is the identity and the products are fp32
 * MFMA products), topk_weights fp32 [numel]. k_dim and lda multiples of 8 (bf16 / fp16) or 4
 * (fp32); a and w 16-byte aligned; block_m a multiple of 16; a holds ceil(numel / a_div) rows.
 * Small calls (decode: fewer than 2048 routes) and every fp32 call run a split-K kernel over
 * 16-row plan blocks that streams each expert's W once per block; larger bf16 / fp16 calls run
 * an LDS-tiled kernel over the experts present in the plan (tiles of up to 320 routes x 256 W
 * rows, so that each expert's W is streamed once when it serves up to 320 routes). The first
 * GEMM of the FFN is a_div = top_k
 * (a = hidden [T, H]) with the activation; the second is a_div = 1 (a = the first GEMM's
 * output [T*k, I]) without it, ldo = H, writing [T, k, H] for pia_moe_sum_reduce.
 * ------------------------------------------------------------------------------------------- */
#define PIA_ACT_NONE (-1)
#define PIA_ACT_SILU 0
#define PIA_ACT_GELU 1
#define PIA_ACT_GELU_TANH 2
int pia_moe_expert_gemm(void* out, const void* a, const void* w, const float* topk_weights,
                        const int32_t* sorted_token_ids, const int32_t* expert_ids,
                        const int32_t* num_tokens_post_pad, int64_t max_num_tokens_padded,
                        int block_m, int64_t numel, int a_div, int64_t lda, int num_experts,
                        int n_rows, int k_dim, int64_t ldo, int activation,
                        int mul_routed_weight, int dtype, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Workspace of pia_moe_expert_gemm in bytes (4-byte aligned; holds the work list built from
 * the plan on every call): (2 * ceil(max_num_tokens_padded / block_m) + 10) * 4. */
int64_t pia_moe_expert_gemm_workspace_bytes(int64_t max_num_tokens_padded, int block_m);

/* y[r, j] = round(act(x[r, j]) * x[r, d + j]) for x [rows, 2d], y [rows, d], bf16, fp16 or fp32
 * (silu_and_mul / gelu_and_mul / gelu_tanh_and_mul, reference
 * src/plastic_infer/kernel/triton/activation.py:63-150). activation: PIA_ACT_SILU, _GELU,
 * _GELU_TANH. */
int pia_act_and_mul(void* out, const void* x, int64_t rows, int64_t d, int activation, int dtype,
                    void* stream);

/* ---------------------------------------------------------------------------------------------
 * Row index copy kernel (fast_index_copy, reference
 * src/plastic_infer/kernel/fast_index_copy.py:124-186, kernel .cuh:190-286):
 *     for i < n:  dst + dst_idx[i]*row_bytes  <-  src + src_idx[i]*row_bytes
 * n = min(*num_indices, length) when num_indices != NULL (device int64), else length.
 * index_is_int32 selects the index width. src/dst may be device memory or pinned host memory
 * mapped into the device address space. Rows whose index is negative or not below the table's
 * row count (dst_num_rows / src_num_rows) are skipped. row_bytes % 16 == 0 and 16-byte aligned
 * bases take the 16-byte vector path; any other row size is copied bytewise.
 * ------------------------------------------------------------------------------------------- */
int pia_index_copy_rows(void* dst, const void* dst_indices, int64_t dst_num_rows,
                        const void* src, const void* src_indices, int64_t src_num_rows,
                        int64_t length, const int64_t* num_indices, int64_t row_bytes,
                        int index_is_int32, void* stream);

/* Device address for kernel access to `ptr`: device memory is returned as is, pinned host
 * memory through its device mapping (the reference's cudaHostGetDevicePointer step,
 * src/plastic_infer/kernel/pinned.py:67-137). Memory HIP does not know (pageable host memory)
 * is rejected with PIA_EINVAL, so a kernel is never handed an address it cannot reach.
 * pia_index_copy_rows applies this to its src/dst itself. */
int pia_device_pointer(const void* ptr, void** device_ptr);

/* Multi-bank variant (fast_index_copy_multi, reference src/plastic_infer/kernel/fast_index_copy.py:
 * 190-243, .cuh:436-505): the same (dst_idx, src_idx) rows for every bank b < num_banks, with
 * per-bank base pointers and row bytes given as DEVICE int64 arrays. Row bytes % 16 == 0. */
int pia_index_copy_rows_multi(const int64_t* dst_ptrs, const int64_t* src_ptrs,
                              const int64_t* row_bytes, int num_banks,
                              const void* dst_indices, const void* src_indices, int64_t length,
                              const int64_t* num_indices, int index_is_int32, void* stream);

/* ---------------------------------------------------------------------------------------------
 * (4) Host-planned row copies with the DMA engines: for i < n,
 *     hipMemcpyAsync(dst + dst_rows[i]*row_bytes, src + src_rows[i]*row_bytes, row_bytes)
 * on `stream`, merging runs where both row indices advance by one into single copies.
 * dst_rows/src_rows are HOST int64 arrays (the plan is host-known, as ExpertSlotPool's LRU is,
 * reference src/plastic_infer/store/experts.py:178-223). dst/src: any of device memory or
 * pinned host memory (the runtime picks the direction). Returns the number of copies issued
 * through *copies_issued when non-NULL.
 * ------------------------------------------------------------------------------------------- */
int pia_copy_rows_async(void* dst, const int64_t* dst_rows, const void* src,
                        const int64_t* src_rows, int64_t n, int64_t row_bytes,
                        int64_t* copies_issued, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Device-side LRU admission of a slot cache (lru_ensure, reference
 * src/plastic_infer/kernel/lru_ensure.py:371-438, victim rule of its sequential kernel
 * :200-265; MoE use src/plastic_infer/moe/offload_kernels.py:19-40). Device arrays:
 *   slot_of_id [num_total] i32 (id -> slot or -1), id_of_slot [num_cached] i32 (-1 = empty),
 *   lru_usage [num_cached] i64, lru_step [] i64 (+1 per call).
 * query [num_queries] i32 ids (+ id_base = global id); duplicates collapse to one slot. Hits
 * get usage = step. The distinct missing ids, ascending, take the evictable slots (usage !=
 * step) in ascending (usage, slot) order; the previous owner of each victim is unmapped.
 * out_indices[i] = slot of query i (may alias query); src_indices[j] = id - id_base and
 * dst_indices[j] = slot for j < *num_copy (the copy plan); stats (NULL or i64[3]) +=
 * (distinct ids, admitted misses, 1). Ids outside [0, num_total) are inert (out = -1). Misses
 * beyond the evictable slots are not admitted (out = -1); the reference leaves that case
 * undefined. Limits: num_queries <= 2048, 1 <= num_cached <= 2^24 (caches of more than 16384
 * slots stream their usage from global memory instead of holding it in LDS, with the same
 * decisions; reference streaming variant src/plastic_infer/kernel/lru_ensure.py:214-270).
 * ------------------------------------------------------------------------------------------- */
int pia_lru_ensure(const int32_t* query, int64_t num_queries, int32_t* slot_of_id,
                   int64_t num_total, int32_t* id_of_slot, int64_t* lru_usage,
                   int64_t num_cached, int64_t* lru_step, int32_t* out_indices,
                   int32_t* src_indices, int32_t* dst_indices, int64_t* num_copy,
                   int64_t* stats, int64_t id_base, void* stream);

/* Slot-cache bookkeeping of OffloadMoeCache (reference
 * src/plastic_infer/moe/offload_kernels.py:208-285, offload_cache.py:597-605):
 *   reset       every id non-resident, every slot empty with usage 0, step = 0, active_mask
 *               (NULL or i32[num_experts]) = 0, *num_indices = 0 (when non-NULL);
 *   materialize partition layer_id's E ids into slots [0, E) in id order (owners of those
 *               slots from other partitions unmapped, this partition's copies elsewhere
 *               emptied), usage = ++step, plan = (src e -> slot e) for e < E, *num_indices = E;
 *   invalidate  slots [slot_begin, slot_end) emptied: owners unmapped, usage 0. */
int pia_slot_cache_reset(int32_t* slot_of_id, int64_t num_total, int32_t* id_of_slot,
                         int64_t* usage, int64_t num_cached, int64_t* step, int32_t* active_mask,
                         int num_experts, int64_t* num_indices, void* stream);
int pia_slot_cache_materialize(int32_t* slot_of_id, int64_t num_total, int32_t* id_of_slot,
                               int64_t* usage, int64_t num_cached, int64_t* step,
                               int32_t* evict_slots, int32_t* src_indices, int64_t* num_indices,
                               int layer_id, int num_experts, void* stream);
int pia_slot_cache_invalidate(int32_t* slot_of_id, int64_t num_total, int32_t* id_of_slot,
                              int64_t* usage, int64_t num_cached, int64_t slot_begin,
                              int64_t slot_end, void* stream);

/* Prefill hit compaction (prefill_hit_compact, reference
 * src/plastic_infer/moe/offload_kernels.py:63-82,413-431): experts e < num_experts whose slot
 * slot_row[e] >= threshold, in expert order: dst[j] = buffer_base + e, src[j] = slot_row[e];
 * *num = count. */
int pia_prefill_hit_compact(const int32_t* slot_row, int32_t* dst, int32_t* src, int64_t* num,
                            int64_t buffer_base, int64_t threshold, int num_experts,
                            void* stream);

/* ---------------------------------------------------------------------------------------------
 * HBM streaming-read probe. No counterpart in the reference: a measurement aid for the
 * rooflines of the kernels above (bench.py --workload hbm-read times it over fresh regions and
 * fits fixed cost + rate). src: 16-byte aligned device memory of `bytes` bytes (a positive
 * multiple of 16). tile_ids NULL: reads the whole buffer front to back. tile_ids non-NULL
 * (device i32[n_tiles]): reads the 4 KiB tiles src + 4096 * tile_ids[i], skipping ids outside
 * [0, bytes / 4096) - the paged-KV access pattern. Persistent grid, 16-byte loads, data
 * discarded; *sink (device, 4-byte aligned) is written only for one 32-bit fold of the data.
 * ------------------------------------------------------------------------------------------- */
int pia_hbm_read_probe(const void* src, int64_t bytes, const int32_t* tile_ids, int64_t n_tiles,
                       uint32_t* sink, void* stream);

/* The same probe for the load shape of a GEMM weight tile (no counterpart in the reference):
 * reads src as 16-row blocks of row_bytes each (contiguous), one wave per block, every load
 * instruction covering rows_per_load rows x 1024 / rows_per_load bytes: 16 is the MFMA
 * operand layout of the expert GEMMs (a 16-byte vector of each of 16 rows), 1 reads 1 KiB of
 * the block contiguously. rows_per_load in {1, 2, 4, 8, 16}; row_bytes a positive multiple of
 * 64 and of 1024 / rows_per_load; bytes >= 16 * row_bytes (whole blocks are read). */
int pia_hbm_read_rows_probe(const void* src, int64_t bytes, int row_bytes, int rows_per_load,
                            uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PLASTIC_INFER_AMD_H */
