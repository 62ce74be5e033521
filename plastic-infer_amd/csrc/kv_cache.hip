// KV pool data movement for the page layout [num_pages, Hkv, D, P] (token innermost):
//   - slot-mapped scatter of new K/V rows (decode and ragged prefill),
//   - block-table gather back into contiguous [tokens, Hkv, D] rows,
//   - page <-> chunk copies used by chunk sinking and prefix loading.
// All three are byte-exact copies; elements are moved as 16- or 32-bit words.
#include "pia_internal.h"

namespace pia {
namespace {

// ---------------------------------------------------------------------------------------------
// Generic scatter (any element size and page size; 16-bit elements with 16-token pages and
// head_dim 64/128/256 take kv_scatter16_kernel below)
// ---------------------------------------------------------------------------------------------
// Full-page fast path: a block owns one destination page-run of up to P tokens. When the P
// tokens i0..i0+P-1 land on one page at offsets 0..P-1 (the prefill case: a sequence's tokens
// fill whole pages in order), the block stages their [Hkv*D] rows in LDS and writes every
// (h, d) row of the page tile as one contiguous P-element run, i.e. whole 32-byte sectors for
// bf16 / P = 16, instead of P scattered 2-byte stores.
//
// General path (any slot pattern): one element store per (token, h, d).
//
// Grid: (groups of P consecutive input tokens) x P. Every block of a group first checks whether
// the group is a full aligned page run; if so block y == 0 writes the page tile and the others
// exit, otherwise block y writes token y of the group (decode: one block per token).
// Two tokens with the same slot land in unspecified order.

template <typename W>
__global__ __launch_bounds__(256) void kv_scatter_kernel(
    const W* __restrict__ k, const W* __restrict__ v, W* __restrict__ kp, W* __restrict__ vp,
    const int64_t* __restrict__ slots, int64_t n, int64_t k_stride, int64_t v_stride, int HD,
    int P, int64_t total_slots, int use_tile) {
  extern __shared__ unsigned char smem_raw[];
  W* tile = reinterpret_cast<W*>(smem_raw);  // [HD][P+1] staged K then V rows (tile path only)
  __shared__ int s_full;

  const int64_t i0 = int64_t(blockIdx.x) * P;
  const int ntok = int(min<int64_t>(P, n - i0));
  const int y = blockIdx.y;
  if (threadIdx.x == 0) {
    int full = use_tile && (ntok == P);
    if (full) {
      const int64_t s0 = slots[i0];
      full = (s0 >= 0) && (s0 + P <= total_slots) && (s0 % P == 0);
      for (int t = 1; full && t < P; ++t) full = (slots[i0 + t] == s0 + t);
    }
    s_full = full;
  }
  __syncthreads();

  if (s_full) {
    if (y != 0) return;
    const int64_t page = slots[i0] / P;
    for (int pass = 0; pass < 2; ++pass) {
      const W* src = pass == 0 ? k : v;
      const int64_t stride = pass == 0 ? k_stride : v_stride;
      W* dst = (pass == 0 ? kp : vp) + page * int64_t(HD) * P;
      for (int e = threadIdx.x; e < P * HD; e += blockDim.x) {
        const int t = e / HD, r = e - t * HD;
        tile[r * (P + 1) + t] = src[(i0 + t) * stride + r];
      }
      __syncthreads();
      // dst row r = (h, d) holds P consecutive tokens: write them contiguously.
      for (int e = threadIdx.x; e < P * HD; e += blockDim.x) {
        const int r = e / P, t = e - r * P;
        dst[int64_t(r) * P + t] = tile[r * (P + 1) + t];
      }
      __syncthreads();
    }
    return;
  }

  if (y >= ntok) return;
  const int64_t slot = slots[i0 + y];
  if (slot < 0 || slot >= total_slots) return;
  const int64_t page = slot / P;
  const int off = int(slot - page * P);
  const W* ks = k + (i0 + y) * k_stride;
  const W* vs = v + (i0 + y) * v_stride;
  W* kd = kp + page * int64_t(HD) * P + off;
  W* vd = vp + page * int64_t(HD) * P + off;
  for (int r = threadIdx.x; r < HD; r += blockDim.x) {
    kd[int64_t(r) * P] = ks[r];
    vd[int64_t(r) * P] = vs[r];
  }
}

// ---------------------------------------------------------------------------------------------
// Generic gather: one block per (logical page, sequence); stage each head's [D][P] tile in LDS
// and write rows [t][h][d] contiguously (16-bit / 16-token pages take kv_gather16_kernel).
// ---------------------------------------------------------------------------------------------
template <typename W>
__global__ __launch_bounds__(256) void kv_gather_kernel(
    W* __restrict__ ko, W* __restrict__ vo, const W* __restrict__ kp, const W* __restrict__ vp,
    const int32_t* __restrict__ bt, int64_t bt_stride, const int64_t* __restrict__ cu, int H,
    int D, int P, int64_t num_pages) {
  extern __shared__ unsigned char smem_raw[];
  W* tile = reinterpret_cast<W*>(smem_raw);  // [D][P+1]
  const int lp = blockIdx.x, b = blockIdx.y;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  if (int64_t(lp) * P >= len || lp >= bt_stride) return;
  const int ntok = int(min<int64_t>(P, len - int64_t(lp) * P));
  const int64_t phys = bt[b * bt_stride + lp];
  const bool ok = phys >= 0 && phys < num_pages;
  const int HD = H * D;
  for (int pass = 0; pass < 2; ++pass) {
    const W* src = pass == 0 ? kp : vp;
    W* dst = pass == 0 ? ko : vo;
    for (int h = 0; h < H; ++h) {
      if (ok) {
        const W* tsrc = src + (phys * H + h) * int64_t(D) * P;
        for (int e = threadIdx.x; e < D * P; e += blockDim.x) {
          const int d = e / P, t = e - d * P;
          tile[d * (P + 1) + t] = tsrc[e];
        }
      }
      __syncthreads();
      for (int e = threadIdx.x; e < ntok * D; e += blockDim.x) {
        const int t = e / D, d = e - t * D;
        const int64_t row = row0 + int64_t(lp) * P + t;
        dst[row * HD + int64_t(h) * D + d] = ok ? tile[d * (P + 1) + t] : W(0);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------------------------
// 16-bit elements, 16-token pages (bf16 / fp16 pools with the reference's default page size):
// one wave per (16 input tokens, kv head) for the scatter and per (sequence page, kv head) for
// the gather. Both move the [16 tokens][D] <-> [D][16 tokens] transpose through LDS with
// 16-byte global loads, and write whole 32-byte page rows (scatter) or 64-byte runs of token
// rows (gather) per store instruction.
// ---------------------------------------------------------------------------------------------
constexpr int T16_P = 16;

// Scatter. Input tokens form page segments: maximal runs whose slots advance by one inside one
// page (a prefill chunk's page, a decode token alone, a padding slot alone). The wave of input
// group g (tokens 16g .. 16g+15) owns every segment that STARTS in its group, including the
// tokens of such a segment that spill into the next group (a segment has at most 16 tokens),
// so each page row is written by one wave and its partial stores meet in L2 at once.
// Owned tokens (at most 31) are staged in an LDS tile [32][D] (row pitch D + 8: the token
// pairs read below fall in distinct banks) with 16-byte loads. Lane (pi = lane & 15,
// dq = lane >> 4) writes owned tokens 2pi, 2pi + 1 for rows d = dq + 4j: one dword store when
// the pair lands on an even offset and the next one of the same page, otherwise 16-bit stores;
// padding or out-of-range slots store nothing.
template <int D>
__global__ __launch_bounds__(64) void kv_scatter16_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* __restrict__ kp,
    uint16_t* __restrict__ vp, const int64_t* __restrict__ slots, int64_t n, int64_t k_stride,
    int64_t v_stride, int H, int64_t total_slots, int wide) {
  constexpr int P = T16_P, PITCH = D + 8, CH = D / 8, MAXT = 32;
  __shared__ __align__(16) uint16_t tile[MAXT * PITCH];
  const int lane = threadIdx.x;
  // workgroup w: kv head w % H of input group w / H, so the H waves of a group run together
  // and read each token's contiguous [H][D] row at once
  const int h = int(blockIdx.x % unsigned(H));
  const int64_t i0 = int64_t(blockIdx.x / unsigned(H)) * P;
  // lane j < 33 looks at token i0 - 1 + j
  const int64_t tj = i0 - 1 + lane;
  long long s = -1;
  if (lane < 33 && tj >= 0 && tj < n) {
    s = slots[tj];
    if (s < 0 || s >= total_slots) s = -1;
  }
  const long long sprev = __shfl_up(s, 1, 64);
  const bool start = lane >= 1 && lane < 33 &&
                     (s < 0 || sprev < 0 || s != sprev + 1 || (s % P) == 0 || tj >= n);
  const uint64_t starts = __ballot(start);
  // first segment start in the group (lanes 1..16) and the first one after it (lanes 17..32)
  const int a = __builtin_ctzll(starts & 0x1fffeull);
  const uint64_t after = starts & ~0x1ffffull;
  const int b = after ? __builtin_ctzll(after) : 33;
  const int m = max(0, min(b, int(min<int64_t>(n - i0 + 1, 33))) - a);  // owned tokens
  const int64_t t0 = i0 - 1 + a;                                        // first owned token
  if (m == 0) return;

  const int pi = lane & 15, dq = lane >> 4;
  const long long s0 = __shfl(s, (a + 2 * pi) & 63, 64), s1 = __shfl(s, (a + 2 * pi + 1) & 63, 64);
  const bool has0 = 2 * pi < m && s0 >= 0, has1 = 2 * pi + 1 < m && s1 >= 0;
  const bool pair = has0 && has1 && s1 == s0 + 1 && (s0 & 1) == 0;
  const int64_t head_off = int64_t(h) * D * P;
  const int64_t b0 = has0 ? (s0 / P) * H * D * P + head_off + (s0 % P) : 0;
  const int64_t b1 = has1 ? (s1 / P) * H * D * P + head_off + (s1 % P) : 0;
  // a whole page (16 consecutive slots from a page start) on 16-byte aligned pools: every page
  // row (32 bytes) goes out as two 16-byte stores, lane l writing row d = 32r + l/2, tokens
  // 8(l&1) .. 8(l&1) + 7, so one store instruction covers 1 KiB of the tile. The owned tokens
  // must form ONE segment: m counts every segment that starts in the group, so several short
  // segments (or a run followed by padding) can also add up to 16; those have a segment start
  // among lanes a + 1 .. a + 15 and take the per-token path below.
  const long long sfirst = __shfl(s, a & 63, 64);
  const bool one_segment = ((starts >> (a + 1)) & 0x7fffull) == 0;
  const bool full = wide && m == P && one_segment && sfirst >= 0 && (sfirst % P) == 0;
  const int64_t fbase = full ? (sfirst / P) * H * D * P + head_off : 0;

  // The first 256 16-byte items of K and of V (all of a 16-token segment for D <= 128) are
  // loaded together up front, so both tensors' reads are in flight at once; the LDS tile then
  // transposes K, then V.
  constexpr int NPRE = 4;
  const int items = m * CH;
  uint4 kpre[NPRE], vpre[NPRE];
#pragma unroll
  for (int j = 0; j < NPRE; ++j) {
    const int it = lane + 64 * j;
    const int t = it / CH, c = it - t * CH;
    kpre[j] = vpre[j] = make_uint4(0u, 0u, 0u, 0u);
    if (it < items) {
      kpre[j] = *reinterpret_cast<const uint4*>(k + (t0 + t) * k_stride + int64_t(h) * D + c * 8);
      vpre[j] = *reinterpret_cast<const uint4*>(v + (t0 + t) * v_stride + int64_t(h) * D + c * 8);
    }
  }

  // one tensor: preloaded items and the rest into the tile, then the tile out to the pages
  auto pass_of = [&](const uint16_t* src, int64_t stride, uint16_t* dst, const uint4 (&pre)[NPRE]) {
#pragma unroll
    for (int j = 0; j < NPRE; ++j) {
      const int it = lane + 64 * j;
      const int t = it / CH, c = it - t * CH;
      if (it < items) *reinterpret_cast<uint4*>(&tile[t * PITCH + c * 8]) = pre[j];
    }
    for (int it = lane + 64 * NPRE; it < items; it += 64) {
      const int t = it / CH, c = it - t * CH;
      *reinterpret_cast<uint4*>(&tile[t * PITCH + c * 8]) =
          *reinterpret_cast<const uint4*>(src + (t0 + t) * stride + int64_t(h) * D + c * 8);
    }
    __syncthreads();
    if (full) {
      const int th = lane & 1;
#pragma unroll
      for (int r = 0; r < D / 32; ++r) {
        const int d = 32 * r + (lane >> 1);
        const uint16_t* col = &tile[(8 * th) * PITCH + d];
        uint32_t wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wv[j] = uint32_t(col[(2 * j) * PITCH]) | (uint32_t(col[(2 * j + 1) * PITCH]) << 16);
        *reinterpret_cast<uint4*>(dst + fbase + int64_t(d) * P + 8 * th) =
            make_uint4(wv[0], wv[1], wv[2], wv[3]);
      }
    } else if (has0 || has1) {
#pragma unroll 4
      for (int d = dq; d < D; d += 4) {
        const uint16_t x0 = tile[(2 * pi) * PITCH + d], x1 = tile[(2 * pi + 1) * PITCH + d];
        if (pair) {
          *reinterpret_cast<uint32_t*>(dst + b0 + int64_t(d) * P) =
              uint32_t(x0) | (uint32_t(x1) << 16);
        } else {
          if (has0) dst[b0 + int64_t(d) * P] = x0;
          if (has1) dst[b1 + int64_t(d) * P] = x1;
        }
      }
    }
    __syncthreads();
  };
  pass_of(k, k_stride, kp, kpre);
  pass_of(v, v_stride, vp, vpre);
}

// Scatter of few tokens (decode: one new token per sequence, each on its own page): one wave
// per (token, kv head), lane l moving rows d = l + 64i of K and of V. Every store is a 2-byte
// write into a 32-byte page row, so the cost is latency, and spreading it over n * H waves
// (2048 for a 256-sequence batch with 8 kv heads) instead of one wave per 16 tokens and head
// keeps that latency to about one load and one store round trip.
template <int D>
__global__ __launch_bounds__(64) void kv_scatter16_rows_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint16_t* __restrict__ kp,
    uint16_t* __restrict__ vp, const int64_t* __restrict__ slots, int64_t k_stride,
    int64_t v_stride, int H, int64_t total_slots) {
  constexpr int P = T16_P, R = (D + 63) / 64;
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y, lane = threadIdx.x;
  const int64_t s = slots[t];
  if (s < 0 || s >= total_slots) return;
  const int64_t base = ((s / P) * H + h) * int64_t(D) * P + (s % P);
  uint16_t kr[R], vr[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      kr[i] = k[t * k_stride + int64_t(h) * D + d];
      vr[i] = v[t * v_stride + int64_t(h) * D + d];
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      kp[base + int64_t(d) * P] = kr[i];
      vp[base + int64_t(d) * P] = vr[i];
    }
  }
}

// Gather: LDS tile [D][16 tokens] (row pitch 24: 16-byte aligned rows for the tile loads).
// Lane (t = lane & 15, ci = lane >> 4) builds 16-byte chunks c = 4co + ci of token t's row, so
// one store instruction writes 64 contiguous bytes of each of 16 token rows.
template <int D>
__global__ __launch_bounds__(64) void kv_gather16_kernel(
    uint16_t* __restrict__ ko, uint16_t* __restrict__ vo, const uint16_t* __restrict__ kp,
    const uint16_t* __restrict__ vp, const int32_t* __restrict__ bt, int64_t bt_stride,
    const int64_t* __restrict__ cu, int H, int64_t num_pages) {
  constexpr int P = T16_P, PITCH = 24, CH = D / 8;
  __shared__ __align__(16) uint16_t tile[D * PITCH];
  const int lane = threadIdx.x;
  // x = kv head + H * sequence page: the H waves of one page run together
  const int h = int(blockIdx.x % unsigned(H)), lp = int(blockIdx.x / unsigned(H));
  const int b = blockIdx.y;
  const int64_t row0 = cu[b];
  const int64_t len = cu[b + 1] - row0;
  if (int64_t(lp) * P >= len || lp >= bt_stride) return;
  const int ntok = int(min<int64_t>(P, len - int64_t(lp) * P));
  const int64_t phys = bt[int64_t(b) * bt_stride + lp];
  const bool ok = phys >= 0 && phys < num_pages;
  const int t = lane & 15, ci = lane >> 4;
  for (int pass = 0; pass < 2; ++pass) {
    const uint16_t* src = (pass == 0 ? kp : vp) + (phys * H + h) * int64_t(D) * P;
    uint16_t* dst = pass == 0 ? ko : vo;
    for (int q = lane; q < 2 * D; q += 64) {  // 16-byte chunk q: row d = q / 2, tokens 8(q&1)..
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (ok) w = *reinterpret_cast<const uint4*>(src + q * 8);
      *reinterpret_cast<uint4*>(&tile[(q >> 1) * PITCH + (q & 1) * 8]) = w;
    }
    __syncthreads();
    if (t < ntok) {
      uint16_t* orow = dst + (row0 + int64_t(lp) * P + t) * int64_t(H) * D + int64_t(h) * D;
#pragma unroll
      for (int co = 0; co < CH / 4; ++co) {
        const int c = 4 * co + ci;
        uint32_t wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wv[j] = uint32_t(tile[(8 * c + 2 * j) * PITCH + t]) |
                  (uint32_t(tile[(8 * c + 2 * j + 1) * PITCH + t]) << 16);
        *reinterpret_cast<uint4*>(orow + 8 * c) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Page <-> chunk copy: element-parallel, both sides contiguous along the token axis.
// ---------------------------------------------------------------------------------------------
template <typename W>
__global__ __launch_bounds__(256) void kv_chunk_copy_kernel(
    W* __restrict__ chunk, W* __restrict__ pages, const int64_t* __restrict__ ids, int L,
    int ppc, int H, int D, int P, int64_t num_pages, int to_chunk, int64_t total) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t r = i;
    const int t = int(r % P); r /= P;
    const int d = int(r % D); r /= D;
    const int h = int(r % H); r /= H;
    const int p = int(r % ppc);
    const int l = int(r / ppc);
    const int64_t phys = ids[int64_t(l) * ppc + p];
    if (phys < 0 || phys >= num_pages) continue;
    const int64_t ci = ((int64_t(l) * H + h) * D + d) * (int64_t(ppc) * P) + int64_t(p) * P + t;
    const int64_t pi = ((phys * H + h) * D + d) * P + t;
    if (to_chunk)
      chunk[ci] = pages[pi];
    else
      pages[pi] = chunk[ci];
  }
}

// Many chunks in one launch, one Word (16 bytes where the page row allows) per thread: chunk c
// (its own base address, device memory or device-mapped pinned host memory) row (l, h, d) is
// assembled from the ppc pages of page_ids[(c * L + l) * ppc .. +ppc). Consecutive threads take
// consecutive words of a chunk row, so the chunk side moves whole rows (tokens_per_chunk * elem
// bytes) contiguously, the page side vpr words of each page row.
template <typename Word>
__global__ __launch_bounds__(256) void kv_chunks_copy_kernel(
    Word* const* __restrict__ chunks, Word* __restrict__ pages, const int64_t* __restrict__ ids,
    int L, int ppc, int H, int D, int vpr, int64_t num_pages, int to_chunk, int64_t total) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t r = i;
    const int v = int(r % vpr); r /= vpr;
    const int p = int(r % ppc); r /= ppc;
    const int d = int(r % D); r /= D;
    const int h = int(r % H); r /= H;
    const int l = int(r % L);
    const int64_t c = r / L;
    const int64_t phys = ids[(c * L + l) * ppc + p];
    if (phys < 0 || phys >= num_pages) continue;
    Word* chunk = chunks[c];
    const int64_t ci = (((int64_t(l) * H + h) * D + d) * ppc + p) * vpr + v;
    const int64_t pi = ((phys * H + h) * D + d) * vpr + v;
    if (to_chunk)
      chunk[ci] = pages[pi];
    else
      pages[pi] = chunk[ci];
  }
}

// Token counts up to this take the one-wave-per-(token, kv head) scatter (decode batches);
// larger ones (prefill chunks) the page-segment kernel, whose dword and sector writes pay off.
constexpr int64_t kScatterRowsMaxTokens = 1024;

int check_common(int H, int D, int P, int64_t num_pages, int eb) {
  if (H <= 0 || D <= 0 || P <= 0 || P > 1024 || num_pages <= 0)
    return fail(PIA_EINVAL, "kv: num_kv_heads, head_dim, num_pages must be > 0 and page_size "
                            "in [1, 1024]");
  if (eb != 2 && eb != 4) return fail(PIA_EINVAL, "kv: elem_bytes must be 2 or 4");
  return 0;
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int pia_kv_scatter(const void* k, const void* v, void* k_pages, void* v_pages,
                              const int64_t* slot_mapping, int64_t num_tokens,
                              int64_t k_token_stride, int64_t v_token_stride, int num_kv_heads,
                              int head_dim, int page_size, int64_t num_pages, int elem_bytes,
                              void* stream) {
  if (int rc = check_common(num_kv_heads, head_dim, page_size, num_pages, elem_bytes)) return rc;
  if (num_tokens < 0) return fail(PIA_EINVAL, "kv_scatter: num_tokens < 0");
  if (num_tokens == 0) return 0;
  if (!k || !v || !k_pages || !v_pages || !slot_mapping)
    return fail(PIA_EINVAL, "kv_scatter: null pointer");
  const int HD = num_kv_heads * head_dim;
  if (k_token_stride < HD || v_token_stride < HD)
    return fail(PIA_EINVAL, "kv_scatter: token stride smaller than num_kv_heads*head_dim");
  // Tile path only when the staged [HD][P+1] tile fits in 64 KiB of LDS.
  size_t smem = size_t(page_size + 1) * HD * elem_bytes;
  const int use_tile = smem <= 65536 ? 1 : 0;
  if (!use_tile) smem = 0;
  const int64_t blocks = ceil_div(num_tokens, page_size);
  if (blocks > 0x7fffffff) return fail(PIA_EINVAL, "kv_scatter: too many tokens");
  const int64_t total_slots = num_pages * page_size;
  hipStream_t s = as_stream(stream);
  if (elem_bytes == 2 && page_size == T16_P &&
      (head_dim == 64 || head_dim == 128 || head_dim == 256) && aligned(k, 16) &&
      aligned(v, 16) && k_token_stride % 8 == 0 && v_token_stride % 8 == 0 &&
      aligned(k_pages, 4) && aligned(v_pages, 4) && num_kv_heads <= 65535) {
    if (num_tokens <= kScatterRowsMaxTokens) {  // few tokens: one wave per (token, kv head)
      dim3 grid = dim3(unsigned(num_tokens), unsigned(num_kv_heads));
#define PIA_SCR(DD)                                                                            \
  hipLaunchKernelGGL(kv_scatter16_rows_kernel<DD>, grid, dim3(64), 0, s, (const uint16_t*)k,   \
                     (const uint16_t*)v, (uint16_t*)k_pages, (uint16_t*)v_pages, slot_mapping, \
                     k_token_stride, v_token_stride, num_kv_heads, total_slots)
      if (head_dim == 64) PIA_SCR(64);
      else if (head_dim == 128) PIA_SCR(128);
      else PIA_SCR(256);
#undef PIA_SCR
      return check_launch("kv_scatter");
    }
    if (blocks * num_kv_heads > 0x7fffffff) return fail(PIA_EINVAL, "kv_scatter: too many tokens");
    dim3 grid = dim3(unsigned(blocks * num_kv_heads));
#define PIA_SC16(DD)                                                                           \
  hipLaunchKernelGGL(kv_scatter16_kernel<DD>, grid, dim3(64), 0, s, (const uint16_t*)k,        \
                     (const uint16_t*)v, (uint16_t*)k_pages, (uint16_t*)v_pages, slot_mapping, \
                     num_tokens, k_token_stride, v_token_stride, num_kv_heads, total_slots, wide)
    const int wide = aligned(k_pages, 16) && aligned(v_pages, 16) ? 1 : 0;
    if (head_dim == 64) PIA_SC16(64);
    else if (head_dim == 128) PIA_SC16(128);
    else PIA_SC16(256);
#undef PIA_SC16
    return check_launch("kv_scatter");
  }
  if (elem_bytes == 2)
    hipLaunchKernelGGL(kv_scatter_kernel<uint16_t>, dim3(unsigned(blocks), unsigned(page_size)),
                       dim3(256), smem, s,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)k_pages,
                       (uint16_t*)v_pages, slot_mapping, num_tokens, k_token_stride,
                       v_token_stride, HD, page_size, total_slots, use_tile);
  else
    hipLaunchKernelGGL(kv_scatter_kernel<uint32_t>, dim3(unsigned(blocks), unsigned(page_size)),
                       dim3(256), smem, s,
                       (const uint32_t*)k, (const uint32_t*)v, (uint32_t*)k_pages,
                       (uint32_t*)v_pages, slot_mapping, num_tokens, k_token_stride,
                       v_token_stride, HD, page_size, total_slots, use_tile);
  return check_launch("kv_scatter");
}

extern "C" int pia_kv_gather(void* k_out, void* v_out, const void* k_pages, const void* v_pages,
                             const int32_t* block_tables, int64_t bt_stride,
                             const int64_t* cu_seqlens, int num_seqs, int64_t max_seq_len,
                             int num_kv_heads, int head_dim, int page_size, int64_t num_pages,
                             int elem_bytes, void* stream) {
  if (int rc = check_common(num_kv_heads, head_dim, page_size, num_pages, elem_bytes)) return rc;
  if (num_seqs < 0 || max_seq_len < 0 || bt_stride < 0)
    return fail(PIA_EINVAL, "kv_gather: negative size");
  if (num_seqs == 0 || max_seq_len == 0 || bt_stride == 0) return 0;
  if (!k_out || !v_out || !k_pages || !v_pages || !block_tables || !cu_seqlens)
    return fail(PIA_EINVAL, "kv_gather: null pointer");
  if (num_seqs > 65535) return fail(PIA_EINVAL, "kv_gather: num_seqs > 65535");
  const size_t smem = size_t(page_size + 1) * head_dim * elem_bytes;
  if (smem > 65536) return fail(PIA_EUNSUPPORTED, "kv_gather: page tile exceeds 64 KiB of LDS");
  const int64_t pages = std::min<int64_t>(ceil_div(max_seq_len, page_size), bt_stride);
  if (pages > 0x7fffffff) return fail(PIA_EINVAL, "kv_gather: too many pages");
  hipStream_t s = as_stream(stream);
  if (elem_bytes == 2 && page_size == T16_P &&
      (head_dim == 64 || head_dim == 128 || head_dim == 256) && aligned(k_pages, 16) &&
      aligned(v_pages, 16) && aligned(k_out, 16) && aligned(v_out, 16) &&
      num_kv_heads <= 65535) {
    if (pages * num_kv_heads > 0x7fffffff) return fail(PIA_EINVAL, "kv_gather: too many pages");
    dim3 grid16 = dim3(unsigned(pages * num_kv_heads), unsigned(num_seqs));
#define PIA_GA16(DD)                                                                           \
  hipLaunchKernelGGL(kv_gather16_kernel<DD>, grid16, dim3(64), 0, s, (uint16_t*)k_out,         \
                     (uint16_t*)v_out, (const uint16_t*)k_pages, (const uint16_t*)v_pages,     \
                     block_tables, bt_stride, cu_seqlens, num_kv_heads, num_pages)
    if (head_dim == 64) PIA_GA16(64);
    else if (head_dim == 128) PIA_GA16(128);
    else PIA_GA16(256);
#undef PIA_GA16
    return check_launch("kv_gather");
  }
  dim3 grid = dim3(unsigned(pages), unsigned(num_seqs));
  if (elem_bytes == 2)
    hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, grid, dim3(256), smem, s, (uint16_t*)k_out,
                       (uint16_t*)v_out, (const uint16_t*)k_pages, (const uint16_t*)v_pages,
                       block_tables, bt_stride, cu_seqlens, num_kv_heads, head_dim, page_size,
                       num_pages);
  else
    hipLaunchKernelGGL(kv_gather_kernel<uint32_t>, grid, dim3(256), smem, s, (uint32_t*)k_out,
                       (uint32_t*)v_out, (const uint32_t*)k_pages, (const uint32_t*)v_pages,
                       block_tables, bt_stride, cu_seqlens, num_kv_heads, head_dim, page_size,
                       num_pages);
  return check_launch("kv_gather");
}

extern "C" int pia_kv_pages_chunks_copy(void* const* chunks, int num_chunks, void* pages,
                                        const int64_t* page_ids, int num_layers,
                                        int pages_per_chunk, int num_kv_heads, int head_dim,
                                        int page_size, int64_t num_pages, int elem_bytes,
                                        int to_chunk, void* stream) {
  if (int rc = check_common(num_kv_heads, head_dim, page_size, num_pages, elem_bytes)) return rc;
  if (num_chunks < 0 || num_layers < 0 || pages_per_chunk < 0)
    return fail(PIA_EINVAL, "kv_chunks_copy: negative size");
  const int row_bytes = page_size * elem_bytes;
  int word = 16;
  while (word > 1 && (row_bytes % word || !aligned(pages, word))) word >>= 1;
  const int vpr = row_bytes / word;
  const int64_t total = int64_t(num_chunks) * num_layers * pages_per_chunk * num_kv_heads *
                        head_dim * vpr;
  if (total == 0) return 0;
  if (!chunks || !pages || !page_ids) return fail(PIA_EINVAL, "kv_chunks_copy: null pointer");
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), int64_t(device_cus()) * 16);
  auto launch = [&](auto tag) {
    using Word = decltype(tag);
    hipLaunchKernelGGL(kv_chunks_copy_kernel<Word>, dim3(unsigned(blocks)), dim3(256), 0,
                       as_stream(stream), reinterpret_cast<Word* const*>(chunks),
                       reinterpret_cast<Word*>(pages), page_ids, num_layers, pages_per_chunk,
                       num_kv_heads, head_dim, vpr, num_pages, to_chunk, total);
  };
  switch (word) {
    case 16: launch(uint4{}); break;
    case 8: launch(uint2{}); break;
    case 4: launch(uint32_t{}); break;
    case 2: launch(uint16_t{}); break;
    default: launch(uint8_t{}); break;
  }
  return check_launch("kv_chunks_copy");
}

extern "C" int pia_kv_pages_chunk_copy(void* chunk, void* pages, const int64_t* page_ids,
                                       int num_layers, int pages_per_chunk, int num_kv_heads,
                                       int head_dim, int page_size, int64_t num_pages,
                                       int elem_bytes, int to_chunk, void* stream) {
  if (int rc = check_common(num_kv_heads, head_dim, page_size, num_pages, elem_bytes)) return rc;
  if (num_layers < 0 || pages_per_chunk < 0) return fail(PIA_EINVAL, "kv_chunk_copy: negative size");
  const int64_t total = int64_t(num_layers) * pages_per_chunk * num_kv_heads * head_dim * page_size;
  if (total == 0) return 0;
  if (!chunk || !pages || !page_ids) return fail(PIA_EINVAL, "kv_chunk_copy: null pointer");
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
  hipStream_t s = as_stream(stream);
  if (elem_bytes == 2)
    hipLaunchKernelGGL(kv_chunk_copy_kernel<uint16_t>, dim3(blocks), dim3(256), 0, s,
                       (uint16_t*)chunk, (uint16_t*)pages, page_ids, num_layers, pages_per_chunk,
                       num_kv_heads, head_dim, page_size, num_pages, to_chunk, total);
  else
    hipLaunchKernelGGL(kv_chunk_copy_kernel<uint32_t>, dim3(blocks), dim3(256), 0, s,
                       (uint32_t*)chunk, (uint32_t*)pages, page_ids, num_layers, pages_per_chunk,
                       num_kv_heads, head_dim, page_size, num_pages, to_chunk, total);
  return check_launch("kv_chunk_copy");
}
