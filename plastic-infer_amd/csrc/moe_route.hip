// MoE routing and token permutation:
//   moe_topk_kernel       softmax / top-k / renormalise (one wave per token)
//   moe_align_*           deterministic stable permute plan (counting sort by expert)
//   moe_permute_kernel    hidden rows -> expert-contiguous rows
//   moe_combine_kernel    weighted unpermute (and the plain top-k sum) with fp32 accumulation
#include "pia_internal.h"

namespace pia {
namespace {

// ---------------------------------------------------------------------------------------------
// Top-k router. Lane l holds experts e = l + 64*i. Selection is by descending logit with the
// lowest expert index winning exact ties; softmax is monotone in the logit, so this is the order
// of descending probability.
// ---------------------------------------------------------------------------------------------
template <int DT, int EPL>
__global__ __launch_bounds__(256) void moe_topk_kernel(
    float* __restrict__ w_out, int32_t* __restrict__ id_out, const void* __restrict__ logits_,
    int64_t T, int E, int k, int renorm, int mode, int64_t n_non_padded) {
  using El = Elem<DT>;
  const auto* logits = reinterpret_cast<const typename El::T*>(logits_);
  const int lane = threadIdx.x & 63;
  const int64_t tok = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  float x[EPL];
  bool taken[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    x[i] = e < E ? El::load(logits, tok * E + e) : -INFINITY;
    taken[i] = e >= E;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) mx = fmaxf(mx, x[i]);
  mx = wave_max(mx);
  float ex[EPL], sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    ex[i] = (lane + 64 * i) < E ? expf(x[i] - mx) : 0.f;
    sum += ex[i];
  }
  sum = wave_sum(sum);

  // k rounds of wave argmax; lane kk keeps the kk-th pick.
  float my_x = 0.f, my_ex = 0.f;
  int my_id = -1;
  for (int kk = 0; kk < k; ++kk) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      if (!taken[i] && (x[i] > bv || (x[i] == bv && e < be) || be == 0x7fffffff)) {
        bv = x[i];
        be = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oe = __shfl_xor(be, o, 64);
      if (oe != 0x7fffffff && (be == 0x7fffffff || ov > bv || (ov == bv && oe < be))) {
        bv = ov;
        be = oe;
      }
    }
    // owner of expert be marks it taken and publishes its exp value
    const int owner = be & 63, slot = be >> 6;
    float ex_be = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (i == slot) {
        ex_be = ex[i];
        if (lane == owner) taken[i] = true;
      }
    ex_be = __shfl(ex_be, owner, 64);
    if (lane == kk) {
      my_x = bv;
      my_ex = ex_be;
      my_id = be;
    }
  }

  float w;
  if (mode == 0) {
    w = my_ex / sum;
    if (renorm) {
      const float ws = wave_sum(lane < k ? w : 0.f);
      w = w / ws;
    }
  } else {
    const float top = __shfl(my_x, 0, 64);
    const float e = lane < k ? expf(my_x - top) : 0.f;
    w = e / wave_sum(e);
  }
  if (lane < k) {
    w_out[tok * k + lane] = w;
    id_out[tok * k + lane] = (n_non_padded >= 0 && tok >= n_non_padded) ? -1 : my_id;
  }
}

// ---------------------------------------------------------------------------------------------
// Permute plan. Workspace: counts[E_eff] (int32).
//   moe_align_zero:   counts = 0
//   moe_align_count:  histogram (LDS per block, then global atomics); route_pos[i] = -1 for
//                     dropped routes
//   moe_align_place:  one block per expert e: padded base = sum of padded counts below e;
//                     stable compaction of the routes of e (ascending route index) by wave
//                     ballots; sentinel fill of the padding; expert_ids of its blocks. The last
//                     expert's block also fills the tail beyond num_tokens_post_pad.
// ---------------------------------------------------------------------------------------------
__global__ void moe_align_zero(int32_t* __restrict__ counts, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) counts[i] = 0;
}

__global__ __launch_bounds__(256) void moe_align_count(
    int32_t* __restrict__ counts, int32_t* __restrict__ route_pos,
    const int32_t* __restrict__ ids, int64_t numel, int E_eff) {
  extern __shared__ int32_t hist[];
  for (int i = threadIdx.x; i < E_eff; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < numel;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int e = ids[i];
    if (e >= 0 && e < E_eff)
      atomicAdd(&hist[e], 1);
    else if (route_pos)
      route_pos[i] = -1;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E_eff; i += blockDim.x)
    if (hist[i]) atomicAdd(&counts[i], hist[i]);
}

__global__ __launch_bounds__(256) void moe_align_place(
    int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ npp_out, int32_t* __restrict__ route_pos,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ ids, int64_t numel,
    int E_eff, int bs, int64_t max_padded) {
  __shared__ int32_t red[256];
  __shared__ int32_t wave_cnt[4];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // padded prefix below e and the grand total
  int32_t below = 0, total = 0;
  for (int i = tid; i < E_eff; i += 256) {
    const int32_t pc = ((counts[i] + bs - 1) / bs) * bs;
    total += pc;
    if (i < e) below += pc;
  }
  red[tid] = below;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const int32_t base = red[0];
  __syncthreads();
  red[tid] = total;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const int32_t npp = red[0];
  const int32_t cnt = counts[e];
  const int32_t padded = ((cnt + bs - 1) / bs) * bs;
  if (e == 0 && tid == 0) npp_out[0] = npp;
  for (int i = tid; i < padded / bs; i += 256) expert_ids[base / bs + i] = e;
  for (int i = cnt + tid; i < padded; i += 256) sorted[base + i] = int32_t(numel);
  if (e == E_eff - 1) {
    for (int64_t i = npp + tid; i < max_padded; i += 256) sorted[i] = int32_t(numel);
    const int64_t max_blocks = (max_padded + bs - 1) / bs;
    for (int64_t i = npp / bs + tid; i < max_blocks; i += 256) expert_ids[i] = -1;
  }
  if (cnt == 0) return;

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int32_t running = 0;
  for (int64_t start = 0; start < numel && running < cnt; start += 256) {
    const int64_t i = start + tid;
    const bool match = i < numel && ids[i] == e;
    const uint64_t m = __ballot(match);
    if (lane == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int32_t before = 0, chunk = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w < wave) before += wave_cnt[w];
      chunk += wave_cnt[w];
    }
    if (match) {
      const int32_t pos = base + running + before + __popcll(m & lt_mask);
      sorted[pos] = int32_t(i);
      if (route_pos) route_pos[i] = pos;
    }
    running += chunk;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Permute: one block per destination row; 16-byte words when the row allows it.
// ---------------------------------------------------------------------------------------------
template <typename W>
__global__ __launch_bounds__(256) void moe_permute_kernel(
    W* __restrict__ xp, const W* __restrict__ hidden, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ npp, int64_t numel, int topk, int64_t row_words,
    int64_t hidden_stride_words) {
  const int64_t r = blockIdx.x;
  if (r >= npp[0]) return;
  const int64_t route = sorted[r];
  W* dst = xp + r * row_words;
  if (route < 0 || route >= numel) {
    for (int64_t c = threadIdx.x; c < row_words; c += blockDim.x) dst[c] = W{};
    return;
  }
  const W* src = hidden + (route / topk) * hidden_stride_words;
  for (int64_t c = threadIdx.x; c < row_words; c += blockDim.x) dst[c] = src[c];
}

// ---------------------------------------------------------------------------------------------
// Combine: out[t, c] = sum_s w[t,s] * y[row(t,s), c] in fp32, s ascending; multiply and add are
// rounded separately (no fused multiply-add) so the result is reproducible bit for bit.
// VEC consecutive elements per thread (8 for 16-bit types on 16-byte aligned rows).
// ---------------------------------------------------------------------------------------------
template <int DT, int VEC>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    void* __restrict__ out_, const void* __restrict__ y_, const int32_t* __restrict__ route_pos,
    const float* __restrict__ weights, int64_t y_rows, int64_t T, int k, int H) {
  using El = Elem<DT>;
  using T_ = typename El::T;
  T_* out = reinterpret_cast<T_*>(out_);
  const T_* y = reinterpret_cast<const T_*>(y_);
  const int64_t t = blockIdx.x;
  for (int c0 = threadIdx.x * VEC; c0 < H; c0 += 256 * VEC) {
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
    for (int s = 0; s < k; ++s) {
      const int64_t route = t * k + s;
      const int64_t row = route_pos ? int64_t(route_pos[route]) : route;
      if (row < 0 || row >= y_rows) continue;
      const float w = weights ? weights[route] : 1.f;
      const T_* yr = y + row * H + c0;
      if constexpr (VEC == 8 && sizeof(T_) == 2) {
        const uint4 u = *reinterpret_cast<const uint4*>(yr);
        const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const T_ lo = T_(words[v] & 0xffffu), hi = T_(words[v] >> 16);
          acc[2 * v] = __fadd_rn(acc[2 * v], __fmul_rn(w, El::load(&lo, 0)));
          acc[2 * v + 1] = __fadd_rn(acc[2 * v + 1], __fmul_rn(w, El::load(&hi, 0)));
        }
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          acc[v] = __fadd_rn(acc[v], __fmul_rn(w, El::load(yr, v)));
      }
    }
    T_* o = out + t * H + c0;
#pragma unroll
    for (int v = 0; v < VEC; ++v) El::store(o, v, acc[v]);
  }
}

int launch_combine(void* out, const void* y, int64_t y_rows, const int32_t* route_pos,
                   const float* weights, int64_t T, int k, int H, int dtype, hipStream_t s) {
  if (T == 0 || H == 0) return 0;
  if (T > 0x7fffffff) return fail(PIA_EINVAL, "moe combine: too many tokens");
  const bool vec = dtype != PIA_DTYPE_F32 && H % 8 == 0 && aligned(y, 16);
  dim3 grid = dim3(unsigned(T));
#define PIA_CMB(DT, V)                                                                   \
  hipLaunchKernelGGL((moe_combine_kernel<DT, V>), grid, dim3(256), 0, s, out, y, route_pos, \
                     weights, y_rows, T, k, H)
  switch (dtype) {
    case PIA_DTYPE_F32: PIA_CMB(PIA_DTYPE_F32, 1); break;
    case PIA_DTYPE_BF16:
      if (vec) PIA_CMB(PIA_DTYPE_BF16, 8); else PIA_CMB(PIA_DTYPE_BF16, 1);
      break;
    case PIA_DTYPE_F16:
      if (vec) PIA_CMB(PIA_DTYPE_F16, 8); else PIA_CMB(PIA_DTYPE_F16, 1);
      break;
    default: return fail(PIA_EINVAL, "moe combine: unknown dtype");
  }
#undef PIA_CMB
  return check_launch("moe_combine");
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int pia_moe_topk(float* topk_weights, int32_t* topk_ids, const void* logits,
                            int logits_dtype, int64_t num_tokens, int num_experts, int topk,
                            int renormalize, int mode, int64_t num_token_non_padded,
                            void* stream) {
  if (num_tokens < 0 || num_experts <= 0 || topk <= 0)
    return fail(PIA_EINVAL, "moe_topk: num_tokens >= 0, num_experts > 0, topk > 0 required");
  if (topk > num_experts || topk > 64) return fail(PIA_EINVAL, "moe_topk: topk > min(num_experts, 64)");
  if (num_experts > 1024) return fail(PIA_EUNSUPPORTED, "moe_topk: num_experts > 1024");
  if (mode != 0 && mode != 1) return fail(PIA_EINVAL, "moe_topk: mode must be 0 or 1");
  if (num_tokens == 0) return 0;
  if (!topk_weights || !topk_ids || !logits) return fail(PIA_EINVAL, "moe_topk: null pointer");
  const int64_t blocks = ceil_div(num_tokens, 4);
  if (blocks > 0x7fffffff) return fail(PIA_EINVAL, "moe_topk: too many tokens");
  hipStream_t s = as_stream(stream);
  const int epl = int(ceil_div(num_experts, 64));
#define PIA_TK(DT, EPL)                                                                         \
  hipLaunchKernelGGL((moe_topk_kernel<DT, EPL>), dim3(unsigned(blocks)), dim3(256), 0, s,       \
                     topk_weights, topk_ids, logits, num_tokens, num_experts, topk, renormalize, \
                     mode, num_token_non_padded)
#define PIA_TK_DT(DT)                       \
  if (epl <= 1) PIA_TK(DT, 1);              \
  else if (epl <= 2) PIA_TK(DT, 2);         \
  else if (epl <= 4) PIA_TK(DT, 4);         \
  else if (epl <= 8) PIA_TK(DT, 8);         \
  else PIA_TK(DT, 16);
  switch (logits_dtype) {
    case PIA_DTYPE_F32: PIA_TK_DT(PIA_DTYPE_F32); break;
    case PIA_DTYPE_BF16: PIA_TK_DT(PIA_DTYPE_BF16); break;
    case PIA_DTYPE_F16: PIA_TK_DT(PIA_DTYPE_F16); break;
    default: return fail(PIA_EINVAL, "moe_topk: unknown logits dtype");
  }
#undef PIA_TK_DT
#undef PIA_TK
  return check_launch("moe_topk");
}

extern "C" int64_t pia_moe_align_workspace_bytes(int num_experts) {
  return num_experts < 0 ? 0 : int64_t(num_experts + 1) * int64_t(sizeof(int32_t));
}

extern "C" int pia_moe_align_block_size(int32_t* sorted_token_ids, int32_t* expert_ids,
                                        int32_t* num_tokens_post_pad, int32_t* route_pos,
                                        const int32_t* topk_ids, int64_t numel, int num_experts,
                                        int block_size, int64_t max_num_tokens_padded,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  if (numel < 0 || num_experts <= 0 || block_size <= 0 || max_num_tokens_padded < 0)
    return fail(PIA_EINVAL, "moe_align: invalid size");
  if (numel >= 0x7fffffff || max_num_tokens_padded >= 0x7fffffff)
    return fail(PIA_EINVAL, "moe_align: sizes must fit int32");
  const int E_eff = num_experts + 1;
  if (E_eff > 16384) return fail(PIA_EUNSUPPORTED, "moe_align: more than 16383 experts");
  if (!num_tokens_post_pad || !workspace || (numel > 0 && !topk_ids) ||
      (max_num_tokens_padded > 0 && (!sorted_token_ids || !expert_ids)))
    return fail(PIA_EINVAL, "moe_align: null pointer");
  if (workspace_bytes < pia_moe_align_workspace_bytes(num_experts))
    return fail(PIA_EINVAL, "moe_align: workspace too small");
  // Every expert's padded region must fit: sum(ceil(c/bs)*bs) <= numel + E_eff*(bs-1).
  if (max_num_tokens_padded < std::min<int64_t>(numel + int64_t(E_eff) * (block_size - 1),
                                                numel * block_size))
    return fail(PIA_EINVAL, "moe_align: max_num_tokens_padded below the padded worst case");
  hipStream_t s = as_stream(stream);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(moe_align_zero, dim3(1), dim3(256), 0, s, counts, E_eff);
  if (int rc = check_launch("moe_align_zero")) return rc;
  if (numel > 0) {
    const int64_t blocks = std::min<int64_t>(ceil_div(numel, 256), 1024);
    hipLaunchKernelGGL(moe_align_count, dim3(unsigned(blocks)), dim3(256),
                       size_t(E_eff) * sizeof(int32_t), s, counts, route_pos, topk_ids, numel,
                       E_eff);
    if (int rc = check_launch("moe_align_count")) return rc;
  }
  hipLaunchKernelGGL(moe_align_place, dim3(unsigned(E_eff)), dim3(256), 0, s, sorted_token_ids,
                     expert_ids, num_tokens_post_pad, route_pos, counts, topk_ids, numel, E_eff,
                     block_size, max_num_tokens_padded);
  return check_launch("moe_align_place");
}

extern "C" int pia_moe_permute(void* x_perm, const void* hidden, const int32_t* sorted_token_ids,
                               const int32_t* num_tokens_post_pad, int64_t max_rows,
                               int64_t numel, int topk, int64_t row_bytes,
                               int64_t hidden_row_stride_bytes, void* stream) {
  if (max_rows < 0 || numel < 0 || topk <= 0 || row_bytes <= 0)
    return fail(PIA_EINVAL, "moe_permute: invalid size");
  if (row_bytes % 4 || hidden_row_stride_bytes % 4 || hidden_row_stride_bytes < row_bytes)
    return fail(PIA_EINVAL, "moe_permute: row bytes / stride must be multiples of 4, stride >= row");
  if (max_rows == 0) return 0;
  if (!x_perm || !hidden || !sorted_token_ids || !num_tokens_post_pad)
    return fail(PIA_EINVAL, "moe_permute: null pointer");
  if (max_rows > 0x7fffffff) return fail(PIA_EINVAL, "moe_permute: too many rows");
  hipStream_t s = as_stream(stream);
  const bool v16 = row_bytes % 16 == 0 && hidden_row_stride_bytes % 16 == 0 &&
                   aligned(x_perm, 16) && aligned(hidden, 16);
  if (v16)
    hipLaunchKernelGGL(moe_permute_kernel<uint4>, dim3(unsigned(max_rows)), dim3(256), 0, s,
                       (uint4*)x_perm, (const uint4*)hidden, sorted_token_ids,
                       num_tokens_post_pad, numel, topk, row_bytes / 16,
                       hidden_row_stride_bytes / 16);
  else
    hipLaunchKernelGGL(moe_permute_kernel<uint32_t>, dim3(unsigned(max_rows)), dim3(256), 0, s,
                       (uint32_t*)x_perm, (const uint32_t*)hidden, sorted_token_ids,
                       num_tokens_post_pad, numel, topk, row_bytes / 4,
                       hidden_row_stride_bytes / 4);
  return check_launch("moe_permute");
}

extern "C" int pia_moe_unpermute(void* out, const void* y, int64_t y_rows,
                                 const int32_t* route_pos, const float* topk_weights,
                                 int64_t num_tokens, int topk, int hidden_dim, int dtype,
                                 void* stream) {
  if (num_tokens < 0 || topk <= 0 || hidden_dim < 0)
    return fail(PIA_EINVAL, "moe_unpermute: invalid size");
  if (num_tokens == 0 || hidden_dim == 0) return 0;
  if (!out || !y || !route_pos) return fail(PIA_EINVAL, "moe_unpermute: null pointer");
  return launch_combine(out, y, y_rows, route_pos, topk_weights, num_tokens, topk, hidden_dim,
                        dtype,
                        as_stream(stream));
}

extern "C" int pia_moe_sum_reduce(void* out, const void* in, int64_t num_tokens, int topk,
                                  int hidden_dim, int dtype, void* stream) {
  if (num_tokens < 0 || topk <= 0 || hidden_dim < 0)
    return fail(PIA_EINVAL, "moe_sum_reduce: invalid size");
  if (num_tokens == 0 || hidden_dim == 0) return 0;
  if (!out || !in) return fail(PIA_EINVAL, "moe_sum_reduce: null pointer");
  return launch_combine(out, in, num_tokens * topk, nullptr, nullptr, num_tokens, topk,
                        hidden_dim, dtype,
                        as_stream(stream));
}
