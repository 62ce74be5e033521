// MoE routing and token permutation:
//   moe_topk_kernel       softmax / top-k / renormalise (one wave per token)
//   moe_align_*           deterministic stable permute plan (counting sort by expert)
//   moe_permute_kernel    hidden rows -> expert-contiguous rows
//   moe_combine_kernel    weighted unpermute (and the plain top-k sum) with fp32 accumulation
#include "pia_internal.h"

namespace pia {
namespace {

// DPP exchanges inside rows of 16 lanes (every source lane valid): quad xor 1 / xor 2, then
// rotations by 4 and 8 reach all 16 lanes of the row.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(dpp_i32<CTRL>(__float_as_int(x)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128;

// ---------------------------------------------------------------------------------------------
// Top-k router. A token is served by LPT lanes (16: four tokens per wave, when k <= 16 and
// E <= 256; else 64); lane s of its group holds experts e = s + LPT*i. Selection is by
// descending logit with the lowest expert index winning exact ties; softmax is monotone in
// the logit, so this is the order of descending probability.
// ---------------------------------------------------------------------------------------------
template <int LPT>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (LPT == 16) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppRor4>(v));
    return fmaxf(v, dpp_f32<kDppRor8>(v));
  } else {
#pragma unroll
    for (int o = LPT / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
  }
}
template <int LPT>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPT == 16) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppRor4>(v);
    return v + dpp_f32<kDppRor8>(v);
  } else {
#pragma unroll
    for (int o = LPT / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
  }
}
// (value, expert) argmax step: keep the other lane's pick when it is larger, or equal with a
// lower expert index; be == INT_MAX marks "nothing left".
__device__ __forceinline__ void argmax_take(float& bv, int& be, float ov, int oe) {
  if (oe != 0x7fffffff && (be == 0x7fffffff || ov > bv || (ov == bv && oe < be))) {
    bv = ov;
    be = oe;
  }
}

template <int DT, int EPL, int LPT>
__global__ __launch_bounds__(256) void moe_topk_kernel(
    float* __restrict__ w_out, int32_t* __restrict__ id_out, const void* __restrict__ logits_,
    int64_t T, int E, int k, int renorm, int mode, int64_t n_non_padded) {
  using El = Elem<DT>;
  const auto* logits = reinterpret_cast<const typename El::T*>(logits_);
  const int lane = threadIdx.x & 63, sub = lane % LPT, gbase = lane - sub;
  const int64_t tok = (int64_t(blockIdx.x) * 256 + threadIdx.x) / LPT;
  if (tok >= T) return;  // whole groups leave together; shuffles stay inside a group
  float x[EPL];
  bool taken[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = sub + LPT * i;
    x[i] = e < E ? El::load(logits, tok * E + e) : -INFINITY;
    taken[i] = e >= E;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) mx = fmaxf(mx, x[i]);
  mx = group_max<LPT>(mx);
  float ex[EPL], sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    ex[i] = (sub + LPT * i) < E ? expf(x[i] - mx) : 0.f;
    sum += ex[i];
  }
  sum = group_sum<LPT>(sum);

  // k rounds of group argmax; lane kk of the group keeps the kk-th pick.
  float my_x = 0.f, my_ex = 0.f;
  int my_id = -1;
  for (int kk = 0; kk < k; ++kk) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = sub + LPT * i;
      if (!taken[i] && (x[i] > bv || (x[i] == bv && e < be) || be == 0x7fffffff)) {
        bv = x[i];
        be = e;
      }
    }
    if constexpr (LPT == 16) {
      argmax_take(bv, be, dpp_f32<kDppXor1>(bv), dpp_i32<kDppXor1>(be));
      argmax_take(bv, be, dpp_f32<kDppXor2>(bv), dpp_i32<kDppXor2>(be));
      argmax_take(bv, be, dpp_f32<kDppRor4>(bv), dpp_i32<kDppRor4>(be));
      argmax_take(bv, be, dpp_f32<kDppRor8>(bv), dpp_i32<kDppRor8>(be));
    } else {
#pragma unroll
      for (int o = LPT / 2; o > 0; o >>= 1)
        argmax_take(bv, be, __shfl_xor(bv, o, 64), __shfl_xor(be, o, 64));
    }
    // owner of expert be marks it taken and publishes its exp value
    const int owner = be % LPT, slot = be / LPT;
    float ex_be = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (i == slot) {
        ex_be = ex[i];
        if (sub == owner) taken[i] = true;
      }
    ex_be = __shfl(ex_be, gbase + owner, 64);
    if (sub == kk) {
      my_x = bv;
      my_ex = ex_be;
      my_id = be;
    }
  }

  float w;
  if (mode == 0) {
    w = my_ex / sum;
    if (renorm) {
      const float ws = group_sum<LPT>(sub < k ? w : 0.f);
      w = w / ws;
    }
  } else {
    const float top = __shfl(my_x, gbase, 64);
    const float e = sub < k ? expf(my_x - top) : 0.f;
    w = e / group_sum<LPT>(e);
  }
  if (sub < k) {
    w_out[tok * k + sub] = w;
    id_out[tok * k + sub] = (n_non_padded >= 0 && tok >= n_non_padded) ? -1 : my_id;
  }
}

// ---------------------------------------------------------------------------------------------
// Permute plan: a stable counting sort of the routes by expert, in three launches.
// The routes are cut into nch <= ALIGN_MAX_CHUNKS chunks of csz (a multiple of 256) routes.
// Workspace: chunk_off [E_eff][ALIGN_MAX_CHUNKS] then base [E_eff] (int32).
//   moe_align_hist:    one block per chunk: LDS histogram -> chunk_off[e][c] = count of e in c;
//                      route_pos[i] = -1 for dropped routes (expert outside [0, E_eff))
//   moe_align_scan:    one block: per expert (one wave each in turn), exclusive scan over the
//                      chunks in place and its total; base[e] = exclusive scan of the padded
//                      totals; expert_ids of every block, sentinel fill of the padding and of
//                      the tail past num_tokens_post_pad, expert_ids = -1 past the used blocks
//   moe_align_scatter: one block per chunk, 256 routes at a time: the rank of a route among
//                      the earlier routes of its expert in those 256 (LDS scan) plus a running
//                      per-expert count in LDS gives sorted position
//                      base[e] + chunk_off[e][c] + running[e] + rank (ascending route index).
// ---------------------------------------------------------------------------------------------
constexpr int ALIGN_MAX_CHUNKS = 128;
constexpr int ALIGN_SCAN_THREADS = 1024;

__global__ __launch_bounds__(256) void moe_align_hist(int32_t* __restrict__ chunk_off,
                                                      int32_t* __restrict__ route_pos,
                                                      const int32_t* __restrict__ ids,
                                                      int64_t numel, int64_t csz, int E_eff) {
  extern __shared__ int32_t hist[];
  const int c = blockIdx.x;
  for (int e = threadIdx.x; e < E_eff; e += 256) hist[e] = 0;
  __syncthreads();
  const int64_t lo = int64_t(c) * csz, hi = min(numel, lo + csz);
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
    const int e = ids[i];
    if (e >= 0 && e < E_eff)
      atomicAdd(&hist[e], 1);
    else if (route_pos)
      route_pos[i] = -1;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E_eff; e += 256)
    chunk_off[int64_t(e) * ALIGN_MAX_CHUNKS + c] = hist[e];
}

__global__ __launch_bounds__(ALIGN_SCAN_THREADS) void moe_align_scan(
    int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ npp_out, int32_t* __restrict__ chunk_off, int32_t* __restrict__ base,
    int nch, int E_eff, int bs, int64_t numel, int64_t max_padded) {
  extern __shared__ int32_t cnt_lds[];  // [E_eff] route count per expert
  __shared__ int32_t wsum[ALIGN_SCAN_THREADS / 64];
  __shared__ int32_t total_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // per expert: exclusive scan of its chunk counts, kept in place. SEGS threads per expert,
  // each scanning SEG consecutive chunks; segment totals meet in LDS.
  constexpr int SEG = 16, SEGS = ALIGN_MAX_CHUNKS / SEG, EPP = ALIGN_SCAN_THREADS / SEGS;
  __shared__ int32_t seg_tot[ALIGN_SCAN_THREADS];
  for (int ebase = 0; ebase < E_eff; ebase += EPP) {
    const int e = ebase + tid / SEGS, sg = tid % SEGS;
    int32_t v[SEG];
    int32_t run = 0;
    if (e < E_eff) {
      const int4* row = reinterpret_cast<const int4*>(chunk_off + int64_t(e) * ALIGN_MAX_CHUNKS +
                                                      sg * SEG);
#pragma unroll
      for (int q = 0; q < SEG / 4; ++q) {
        const int4 w4 = row[q];
        v[4 * q] = w4.x;
        v[4 * q + 1] = w4.y;
        v[4 * q + 2] = w4.z;
        v[4 * q + 3] = w4.w;
      }
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const int32_t x = (sg * SEG + i < nch) ? v[i] : 0;  // chunks past nch were never written
        v[i] = run;
        run += x;
      }
    }
    seg_tot[tid] = run;
    __syncthreads();
    if (e < E_eff) {
      int32_t before = 0;
      for (int j = 0; j < sg; ++j) before += seg_tot[tid - sg + j];
      int32_t* row = chunk_off + int64_t(e) * ALIGN_MAX_CHUNKS + sg * SEG;
#pragma unroll
      for (int i = 0; i < SEG; ++i)
        if (sg * SEG + i < nch) row[i] = before + v[i];
      if (sg == SEGS - 1) cnt_lds[e] = before + run;
    }
    __syncthreads();
  }
  // exclusive scan of the padded counts over the experts: consecutive experts per thread
  const int per = (E_eff + ALIGN_SCAN_THREADS - 1) / ALIGN_SCAN_THREADS;
  const int e0 = tid * per, e1 = min(E_eff, e0 + per);
  int32_t mine = 0;
  for (int e = e0; e < e1; ++e) mine += ((cnt_lds[e] + bs - 1) / bs) * bs;
  int32_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t off = incl - mine;
  for (int w = 0; w < wave; ++w) off += wsum[w];
  if (tid == ALIGN_SCAN_THREADS - 1) total_lds = off + mine;
  __syncthreads();
  const int32_t npp = total_lds;
  for (int e = e0; e < e1; ++e) {
    const int32_t cnt = cnt_lds[e];
    const int32_t padded = ((cnt + bs - 1) / bs) * bs;
    base[e] = off;
    for (int b = 0; b < padded / bs; ++b) expert_ids[off / bs + b] = e;
    for (int i = cnt; i < padded; ++i) sorted[off + i] = int32_t(numel);
    off += padded;
  }
  if (tid == 0) npp_out[0] = npp;
  for (int64_t i = npp + tid; i < max_padded; i += ALIGN_SCAN_THREADS) sorted[i] = int32_t(numel);
  const int64_t max_blocks = (max_padded + bs - 1) / bs;
  for (int64_t i = npp / bs + tid; i < max_blocks; i += ALIGN_SCAN_THREADS) expert_ids[i] = -1;
}

__global__ __launch_bounds__(256) void moe_align_scatter(
    int32_t* __restrict__ sorted, int32_t* __restrict__ route_pos,
    const int32_t* __restrict__ chunk_off, const int32_t* __restrict__ base,
    const int32_t* __restrict__ ids, int64_t numel, int64_t csz, int E_eff) {
  extern __shared__ int32_t running[];  // [E_eff]
  __shared__ int32_t ids_lds[256];
  const int c = blockIdx.x, tid = threadIdx.x;
  for (int e = tid; e < E_eff; e += 256) running[e] = 0;
  const int64_t lo = int64_t(c) * csz, hi = min(numel, lo + csz);
  for (int64_t s0 = lo; s0 < hi; s0 += 256) {
    const int64_t i = s0 + tid;
    const int e = i < hi ? ids[i] : -1;
    const bool ok = e >= 0 && e < E_eff;
    ids_lds[tid] = ok ? e : -1;
    __syncthreads();
    if (ok) {
      int rank = 0;
      for (int j = 0; j < tid; ++j) rank += ids_lds[j] == e ? 1 : 0;
      const int32_t pos =
          base[e] + chunk_off[int64_t(e) * ALIGN_MAX_CHUNKS + c] + running[e] + rank;
      sorted[pos] = int32_t(i);
      if (route_pos) route_pos[i] = pos;
    }
    __syncthreads();
    if (ok) atomicAdd(&running[e], 1);
    __syncthreads();
  }
}

// Small plans (numel <= ALIGN_SMALL_MAX, the decode sizes) in one launch of one 1024-thread
// block: ids and a per-expert count live in LDS; the exclusive scan and the fills are those of
// moe_align_scan; a route's position is its expert's padded base plus the number of earlier
// routes of that expert (ascending route index, the same plan as the three-launch path).
constexpr int ALIGN_SMALL_MAX = 4096;
constexpr int ALIGN_SMALL_MAX_E = 12288;  // cnt[] of 48 KiB next to the 16 KiB of ids

__global__ __launch_bounds__(1024) void moe_align_small(
    int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids, int32_t* __restrict__ npp_out,
    int32_t* __restrict__ route_pos, const int32_t* __restrict__ ids, int numel, int E_eff, int bs,
    int64_t max_padded) {
  __shared__ __attribute__((aligned(16))) int32_t ids_lds[ALIGN_SMALL_MAX];
  __shared__ int32_t wsum[16];
  __shared__ int32_t total_lds;
  extern __shared__ int32_t cnt[];  // [E_eff]: count, then the padded base plus routes placed
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E_eff; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < numel; i += 1024) {
    const int e = ids[i];
    const bool ok = e >= 0 && e < E_eff;
    ids_lds[i] = ok ? e : -1;
    if (ok)
      atomicAdd(&cnt[e], 1);
    else if (route_pos)
      route_pos[i] = -1;
  }
  __syncthreads();
  const int per = (E_eff + 1023) / 1024;
  const int e0 = min(E_eff, tid * per), e1 = min(E_eff, e0 + per);
  int32_t mine = 0;
  for (int e = e0; e < e1; ++e) mine += ((cnt[e] + bs - 1) / bs) * bs;
  int32_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t off = incl - mine;
  for (int w = 0; w < wave; ++w) off += wsum[w];
  if (tid == 1023) total_lds = off + mine;
  __syncthreads();
  const int32_t npp = total_lds;
  for (int e = e0; e < e1; ++e) {
    const int32_t c = cnt[e];
    const int32_t padded = ((c + bs - 1) / bs) * bs;
    for (int b = 0; b < padded / bs; ++b) expert_ids[off / bs + b] = e;
    for (int i = c; i < padded; ++i) sorted[off + i] = numel;
    cnt[e] = off;
    off += padded;
  }
  if (tid == 0) npp_out[0] = npp;
  for (int64_t i = npp + tid; i < max_padded; i += 1024) sorted[i] = numel;
  const int64_t max_blocks = (max_padded + bs - 1) / bs;
  for (int64_t i = npp / bs + tid; i < max_blocks; i += 1024) expert_ids[i] = -1;
  __syncthreads();
  // Routes go in 64-route groups, one per wave, in group order: a wave reads the running count
  // of its experts, adds the rank among its own lower lanes (readlane loop), writes, then adds
  // its counts; one barrier per group keeps the groups in order.
  for (int g0 = 0; g0 < numel; g0 += 64 * 16) {
    const int i = g0 + tid;
    const int e = i < numel ? ids_lds[i] : -1;
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < 64; ++j) {
      const int ej = __builtin_amdgcn_readlane(e, j);
      rank += (j < lane && ej == e) ? 1 : 0;
    }
    const int groups = min(16, (numel - g0 + 63) / 64);
    for (int w = 0; w < groups; ++w) {
      if (wave == w && e >= 0) {
        const int32_t pos = cnt[e] + rank;
        sorted[pos] = i;
        if (route_pos) route_pos[i] = pos;
        atomicAdd(&cnt[e], 1);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Permute: a wave moves four destination rows (sixteen per 256-thread block) with the loads of
// all four issued before their stores; 16-byte words when the row allows it. Rows past
// *num_tokens_post_pad are left untouched, padding rows are zeroed.
// ---------------------------------------------------------------------------------------------
constexpr int PERM_ROWS_PER_WAVE = 4;
constexpr int PERM_ROWS_PER_BLOCK = 4 * PERM_ROWS_PER_WAVE;

template <typename W>
__global__ __launch_bounds__(256) void moe_permute_kernel(
    W* __restrict__ xp, const W* __restrict__ hidden, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ npp, int64_t max_rows, int64_t numel, int topk,
    int64_t row_words, int64_t hidden_stride_words) {
  constexpr int R = PERM_ROWS_PER_WAVE, U = 4;  // rows per wave, words per lane per row
  const int lane = threadIdx.x & 63;
  const int64_t r0 = int64_t(blockIdx.x) * PERM_ROWS_PER_BLOCK + (threadIdx.x >> 6) * R;
  const int64_t nrows = min<int64_t>(max_rows, npp[0]);
  if (r0 >= nrows) return;
  int64_t my_route = -1;
  if (lane < R && r0 + lane < nrows) my_route = sorted[r0 + lane];
  const W* src[R];
  bool live[R], pad[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int64_t route = __shfl(my_route, j, 64);
    live[j] = r0 + j < nrows;
    pad[j] = route < 0 || route >= numel;
    src[j] = hidden + (pad[j] ? 0 : (route / topk) * hidden_stride_words);
  }
  for (int64_t c0 = 0; c0 < row_words; c0 += 64 * U) {
    W buf[R][U];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + lane + 64 * u;
        buf[j][u] = (live[j] && !pad[j] && c < row_words) ? src[j][c] : W{};
      }
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + lane + 64 * u;
        if (live[j] && c < row_words) xp[(r0 + j) * row_words + c] = buf[j][u];
      }
  }
}

// Token-major permute (route_pos given): blocks [0, token_blocks) give one wave per token,
// which reads the token's row once and stores it to each of its routes' rows; the remaining
// blocks check 256 destination rows each and zero the padding rows among them.
template <typename W>
__global__ __launch_bounds__(256) void moe_permute_tokens_kernel(
    W* __restrict__ xp, const W* __restrict__ hidden, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ route_pos, const int32_t* __restrict__ npp, int64_t max_rows,
    int64_t numel, int topk, int64_t row_words, int64_t hidden_stride_words,
    int64_t token_blocks) {
  constexpr int U = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nrows = min<int64_t>(max_rows, npp[0]);
  if (int64_t(blockIdx.x) < token_blocks) {
    const int64_t t = int64_t(blockIdx.x) * 4 + wave;
    if (t >= numel / topk) return;
    const int my_r = lane < topk ? route_pos[t * topk + lane] : -1;
    const W* src = hidden + t * hidden_stride_words;
    for (int64_t c0 = 0; c0 < row_words; c0 += 64 * U) {
      W buf[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + lane + 64 * u;
        buf[u] = c < row_words ? src[c] : W{};
      }
      for (int sl = 0; sl < topk; ++sl) {
        const int r = __shfl(my_r, sl, 64);
        if (r < 0 || r >= nrows) continue;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + lane + 64 * u;
          if (c < row_words) xp[int64_t(r) * row_words + c] = buf[u];
        }
      }
    }
    return;
  }
  const int64_t rbase = (int64_t(blockIdx.x) - token_blocks) * 256 + wave * 64;
  const int64_t r = rbase + lane;
  bool is_pad = false;
  if (r < nrows) {
    const int32_t route = sorted[r];
    is_pad = route < 0 || route >= numel;
  }
  uint64_t pads = __ballot(is_pad);
  while (pads) {
    const int j = __builtin_ctzll(pads);
    pads &= pads - 1;
    W* dst = xp + (rbase + j) * row_words;
    for (int64_t c = lane; c < row_words; c += 64) dst[c] = W{};
  }
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
  constexpr int KU = 8;  // routes whose rows are loaded before they are accumulated
  T_* out = reinterpret_cast<T_*>(out_);
  const T_* y = reinterpret_cast<const T_*>(y_);
  const int64_t t = blockIdx.x;
  for (int c0 = threadIdx.x * VEC; c0 < H; c0 += 256 * VEC) {
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
    if constexpr (VEC == 8 && sizeof(T_) == 2) {
      for (int s0 = 0; s0 < k; s0 += KU) {
        uint4 u[KU];
        float w[KU];
        bool ok[KU];
#pragma unroll
        for (int j = 0; j < KU; ++j) {
          const int s = s0 + j;
          const int64_t route = t * k + s;
          const int64_t row = s < k ? (route_pos ? int64_t(route_pos[route]) : route) : -1;
          ok[j] = row >= 0 && row < y_rows;
          w[j] = (ok[j] && weights) ? weights[route] : 1.f;
          u[j] = ok[j] ? *reinterpret_cast<const uint4*>(y + row * H + c0) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < KU; ++j) {
          if (!ok[j]) continue;
          const uint32_t words[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const T_ lo = T_(words[v] & 0xffffu), hi = T_(words[v] >> 16);
            acc[2 * v] = __fadd_rn(acc[2 * v], __fmul_rn(w[j], El::load(&lo, 0)));
            acc[2 * v + 1] = __fadd_rn(acc[2 * v + 1], __fmul_rn(w[j], El::load(&hi, 0)));
          }
        }
      }
    } else {
      for (int s = 0; s < k; ++s) {
        const int64_t route = t * k + s;
        const int64_t row = route_pos ? int64_t(route_pos[route]) : route;
        if (row < 0 || row >= y_rows) continue;
        const float w = weights ? weights[route] : 1.f;
        const T_* yr = y + row * H + c0;
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __fadd_rn(acc[v], __fmul_rn(w, El::load(yr, v)));
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
  hipStream_t s = as_stream(stream);
  const bool narrow = topk <= 16 && num_experts <= 256;  // 16 lanes per token
  const int lpt = narrow ? 16 : 64;
  const int64_t blocks = ceil_div(num_tokens * lpt, 256);
  if (blocks > 0x7fffffff) return fail(PIA_EINVAL, "moe_topk: too many tokens");
  const int epl = int(ceil_div(num_experts, lpt));
#define PIA_TK(DT, EPL, LPT)                                                                    \
  hipLaunchKernelGGL((moe_topk_kernel<DT, EPL, LPT>), dim3(unsigned(blocks)), dim3(256), 0, s,  \
                     topk_weights, topk_ids, logits, num_tokens, num_experts, topk, renormalize, \
                     mode, num_token_non_padded)
#define PIA_TK_DT(DT)                                \
  if (narrow) {                                      \
    if (epl <= 1) PIA_TK(DT, 1, 16);                 \
    else if (epl <= 2) PIA_TK(DT, 2, 16);            \
    else if (epl <= 4) PIA_TK(DT, 4, 16);            \
    else if (epl <= 8) PIA_TK(DT, 8, 16);            \
    else PIA_TK(DT, 16, 16);                         \
  } else {                                           \
    if (epl <= 1) PIA_TK(DT, 1, 64);                 \
    else if (epl <= 2) PIA_TK(DT, 2, 64);            \
    else if (epl <= 4) PIA_TK(DT, 4, 64);            \
    else if (epl <= 8) PIA_TK(DT, 8, 64);            \
    else PIA_TK(DT, 16, 64);                         \
  }
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
  return num_experts < 0 ? 0
                         : int64_t(ALIGN_MAX_CHUNKS + 1) * int64_t(num_experts + 1) *
                               int64_t(sizeof(int32_t));
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
  if (!aligned(workspace, 16)) return fail(PIA_EINVAL, "moe_align: workspace must be 16-byte aligned");
  // Every expert's padded region must fit: sum(ceil(c/bs)*bs) <= numel + E_eff*(bs-1).
  if (max_num_tokens_padded < std::min<int64_t>(numel + int64_t(E_eff) * (block_size - 1),
                                                numel * block_size))
    return fail(PIA_EINVAL, "moe_align: max_num_tokens_padded below the padded worst case");
  hipStream_t s = as_stream(stream);
  if (numel <= ALIGN_SMALL_MAX && E_eff <= ALIGN_SMALL_MAX_E) {
    hipLaunchKernelGGL(moe_align_small, dim3(1), dim3(1024), size_t(E_eff) * sizeof(int32_t), s,
                       sorted_token_ids, expert_ids, num_tokens_post_pad, route_pos, topk_ids,
                       int(numel), E_eff, block_size, max_num_tokens_padded);
    return check_launch("moe_align_small");
  }
  int32_t* chunk_off = reinterpret_cast<int32_t*>(workspace);
  int32_t* base = chunk_off + int64_t(ALIGN_MAX_CHUNKS) * E_eff;
  const int64_t csz = std::max<int64_t>(256, ceil_div(ceil_div(numel, ALIGN_MAX_CHUNKS), 256) * 256);
  const int nch = int(ceil_div(numel, csz));
  const size_t lds = size_t(E_eff) * sizeof(int32_t);
  if (nch > 0) {
    hipLaunchKernelGGL(moe_align_hist, dim3(unsigned(nch)), dim3(256), lds, s, chunk_off,
                       route_pos, topk_ids, numel, csz, E_eff);
    if (int rc = check_launch("moe_align_hist")) return rc;
  }
  hipLaunchKernelGGL(moe_align_scan, dim3(1), dim3(ALIGN_SCAN_THREADS), lds, s, sorted_token_ids,
                     expert_ids, num_tokens_post_pad, chunk_off, base, nch, E_eff, block_size,
                     numel, max_num_tokens_padded);
  if (int rc = check_launch("moe_align_scan")) return rc;
  if (nch > 0) {
    hipLaunchKernelGGL(moe_align_scatter, dim3(unsigned(nch)), dim3(256), lds, s,
                       sorted_token_ids, route_pos, chunk_off, base, topk_ids, numel, csz, E_eff);
    if (int rc = check_launch("moe_align_scatter")) return rc;
  }
  return 0;
}

extern "C" int pia_moe_permute(void* x_perm, const void* hidden, const int32_t* sorted_token_ids,
                               const int32_t* route_pos, const int32_t* num_tokens_post_pad,
                               int64_t max_rows, int64_t numel, int topk, int64_t row_bytes,
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
  if (route_pos && topk <= 64) {
    const int64_t token_blocks = ceil_div(numel / topk, 4);
    const int64_t blocks = token_blocks + ceil_div(max_rows, 256);
    if (blocks > 0x7fffffff) return fail(PIA_EINVAL, "moe_permute: too many rows");
    if (v16)
      hipLaunchKernelGGL(moe_permute_tokens_kernel<uint4>, dim3(unsigned(blocks)), dim3(256), 0,
                         s, (uint4*)x_perm, (const uint4*)hidden, sorted_token_ids, route_pos,
                         num_tokens_post_pad, max_rows, numel, topk, row_bytes / 16,
                         hidden_row_stride_bytes / 16, token_blocks);
    else
      hipLaunchKernelGGL(moe_permute_tokens_kernel<uint32_t>, dim3(unsigned(blocks)), dim3(256),
                         0, s, (uint32_t*)x_perm, (const uint32_t*)hidden, sorted_token_ids,
                         route_pos, num_tokens_post_pad, max_rows, numel, topk, row_bytes / 4,
                         hidden_row_stride_bytes / 4, token_blocks);
    return check_launch("moe_permute");
  }
  const unsigned blocks = unsigned(ceil_div(max_rows, PERM_ROWS_PER_BLOCK));
  if (v16)
    hipLaunchKernelGGL(moe_permute_kernel<uint4>, dim3(blocks), dim3(256), 0, s, (uint4*)x_perm,
                       (const uint4*)hidden, sorted_token_ids, num_tokens_post_pad, max_rows,
                       numel, topk, row_bytes / 16, hidden_row_stride_bytes / 16);
  else
    hipLaunchKernelGGL(moe_permute_kernel<uint32_t>, dim3(blocks), dim3(256), 0, s,
                       (uint32_t*)x_perm, (const uint32_t*)hidden, sorted_token_ids,
                       num_tokens_post_pad, max_rows, numel, topk, row_bytes / 4,
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
