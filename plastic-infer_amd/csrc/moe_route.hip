// MoE routing and token permutation:
//   moe_topk_wave_kernel  softmax / top-k / renormalise (one wave per token, radix select)
//   moe_topk_hist_kernel  the same, also counting the permute plan's per-chunk experts
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

// Plan chunks of the counting-sort permute plan (histogram table row length: one top-k block
// of 16 tokens per chunk up to 4096 tokens).
constexpr int ALIGN_MAX_CHUNKS = 256;

__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave reductions: DPP inside each row of 16 lanes (every lane of a row then holds the row's
// result), then the four row results read as scalars (no LDS round trip), summed as
// (row0 + row1) + (row2 + row3) in every lane.
__device__ __forceinline__ float row_lane(float v, int row) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * row));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRor4>(v));
  v = fmaxf(v, dpp_f32<kDppRor8>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 1)), fmaxf(row_lane(v, 2), row_lane(v, 3)));
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppRor4>(v);
  v += dpp_f32<kDppRor8>(v);
  return (row_lane(v, 0) + row_lane(v, 1)) + (row_lane(v, 2) + row_lane(v, 3));
}

// One token's top-k on one wave: writes k (weight, id) pairs at tok * k + slot and returns,
// per held expert, whether it was selected (for the caller's histogram).
template <int DT, int EPL>
__device__ __forceinline__ void topk_one_token(float* __restrict__ w_out,
                                               int32_t* __restrict__ id_out,
                                               const typename Elem<DT>::T* __restrict__ logits,
                                               int64_t tok, int E, int k, int renorm, int mode,
                                               bool padded_tok, int lane, bool (&sel)[EPL]) {
  using El = Elem<DT>;
  float x[EPL];
  uint32_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    x[i] = e < E ? El::load(logits, tok * E + e) : -INFINITY;
    key[i] = e < E ? order_key(x[i]) : 0u;
  }
  // k-th largest key
  uint32_t t = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = t | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) cnt += __popcll(__ballot(key[i] >= cand));
    if (cnt >= k) t = cand;
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) gt += __popcll(__ballot(key[i] > t));
  int need = k - gt;  // keys == t to take, lowest expert index first
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t msk[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    const uint64_t eq = __ballot(e < E && key[i] == t);
    sel[i] = (e < E) && (key[i] > t || (key[i] == t && __popcll(eq & below) < need));
    need -= min(need, __popcll(eq));
    msk[i] = __ballot(sel[i]);
  }
  // output slots
  int slot[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) slot[i] = 0;
#pragma unroll
  for (int i2 = 0; i2 < EPL; ++i2) {
    uint64_t m = msk[i2];
    while (m) {
      const int j = __builtin_ctzll(m);
      m &= m - 1;
      const uint32_t kj = __builtin_amdgcn_readlane(key[i2], j);
      const int ej = j + 64 * i2;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int e = lane + 64 * i;
        slot[i] += (kj > key[i] || (kj == key[i] && ej < e)) ? 1 : 0;
      }
    }
  }
  // weights
  float wv[EPL];
  if (mode == 0) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; ++i) mx = fmaxf(mx, x[i]);
    mx = wave_max_f(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      wv[i] = (lane + 64 * i) < E ? expf(x[i] - mx) : 0.f;
      sum += wv[i];
    }
    sum = wave_sum_f(sum);
    float ssel = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      wv[i] = wv[i] / sum;
      ssel += sel[i] ? wv[i] : 0.f;
    }
    if (renorm) {
      ssel = wave_sum_f(ssel);
#pragma unroll
      for (int i = 0; i < EPL; ++i) wv[i] = wv[i] / ssel;
    }
  } else {
    float top = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; ++i) top = fmaxf(top, sel[i] ? x[i] : -INFINITY);
    top = wave_max_f(top);
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      wv[i] = sel[i] ? expf(x[i] - top) : 0.f;
      ssum += wv[i];
    }
    ssum = wave_sum_f(ssum);
#pragma unroll
    for (int i = 0; i < EPL; ++i) wv[i] = wv[i] / ssum;
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    if (sel[i]) {
      w_out[tok * k + slot[i]] = wv[i];
      id_out[tok * k + slot[i]] = padded_tok ? -1 : lane + 64 * i;
    }
  }
}

template <int DT, int EPL>
__global__ __launch_bounds__(256) void moe_topk_wave_kernel(
    float* __restrict__ w_out, int32_t* __restrict__ id_out, const void* __restrict__ logits_,
    int64_t T, int E, int k, int renorm, int mode, int64_t n_non_padded) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  if (tok >= T) return;  // whole waves leave together
  bool sel[EPL];
  topk_one_token<DT, EPL>(w_out, id_out,
                          reinterpret_cast<const typename Elem<DT>::T*>(logits_), tok, E, k,
                          renorm, mode, n_non_padded >= 0 && tok >= n_non_padded, lane, sel);
}

// Top-k with the permute plan's histogram: block c (16 waves) routes tokens
// [c * tpb, (c + 1) * tpb), which are exactly plan chunk c (csz = tpb * k routes), and writes
// chunk_cnt[e][c] = routes of expert e in the chunk, one byte each (a token routes to an expert
// at most once, so a count is at most tpb <= 240); routes of padded tokens (id -1) get
// route_pos = -1. moe_align_place<uint8_t> then builds the plan from the table.
template <int DT, int EPL>
__global__ __launch_bounds__(1024) void moe_topk_hist_kernel(
    float* __restrict__ w_out, int32_t* __restrict__ id_out, const void* __restrict__ logits_,
    int64_t T, int E, int k, int renorm, int mode, int64_t n_non_padded, int tpb,
    uint8_t* __restrict__ chunk_cnt, int32_t* __restrict__ route_pos) {
  extern __shared__ int32_t hist[];  // [E + 1]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x;
  for (int e = tid; e <= E; e += 1024) hist[e] = 0;
  __syncthreads();
  for (int j = wave; j < tpb; j += 16) {
    const int64_t tok = int64_t(c) * tpb + j;
    if (tok >= T) break;
    const bool padded_tok = n_non_padded >= 0 && tok >= n_non_padded;
    bool sel[EPL];
    topk_one_token<DT, EPL>(w_out, id_out,
                            reinterpret_cast<const typename Elem<DT>::T*>(logits_), tok, E, k,
                            renorm, mode, padded_tok, lane, sel);
    if (padded_tok) {
      if (route_pos && lane < k) route_pos[tok * k + lane] = -1;
    } else {
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (sel[i]) atomicAdd(&hist[lane + 64 * i], 1);
    }
  }
  __syncthreads();
  for (int e = tid; e <= E; e += 1024)
    chunk_cnt[int64_t(e) * ALIGN_MAX_CHUNKS + c] = uint8_t(hist[e]);
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

// Placement in one launch after moe_align_hist (replaces scan + scatter when E_eff <= 1024):
// one 256-thread block per chunk c. Each block derives what it needs from the histogram table
// itself: for every expert e (a thread per expert) its total over all chunks and its count in
// the chunks before c; an exclusive scan of the padded totals gives the expert bases (every
// block computes the same bases), so a route of chunk c goes to
//     base[e] + (routes of e in chunks < c) + (routes of e earlier in chunk c).
// The last term: in rounds of 256 routes, the rank among the earlier lanes of its wave
// (readlane loop), plus the routes of e in the earlier waves of the round (per-wave counts in
// LDS), plus the routes of e in the earlier rounds (a running count per expert).
// Block c also does a stripe of the fills: expert_ids and padding sentinels of the experts
// e = c, c + nch, ..., and of the tail past num_tokens_post_pad.
constexpr int ALIGN_PLACE_MAX_E = 512;   // LDS: (4 + 16 waves) x E_eff ints

// Sum over the wave (modulo 2^32), wave-uniform: DPP inside rows of 16, then the four row sums
// by readlane.
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
  v += uint32_t(dpp_i32<kDppXor1>(int(v)));
  v += uint32_t(dpp_i32<kDppXor2>(int(v)));
  v += uint32_t(dpp_i32<kDppRor4>(int(v)));
  v += uint32_t(dpp_i32<kDppRor8>(int(v)));
  return uint32_t(__builtin_amdgcn_readlane(int(v), 0)) +
         uint32_t(__builtin_amdgcn_readlane(int(v), 16)) +
         uint32_t(__builtin_amdgcn_readlane(int(v), 32)) +
         uint32_t(__builtin_amdgcn_readlane(int(v), 48));
}

// Inclusive prefix sum over the 64 lanes by DPP: row_shr 1/2/4/8 inside rows of 16 (lanes
// without a source add 0), then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2, 3.
__device__ __forceinline__ int wave_incl_scan_dpp(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  return x;
}

constexpr int PLACE_THREADS = 1024, PLACE_WAVES = PLACE_THREADS / 64;

// Bytes b..b+3 of a word that belong to chunks below lim (chunk of byte b: cb).
__device__ __forceinline__ uint32_t bytes_below(uint32_t word, int cb, int lim) {
  const int n = min(max(lim - cb, 0), 4);
  return n >= 4 ? word : word & ((1u << (8 * n)) - 1u);
}

template <typename CT>
__global__ __launch_bounds__(PLACE_THREADS) void moe_align_place(
    int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ npp_out, int32_t* __restrict__ route_pos,
    const CT* __restrict__ chunk_off, const int32_t* __restrict__ ids, int64_t numel,
    int64_t csz, int nch, int E_eff, int bs, int64_t max_padded) {
  // start[E_eff] | total[E_eff] | running[E_eff] | count[E_eff] | wcnt[PLACE_WAVES][E_eff]
  extern __shared__ int32_t pl[];
  int32_t* start = pl;
  int32_t* total = pl + E_eff;
  int32_t* running = pl + 2 * E_eff;
  int32_t* count = pl + 3 * E_eff;
  int32_t* wcnt = pl + 4 * E_eff;
  __shared__ int32_t npp_lds;
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t lo = int64_t(c) * csz, hi = min(numel, lo + csz);
  // the first round's expert ids, fetched before the histogram reads and parked in LDS right
  // after those reads are issued, so both latencies overlap
  __shared__ int32_t first_ids[PLACE_THREADS];
  int e_first = -1;
  if (lo + tid < hi) e_first = ids[lo + tid];

  // 1. per expert: routes in the chunks before c, and in all chunks.
  if constexpr (sizeof(CT) == 1) {
    // One byte per chunk: a row of 256 counts is 16 lanes' 16 bytes, so one load instruction
    // reads four experts' rows (lanes 16 g .. 16 g + 15: expert row g of the four, chunks
    // 16 j .. 16 j + 15 in lane j). Byte sums by v_sad_u8, both counts packed in one word
    // (an expert's total is at most the token count, < 2^16) and summed inside each row of
    // 16 lanes by DPP.
    constexpr int EB8 = 3;   // groups of four rows in flight per wave
    const int g = lane >> 4, j = lane & 15;
    for (int eb = wave * 4 * EB8; eb < E_eff; eb += PLACE_WAVES * 4 * EB8) {
      uint4 v[EB8];
#pragma unroll
      for (int q = 0; q < EB8; ++q) {
        const int e = eb + 4 * q + g;
        v[q] = make_uint4(0, 0, 0, 0);
        if (e < E_eff)
          v[q] = *reinterpret_cast<const uint4*>(chunk_off + int64_t(e) * ALIGN_MAX_CHUNKS + 16 * j);
      }
      if (eb == wave * 4 * EB8) first_ids[tid] = e_first;
#pragma unroll
      for (int q = 0; q < EB8; ++q) {
        const uint32_t w4[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
        uint32_t sum_l = 0, pre_l = 0;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int cb = 16 * j + 4 * h;   // chunk of the word's first byte
          const uint32_t valid = bytes_below(w4[h], cb, nch);   // chunks past nch: unwritten
          sum_l = __builtin_amdgcn_sad_u8(valid, 0u, sum_l);
          pre_l = __builtin_amdgcn_sad_u8(bytes_below(valid, cb, c), 0u, pre_l);
        }
        int both = int((sum_l << 16) | pre_l);
        both += dpp_i32<kDppXor1>(both);
        both += dpp_i32<kDppXor2>(both);
        both += dpp_i32<kDppRor4>(both);
        both += dpp_i32<kDppRor8>(both);
        const int e = eb + 4 * q + g;
        if (j == 0 && e < E_eff) {
          const int all = int(uint32_t(both) >> 16), pre = both & 0xffff;
          start[e] = pre;
          total[e] = all;
          count[e] = all;
          running[e] = 0;
        }
      }
    }
    if (wave * 4 * EB8 >= E_eff) first_ids[tid] = e_first;   // waves without expert rows
  } else {
    // A wave reads an expert's row of chunk counts with one instruction (lane: chunks
    // 4l .. 4l + 3), EB rows in flight at once, and folds each row with one wave sum (both
    // counts packed in one word when the plan has fewer than 2^16 routes).
    constexpr int EB = 12, CPL = ALIGN_MAX_CHUNKS / 64;   // chunks per lane
    static_assert(CPL == 4, "one int4 of chunk counts per lane");
    const bool packed = numel < 65536;
    const int cb = CPL * lane;
    for (int eb = wave * EB; eb < E_eff; eb += PLACE_WAVES * EB) {
      int4 v[EB];
#pragma unroll
      for (int j = 0; j < EB; ++j) {
        const int e = eb + j;
        v[j] = make_int4(0, 0, 0, 0);
        if (e < E_eff && cb < nch)
          v[j] = *reinterpret_cast<const int4*>(chunk_off + int64_t(e) * ALIGN_MAX_CHUNKS + cb);
      }
      if (eb == wave * EB) first_ids[tid] = e_first;
#pragma unroll
      for (int j = 0; j < EB; ++j) {
        const int x[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        int sum_l = 0, pre_s = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int xv = cb + q < nch ? x[q] : 0;   // chunks past nch were never written
          sum_l += xv;
          pre_s += cb + q < c ? xv : 0;
        }
        const uint32_t pre_l = uint32_t(pre_s);
        int all, pre;
        if (packed) {   // both sums < 2^16: no carry between the halves
          const uint32_t both = wave_sum_u((uint32_t(sum_l) << 16) | pre_l);
          all = int(both >> 16);
          pre = int(both & 0xffffu);
        } else {
          all = int(wave_sum_u(uint32_t(sum_l)));
          pre = int(wave_sum_u(pre_l));
        }
        const int e = eb + j;
        if (lane == 0 && e < E_eff) {
          start[e] = pre;
          total[e] = all;
          count[e] = all;
          running[e] = 0;
        }
      }
    }
    if (wave * EB >= E_eff) first_ids[tid] = e_first;   // waves without expert rows
  }
  for (int i = tid; i < PLACE_WAVES * E_eff; i += PLACE_THREADS) wcnt[i] = 0;
  __syncthreads();
  // 2. exclusive scan of the padded totals, by wave 0 (consecutive experts per lane)
  if (wave == 0) {
    const int per = (E_eff + 63) / 64;
    const int e0 = min(E_eff, lane * per), e1 = min(E_eff, e0 + per);
    int32_t mine = 0;
    for (int e = e0; e < e1; ++e) mine += ((total[e] + bs - 1) / bs) * bs;
    const int32_t incl = wave_incl_scan_dpp(mine);
    int32_t off = incl - mine;
    if (lane == 63) npp_lds = incl;
    for (int e = e0; e < e1; ++e) {
      const int32_t padded = ((total[e] + bs - 1) / bs) * bs;
      start[e] += off;                   // base[e] + routes of e in the chunks before c
      total[e] = off;                    // from here on: base[e]
      off += padded;
    }
  }
  __syncthreads();
  const int32_t npp = npp_lds;
  // 3. fills of this block's stripe of experts and of the tail
  for (int e = c; e < E_eff; e += nch) {
    const int32_t base = total[e];
    const int32_t cnt = (e + 1 < E_eff ? total[e + 1] : npp) - base;  // padded extent
    const int32_t n_e = count[e];                                      // unpadded count
    for (int b = tid; b < cnt / bs; b += PLACE_THREADS) expert_ids[base / bs + b] = e;
    for (int i = n_e + tid; i < cnt; i += PLACE_THREADS) sorted[base + i] = int32_t(numel);
  }
  for (int64_t i = npp + int64_t(c) * PLACE_THREADS + tid; i < max_padded;
       i += int64_t(nch) * PLACE_THREADS)
    sorted[i] = int32_t(numel);
  const int64_t max_blocks = (max_padded + bs - 1) / bs;
  for (int64_t i = npp / bs + int64_t(c) * PLACE_THREADS + tid; i < max_blocks;
       i += int64_t(nch) * PLACE_THREADS)
    expert_ids[i] = -1;
  if (c == 0 && tid == 0) npp_out[0] = npp;
  // 4. placement of the chunk's routes, PLACE_THREADS at a time in route order
  for (int64_t s0 = lo; s0 < hi; s0 += PLACE_THREADS) {
    const int64_t i = s0 + tid;
    int e = s0 == lo ? first_ids[tid] : (i < hi ? ids[i] : -1);
    if (e < 0 || e >= E_eff) e = -1;
    int rank = 0;
    if (s0 + int64_t(wave) * 64 < hi) {   // wave-uniform: waves past the chunk's end skip
#pragma unroll 16
      for (int j = 0; j < 64; ++j) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        rank += (j < lane && ej == e) ? 1 : 0;
      }
    }
    if (e >= 0) atomicAdd(&wcnt[wave * E_eff + e], 1);
    __syncthreads();
    if (e >= 0) {
      int32_t before = 0;
      for (int w = 0; w < wave; ++w) before += wcnt[w * E_eff + e];
      const int32_t pos = start[e] + running[e] + before + rank;
      sorted[pos] = int32_t(i);
      if (route_pos) route_pos[i] = pos;
    }
    __syncthreads();
    if (s0 + PLACE_THREADS < hi) {
      for (int x = tid; x < E_eff; x += PLACE_THREADS) {
        int32_t sum = 0;
        for (int w = 0; w < PLACE_WAVES; ++w) {
          sum += wcnt[w * E_eff + x];
          wcnt[w * E_eff + x] = 0;
        }
        running[x] += sum;
      }
      __syncthreads();
    }
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
// all four issued before their stores; 16-byte words when the row allows it. Padding rows
// (sentinel routes) and rows past *num_tokens_post_pad are left untouched: every consumer of a
// plan skips sentinel rows, so writing them would only add HBM traffic.
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
        if (live[j] && !pad[j] && c < row_words) xp[(r0 + j) * row_words + c] = buf[j][u];
      }
  }
}

// Token-major permute (route_pos given): one wave per token reads the token's row once and
// stores it to each of its routes' rows.
template <typename W>
__global__ __launch_bounds__(256) void moe_permute_tokens_kernel(
    W* __restrict__ xp, const W* __restrict__ hidden, const int32_t* __restrict__ route_pos, const int32_t* __restrict__ npp, int64_t max_rows,
    int64_t numel, int topk, int64_t row_words, int64_t hidden_stride_words) {
  constexpr int U = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nrows = min<int64_t>(max_rows, npp[0]);
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
  const int64_t wblocks = ceil_div(num_tokens * 64, 256);
  if (wblocks > 0x7fffffff) return fail(PIA_EINVAL, "moe_topk: too many tokens");
  const int wepl = int(ceil_div(num_experts, 64));
#define PIA_TW(DT, EPL)                                                                       \
  hipLaunchKernelGGL((moe_topk_wave_kernel<DT, EPL>), dim3(unsigned(wblocks)), dim3(256), 0, \
                     s, topk_weights, topk_ids, logits, num_tokens, num_experts, topk,       \
                     renormalize, mode, num_token_non_padded)
#define PIA_TW_DT(DT)              \
  if (wepl <= 1) PIA_TW(DT, 1);    \
  else if (wepl <= 2) PIA_TW(DT, 2); \
  else if (wepl <= 4) PIA_TW(DT, 4); \
  else if (wepl <= 8) PIA_TW(DT, 8); \
  else PIA_TW(DT, 16);
  switch (logits_dtype) {
    case PIA_DTYPE_F32: PIA_TW_DT(PIA_DTYPE_F32); break;
    case PIA_DTYPE_BF16: PIA_TW_DT(PIA_DTYPE_BF16); break;
    case PIA_DTYPE_F16: PIA_TW_DT(PIA_DTYPE_F16); break;
    default: return fail(PIA_EINVAL, "moe_topk: unknown logits dtype");
  }
#undef PIA_TW_DT
#undef PIA_TW
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
  if (nch > 0 && E_eff <= ALIGN_PLACE_MAX_E) {
    hipLaunchKernelGGL(moe_align_place<int32_t>, dim3(unsigned(nch)), dim3(PLACE_THREADS),
                       size_t(4 + PLACE_WAVES) * E_eff * sizeof(int32_t), s, sorted_token_ids, expert_ids,
                       num_tokens_post_pad, route_pos, chunk_off, topk_ids, numel, csz, nch,
                       E_eff, block_size, max_num_tokens_padded);
    return check_launch("moe_align_place");
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

extern "C" int pia_moe_topk_align(float* topk_weights, int32_t* topk_ids, const void* logits,
                                  int logits_dtype, int64_t num_tokens, int num_experts, int topk,
                                  int renormalize, int mode, int64_t num_token_non_padded,
                                  int32_t* sorted_token_ids, int32_t* expert_ids,
                                  int32_t* num_tokens_post_pad, int32_t* route_pos,
                                  int block_size, int64_t max_num_tokens_padded, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  const int64_t numel = num_tokens * int64_t(topk);
  const int E_eff = num_experts + 1;
  // chunks of tpb tokens: one top-k block and one plan chunk each
  int64_t tpb = std::max<int64_t>(16, ceil_div(num_tokens, ALIGN_MAX_CHUNKS));
  tpb = ceil_div(tpb, 16) * 16;
  const bool fused = num_tokens > 0 && topk > 0 && topk <= 64 && num_experts > 0 &&
                     num_experts <= 1024 && numel > ALIGN_SMALL_MAX && E_eff <= ALIGN_PLACE_MAX_E &&
                     tpb <= 240;  // per-chunk counts fit one byte
  if (!fused) {
    if (int rc = pia_moe_topk(topk_weights, topk_ids, logits, logits_dtype, num_tokens,
                              num_experts, topk, renormalize, mode, num_token_non_padded, stream))
      return rc;
    return pia_moe_align_block_size(sorted_token_ids, expert_ids, num_tokens_post_pad, route_pos,
                                    topk_ids, numel, num_experts, block_size,
                                    max_num_tokens_padded, workspace, workspace_bytes, stream);
  }
  if (mode != 0 && mode != 1) return fail(PIA_EINVAL, "moe_topk_align: mode must be 0 or 1");
  if (topk > num_experts) return fail(PIA_EINVAL, "moe_topk_align: topk > num_experts");
  if (block_size <= 0) return fail(PIA_EINVAL, "moe_topk_align: block_size must be > 0");
  if (numel >= 0x7fffffff || max_num_tokens_padded >= 0x7fffffff)
    return fail(PIA_EINVAL, "moe_topk_align: sizes must fit int32");
  if (!topk_weights || !topk_ids || !logits || !sorted_token_ids || !expert_ids ||
      !num_tokens_post_pad || !workspace)
    return fail(PIA_EINVAL, "moe_topk_align: null pointer");
  if (workspace_bytes < pia_moe_align_workspace_bytes(num_experts))
    return fail(PIA_EINVAL, "moe_topk_align: workspace too small");
  if (!aligned(workspace, 16)) return fail(PIA_EINVAL, "moe_topk_align: workspace must be 16-byte aligned");
  if (max_num_tokens_padded < std::min<int64_t>(numel + int64_t(E_eff) * (block_size - 1),
                                                numel * block_size))
    return fail(PIA_EINVAL, "moe_topk_align: max_num_tokens_padded below the padded worst case");
  hipStream_t s = as_stream(stream);
  const int nch = int(ceil_div(num_tokens, tpb));
  uint8_t* chunk_cnt = reinterpret_cast<uint8_t*>(workspace);
  const int epl = int(ceil_div(num_experts, 64));
  const size_t lds = size_t(E_eff) * sizeof(int32_t);
#define PIA_TH(DT, EPL)                                                                           \
  hipLaunchKernelGGL((moe_topk_hist_kernel<DT, EPL>), dim3(unsigned(nch)), dim3(1024), lds, s,    \
                     topk_weights, topk_ids, logits, num_tokens, num_experts, topk, renormalize,  \
                     mode, num_token_non_padded, int(tpb), chunk_cnt, route_pos)
#define PIA_TH_DT(DT)                      \
  if (epl <= 1) PIA_TH(DT, 1);             \
  else if (epl <= 2) PIA_TH(DT, 2);        \
  else if (epl <= 4) PIA_TH(DT, 4);        \
  else if (epl <= 8) PIA_TH(DT, 8);        \
  else PIA_TH(DT, 16);
  switch (logits_dtype) {
    case PIA_DTYPE_F32: PIA_TH_DT(PIA_DTYPE_F32); break;
    case PIA_DTYPE_BF16: PIA_TH_DT(PIA_DTYPE_BF16); break;
    case PIA_DTYPE_F16: PIA_TH_DT(PIA_DTYPE_F16); break;
    default: return fail(PIA_EINVAL, "moe_topk_align: unknown logits dtype");
  }
#undef PIA_TH_DT
#undef PIA_TH
  if (int rc = check_launch("moe_topk_hist")) return rc;
  hipLaunchKernelGGL(moe_align_place<uint8_t>, dim3(unsigned(nch)), dim3(PLACE_THREADS),
                     size_t(4 + PLACE_WAVES) * E_eff * sizeof(int32_t), s, sorted_token_ids,
                     expert_ids, num_tokens_post_pad, route_pos, chunk_cnt, topk_ids, numel,
                     tpb * topk, nch, E_eff, block_size, max_num_tokens_padded);
  return check_launch("moe_align_place");
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
    const int64_t blocks = ceil_div(numel / topk, 4);
    if (blocks == 0) return 0;
    if (blocks > 0x7fffffff) return fail(PIA_EINVAL, "moe_permute: too many rows");
    if (v16)
      hipLaunchKernelGGL(moe_permute_tokens_kernel<uint4>, dim3(unsigned(blocks)), dim3(256), 0,
                         s, (uint4*)x_perm, (const uint4*)hidden, route_pos, num_tokens_post_pad,
                         max_rows, numel, topk, row_bytes / 16, hidden_row_stride_bytes / 16);
    else
      hipLaunchKernelGGL(moe_permute_tokens_kernel<uint32_t>, dim3(unsigned(blocks)), dim3(256),
                         0, s, (uint32_t*)x_perm, (const uint32_t*)hidden, route_pos,
                         num_tokens_post_pad, max_rows, numel, topk, row_bytes / 4,
                         hidden_row_stride_bytes / 4);
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
