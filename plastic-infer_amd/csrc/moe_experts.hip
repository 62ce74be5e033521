// Grouped expert GEMM of the routed MoE FFN and the *_and_mul activations (gfx950).
//
// pia_moe_expert_gemm computes, for every route r listed in a permute plan (sorted_token_ids,
// expert_ids, num_tokens_post_pad of pia_moe_align_block_size):
//     acc = A[r / a_div] . W[e]^T        e = expert of r's plan block, W[e] is [n_rows, K]
// and stores one of two epilogues (w_r = topk_weights[r] when mul_routed_weight, else 1;
// round() is the storage dtype, round to nearest even):
//     act NONE   out[r, n] = round(acc[n] * w_r)                      n in [0, n_rows)
//     act X      g = round(acc[n] * w_r), u = round(acc[n_rows/2 + n] * w_r)
//                out[r, n] = round(X(g) * u)                          n in [0, n_rows/2)
// These are the two GEMMs of the reference's fused experts
// (src/plastic_infer/moe/fused.py:169-359; kernels src/plastic_infer/kernel/triton/fused_moe.py:
// 156-302 and src/plastic_infer/kernel/triton/decode_moe.py:6-75), with the *_and_mul of
// src/plastic_infer/kernel/triton/activation.py:63-113 fused into the first GEMM's epilogue at
// the reference's rounding points: the GEMM output is rounded to the storage dtype before the
// activation reads it, and the activation result is rounded again.
//
// Kernel: moe_gemm_splitk. A work item is (16 plan rows, one column tile): 64 W rows, which are
// 64 output columns, or 32 gate rows plus the matching 32 up rows when the activation is fused.
// The four waves of a workgroup split the K dimension in quarters; each wave multiplies its
// quarter with the operands loaded straight from global memory into registers, one 16-byte
// vector per lane, plan row / W row l%16, at K offset V*(l/16) of a 4V-wide chunk (V = 8
// elements for bf16 / f16, 4 for fp32). bf16 / f16 run one v_mfma_f32_16x16x32 per vector;
// fp32 runs four v_mfma_f32_16x16x4_f32, the j-th taking component j of the A and the W
// vector, so lane group g supplies K index 4g + j of the chunk to both operands and the four
// products cover the chunk's 16 K values once (fp32 products, fp32 sums: no rounding to a
// narrower type anywhere, the epilogue's round() is the identity).
// The four partial tiles meet in LDS and are summed in wave order (deterministic). Workgroups
// are persistent over the items and pipeline them: the next item's plan block and first K stage
// are in flight through the current item's reduction and stores. W rows are streamed once per
// plan block, which is the HBM bound at decode sizes (every expert's weights are read once per
// 16 routes it serves).
//
// Kernel: moe_gemm_cols, for K <= EG_COLS_MAX_K (a K quarter would give each wave too little
// to stream per item: 192 elements at the MoE down projection's K = 768). A work item is one
// wave's: 16 plan rows against 16 W rows (16 output columns), or 16 gate rows plus the matching
// 16 up rows when the activation is fused, over the whole K, with the same lane layout and
// products as above. The waves of a workgroup are independent: no LDS, no barrier; the sibling
// waves of a plan block re-read its A rows from L2. Items are pipelined the same way, and each
// item starts its K walk at its own stage (stage_rot below).
#include <atomic>
#include <type_traits>

#include "pia_internal.h"

namespace pia {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Storage element of a dtype code and the elements in one 16-byte vector.
template <int DT>
using eg_elem = std::conditional_t<DT == PIA_DTYPE_F32, float, uint16_t>;
template <int DT>
constexpr int eg_vec = 16 / int(sizeof(eg_elem<DT>));

constexpr int EG_ROWS = 16;       // plan rows per work item (MFMA M)
constexpr int EG_WAVES = 4;       // waves per workgroup, one K quarter each
constexpr int EG_U = 2;           // 32-wide K chunks per pipeline stage
constexpr int EG_WGS_PER_CU = 4;  // persistent workgroups per compute unit
constexpr int EG_COLS_MAX_K = 1024;  // K up to which moe_gemm_cols runs instead of the split

// 16 bytes of zeros: the load source of masked-off lanes (plan padding, K tail, W row tail).
__device__ __attribute__((aligned(16))) uint16_t g_zero8[8];

template <int DT>
__device__ __forceinline__ f32x4_t mfma_16x16x32(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (DT == PIA_DTYPE_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// One 16-byte vector of A and of W per lane: c += the 16 x 16 product over the 4 * eg_vec<DT>
// K values the wave's lanes hold.
template <int DT>
__device__ __forceinline__ f32x4_t mfma_vec(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (DT == PIA_DTYPE_F32) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0,
                                                0, 0);
  } else {
    return mfma_16x16x32<DT>(a, b, c);
  }
}

template <int DT>
__device__ __forceinline__ eg_elem<DT> to_dt(float v) {
  if constexpr (DT == PIA_DTYPE_F32) return v;
  else if constexpr (DT == PIA_DTYPE_BF16) return f32_to_bf16(v);
  else return f32_to_half(v);
}
template <int DT>
__device__ __forceinline__ float from_dt(eg_elem<DT> x) {
  if constexpr (DT == PIA_DTYPE_F32) return x;
  else if constexpr (DT == PIA_DTYPE_BF16) return bf16_to_f32(x);
  else return half_to_f32(x);
}

// act(g) of the *_and_mul family: silu g/(1+e^-g); gelu 0.5g(1+erf(g/sqrt2));
// gelu_tanh 0.5g(1+tanh(sqrt(2/pi)(g+0.044715g^3))).
template <int ACT>
__device__ __forceinline__ float act_fn(float g) {
  if constexpr (ACT == PIA_ACT_SILU) {
    return g / (1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
  } else if constexpr (ACT == PIA_ACT_GELU) {
    return 0.5f * g * (1.0f + erff(g * 0.7071067811865476f));
  } else {
    return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g)));
  }
}

// First K stage of a work item of the column and wide kernels: a function of the first route of
// its plan block and of its column tile only, so an item sums its K in the same order whichever workgroup, launch or
// weight slot computes it (the routes of an expert keep their ids and their order when the
// routed FFN is split over several calls). The weight rows of an expert are K elements apart,
// so at a common K offset the concurrent items would all read the same offset of their rows;
// starting each item at its own stage spreads those reads over the HBM channels.
__device__ __forceinline__ int stage_rot(int first_route, int t, int ns) {
  const uint32_t key = first_route > 0 ? uint32_t(first_route) : 0u;
  return ns > 0 ? int((key * 5u + uint32_t(t)) % uint32_t(ns)) : 0;
}

template <int DT, int ACT>
__global__ __launch_bounds__(EG_WAVES * 64) void moe_gemm_splitk(
    eg_elem<DT>* __restrict__ out, const eg_elem<DT>* __restrict__ a,
    const eg_elem<DT>* __restrict__ w,
    const float* __restrict__ topk_w, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ npp, int64_t max_rows,
    int64_t numel, int block_m, int a_div, int64_t lda, int num_experts, int n_rows, int K,
    int64_t ldo, int n_tiles, int mulw) {
  using E = eg_elem<DT>;
  constexpr int V = eg_vec<DT>, CH = 4 * V;  // elements per lane vector, K per chunk
  constexpr bool FUSED = ACT != PIA_ACT_NONE;
  __shared__ float red[EG_WAVES][4][4][64];  // [wave][column block][row in quad][lane]
  __shared__ int32_t blk_route[EG_ROWS];
  __shared__ float blk_w[EG_ROWS];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const int64_t rows = min(max_rows, int64_t(npp[0]));
  const int64_t items = ((rows + EG_ROWS - 1) / EG_ROWS) * n_tiles;
  const int nch = (K + CH - 1) / CH;
  const int cpw = (nch + EG_WAVES - 1) / EG_WAVES;
  const int c0 = min(nch, wv * cpw), c1 = min(nch, c0 + cpw);
  const int ns = (c1 - c0 + EG_U - 1) / EG_U;  // pipeline stages of this wave per item
  const int half = n_rows >> 1;
  const E* zero = reinterpret_cast<const E*>(g_zero8);
  // W row of column block cb relative to block 0's (the tile's rows are in four runs of 16)
  auto w_off = [&](int cb) { return (FUSED ? ((cb < 2 ? 0 : half) + (cb & 1) * 16) : cb * 16) * K; };

  // One item's operands for this lane: plan row li of its 16 (route r; A row arow), the W row
  // of column block 0 (wrow0; block cb at wrow0 + w_off[cb]), bit cb of wmask = block cb's
  // row exists, e_ok = the plan block names an expert.
  struct Item {
    const E* arow;
    const E* wrow0;
    int64_t r;
    int wmask;
    bool a_ok, e_ok;
  };
  auto make_item = [&](int64_t it, int e, int64_t r) {
    Item o;
    const int t = int(it - (it / n_tiles) * n_tiles);
    o.e_ok = e >= 0 && e < num_experts;
    o.r = r;
    o.a_ok = r >= 0 && r < numel;
    o.arow = a + (o.a_ok ? (r / a_div) * lda : 0);
    const int n0 = FUSED ? t * 32 + li : t * 64 + li;  // column block 0's row
    o.wrow0 = w + (o.e_ok ? int64_t(e) * n_rows * K : 0) + int64_t(n0) * K;
    o.wmask = 0;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bool ok = FUSED ? (t * 32 + (cb & 1) * 16 + li < half) : (n0 + cb * 16 < n_rows);
      o.wmask |= ok ? (1 << cb) : 0;
    }
    return o;
  };
  // an item's plan block: its expert (uniform) and this lane's route
  auto item_expert = [&](int64_t it) { return expert_ids[((it / n_tiles) * EG_ROWS) / block_m]; };
  auto item_route = [&](int64_t it) -> int64_t {
    const int64_t p = (it / n_tiles) * EG_ROWS + li;
    return p < rows ? int64_t(sorted[p]) : numel;
  };

  // Masked lanes read the zero vector instead, so every load is issued unconditionally and the
  // compiler can keep a whole stage in flight while the previous one is multiplied.
  auto load = [&](uint4(&va)[EG_U], uint4(&vb)[EG_U][4], const Item& o, int c) {
#pragma unroll
    for (int u = 0; u < EG_U; ++u) {
      const int cc = c + u;
      const int k = cc * CH + kg * V;
      const bool k_ok = cc < c1 && k < K;
      va[u] = *reinterpret_cast<const uint4*>((k_ok && o.a_ok) ? o.arow + k : zero);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        vb[u][cb] = *reinterpret_cast<const uint4*>(
            (k_ok && ((o.wmask >> cb) & 1)) ? o.wrow0 + w_off(cb) + k : zero);
    }
  };
  f32x4_t acc[4];
  auto mma = [&](const uint4(&va)[EG_U], const uint4(&vb)[EG_U][4]) {
#pragma unroll
    for (int u = 0; u < EG_U; ++u)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[cb] = mfma_vec<DT>(va[u], vb[u][cb], acc[cb]);
  };

  // Workgroups are persistent over the items, and items are pipelined: the next item's plan
  // block is read when an item starts, and its first K stage is issued with the item's last
  // stage, so it is in flight through the item's reduction and stores. Stage s of an item sits
  // in register set x (s even) or y (s odd); the next item's first stage always goes to x (with
  // an odd stage count, right after x's last product).
  int64_t item = blockIdx.x;
  if (item >= items) return;
  Item cur = make_item(item, item_expert(item), item_route(item));
  uint4 xa[EG_U], xb[EG_U][4], ya[EG_U], yb[EG_U][4];
  if (cur.e_ok && ns > 0) load(xa, xb, cur, c0);
  for (;;) {
    const int64_t next = item + gridDim.x;
    const bool has_next = next < items;
    int e_next = -1;
    int64_t r_next = numel;
    if (has_next) {
      e_next = item_expert(next);
      r_next = item_route(next);
    }
    float w_cur = 1.0f;  // routing weight of plan row li (read by wave 0 for the epilogue)
    if (mulw && wv == 0 && cur.a_ok) w_cur = topk_w[cur.r];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    Item nxt = cur;
    if (has_next) nxt = make_item(next, e_next, r_next);
    auto first_of_next = [&]() {
      if (has_next && nxt.e_ok) load(xa, xb, nxt, c0);
    };
    for (int st = 0; st < ns; st += 2) {
      if (st + 1 < ns && cur.e_ok) load(ya, yb, cur, c0 + (st + 1) * EG_U);
      if (cur.e_ok) mma(xa, xb);
      if (st + 1 < ns) {
        if (st + 2 < ns) {
          if (cur.e_ok) load(xa, xb, cur, c0 + (st + 2) * EG_U);
        } else {
          first_of_next();
        }
        if (cur.e_ok) mma(ya, yb);
      } else {
        first_of_next();
      }
    }

    __syncthreads();  // the previous item's epilogue has finished with red / blk_*
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wv][cb][q][lane] = acc[cb][q];
    if (wv == 0 && lane < EG_ROWS) {  // lane l < 16 of wave 0 holds plan row l's route
      blk_route[lane] = cur.a_ok ? int32_t(cur.r) : -1;
      blk_w[lane] = w_cur;
    }
    __syncthreads();

    // MFMA output layout: lane l holds column l%16 of its block, rows 4*(l/16) + q.
    const int t = int(item - (item / n_tiles) * n_tiles);
    if constexpr (!FUSED) {
      const int cb = wv;
      const int col = t * 64 + cb * 16 + li;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = kg * 4 + q;
        float v = red[0][cb][q][lane];
#pragma unroll
        for (int x = 1; x < EG_WAVES; ++x) v += red[x][cb][q][lane];
        const int32_t rr = blk_route[row];
        if (rr >= 0 && col < n_rows) out[int64_t(rr) * ldo + col] = to_dt<DT>(v * blk_w[row]);
      }
    } else {
      const int pb = wv & 1, qb = (wv >> 1) * 2;
      const int col = t * 32 + pb * 16 + li;
#pragma unroll
      for (int q = qb; q < qb + 2; ++q) {
        const int row = kg * 4 + q;
        float g = red[0][pb][q][lane], u = red[0][pb + 2][q][lane];
#pragma unroll
        for (int x = 1; x < EG_WAVES; ++x) {
          g += red[x][pb][q][lane];
          u += red[x][pb + 2][q][lane];
        }
        const int32_t rr = blk_route[row];
        if (rr >= 0 && col < half) {
          const float wr = blk_w[row];
          const float gr = from_dt<DT>(to_dt<DT>(g * wr));
          const float ur = from_dt<DT>(to_dt<DT>(u * wr));
          out[int64_t(rr) * ldo + col] = to_dt<DT>(act_fn<ACT>(gr) * ur);
        }
      }
    }
    if (!has_next) break;
    cur = nxt;
    item = next;
  }
}

template <int DT, int ACT>
__global__ __launch_bounds__(EG_WAVES * 64) void moe_gemm_cols(
    eg_elem<DT>* __restrict__ out, const eg_elem<DT>* __restrict__ a,
    const eg_elem<DT>* __restrict__ w,
    const float* __restrict__ topk_w, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ npp, int64_t max_rows,
    int64_t numel, int block_m, int a_div, int64_t lda, int num_experts, int n_rows, int K,
    int64_t ldo, int n_tiles, int mulw) {
  using E = eg_elem<DT>;
  constexpr int V = eg_vec<DT>, CH = 4 * V;  // elements per lane vector, K per chunk
  constexpr bool FUSED = ACT != PIA_ACT_NONE;
  constexpr int NB = FUSED ? 2 : 1;  // W row sets per item: the columns, or gate and up
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, kg = lane >> 4;
  const int64_t rows = min(max_rows, int64_t(npp[0]));
  const int64_t items = ((rows + EG_ROWS - 1) / EG_ROWS) * n_tiles;
  const int nch = (K + CH - 1) / CH;
  const int ns = (nch + EG_U - 1) / EG_U;  // pipeline stages per item
  const int half = n_rows >> 1;
  const int out_cols = FUSED ? half : n_rows;
  const int64_t up_off = int64_t(half) * K;  // up row n's offset from gate row n

  // One item's operands for this lane: plan row li (route r, A row arow), W row li of the
  // column tile (wrow; the up row at wrow + up_off), col_ok = that column exists, e_ok = the
  // plan block names an expert. A padding route or a missing column reads row 0 instead: its
  // products land only in outputs that are never stored.
  struct Item {
    const E* arow;
    const E* wrow;
    int r, rot;
    bool a_ok, col_ok, e_ok;
  };
  // (routes and plan rows fit int32: the host checks numel and the plan size)
  auto make_item = [&](int t, int e, int r) {
    Item o;
    const int col = t * EG_ROWS + li;
    o.e_ok = e >= 0 && e < num_experts;
    o.r = r;
    o.a_ok = r >= 0 && r < numel;
    o.col_ok = col < out_cols;
    const int arow_i = o.a_ok ? (a_div == 1 ? r : r / a_div) : 0;  // A row 0 exists: numel > 0
    o.arow = a + int64_t(arow_i) * lda;
    o.wrow = w + (o.e_ok ? int64_t(e) * n_rows * K : 0) + int64_t(o.col_ok ? col : 0) * K;
    o.rot = stage_rot(__builtin_amdgcn_readfirstlane(r), t, ns);  // lane 0: plan row 0
    return o;
  };
  auto block_expert = [&](int64_t mb) {  // wave-uniform: branches on it stay scalar
    return __builtin_amdgcn_readfirstlane(expert_ids[(mb * EG_ROWS) / block_m]);
  };
  auto block_route = [&](int64_t mb) -> int {
    const int64_t p = mb * EG_ROWS + li;
    return p < rows ? sorted[p] : int(numel);
  };

  // Stage loads; every load is issued unconditionally so the compiler can keep a whole stage
  // in flight while the previous one is multiplied. Only the last stage can reach past K: its
  // lanes there read the row's last vector and zero their A vector (a zero product).
  auto chunk = [&](const Item& o, int st) {  // first chunk of stage st of an item
    const int x = st + o.rot;
    return (x >= ns ? x - ns : x) * EG_U;
  };
  auto load = [&](uint4(&va)[EG_U], uint4(&vb)[EG_U][NB], const Item& o, int c) {
    const bool tail = (c + EG_U) * CH > K;
#pragma unroll
    for (int u = 0; u < EG_U; ++u) {
      const int k = (c + u) * CH + kg * V;
      const int kk = tail ? min(k, K - V) : k;
      va[u] = *reinterpret_cast<const uint4*>(o.arow + kk);
      if (tail && k >= K) va[u] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int j = 0; j < NB; ++j)
        vb[u][j] = *reinterpret_cast<const uint4*>(o.wrow + j * up_off + kk);
    }
  };
  f32x4_t acc[NB];
  auto mma = [&](const uint4(&va)[EG_U], const uint4(&vb)[EG_U][NB]) {
#pragma unroll
    for (int u = 0; u < EG_U; ++u)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j] = mfma_vec<DT>(va[u], vb[u][j], acc[j]);
  };

  // Stage s of an item sits in register set x (s even) or y (s odd); the next item's first
  // stage always goes to x (with an odd stage count, right after x's last product).
  int64_t item = int64_t(blockIdx.x) * EG_WAVES + wv;
  const int64_t stride = int64_t(gridDim.x) * EG_WAVES;
  if (item >= items) return;
  // item = mb * n_tiles + t, advanced without dividing
  int64_t mb = item / n_tiles;
  int t = int(item - mb * n_tiles);
  const int64_t stride_mb = stride / n_tiles;
  const int stride_t = int(stride - stride_mb * n_tiles);
  Item cur = make_item(t, block_expert(mb), block_route(mb));
  uint4 xa[EG_U], xb[EG_U][NB], ya[EG_U], yb[EG_U][NB];
  if (cur.e_ok) load(xa, xb, cur, chunk(cur, 0));
  for (;;) {
    const int64_t next = item + stride;
    const bool has_next = next < items;
    int t_next = t + stride_t;
    int64_t mb_next = mb + stride_mb;
    if (t_next >= n_tiles) {
      t_next -= n_tiles;
      ++mb_next;
    }
    int e_next = -1, r_next = int(numel);
    if (has_next) {  // the next item's plan block, read now and used with its first stage
      e_next = block_expert(mb_next);
      r_next = block_route(mb_next);
    }
    const float w_cur = (mulw && cur.a_ok) ? topk_w[cur.r] : 1.0f;  // plan row li's weight
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    Item nxt = cur;
    auto first_of_next = [&]() {  // called once, with the item's last stage
      if (!has_next) return;
      nxt = make_item(t_next, e_next, r_next);
      if (nxt.e_ok) load(xa, xb, nxt, chunk(nxt, 0));
    };
    for (int st = 0; st < ns; st += 2) {
      if (st + 1 < ns && cur.e_ok) load(ya, yb, cur, chunk(cur, st + 1));
      if (cur.e_ok) mma(xa, xb);
      if (st + 1 < ns) {
        if (st + 2 < ns) {
          if (cur.e_ok) load(xa, xb, cur, chunk(cur, st + 2));
        } else {
          first_of_next();
        }
        if (cur.e_ok) mma(ya, yb);
      } else {
        first_of_next();
      }
    }

    // MFMA output layout: lane l holds column l%16 of the tile for plan rows 4*(l/16) + q; the
    // route and weight of plan row i sit in lane i.
    const int col = t * EG_ROWS + li;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = kg * 4 + q;
      const int64_t rr = __shfl(cur.r, row, 64);
      const float wr = __shfl(w_cur, row, 64);
      if (rr < 0 || rr >= numel || col >= out_cols) continue;
      if constexpr (!FUSED) {
        out[rr * ldo + col] = to_dt<DT>(acc[0][q] * wr);
      } else {
        const float gr = from_dt<DT>(to_dt<DT>(acc[0][q] * wr));
        const float ur = from_dt<DT>(to_dt<DT>(acc[1][q] * wr));
        out[rr * ldo + col] = to_dt<DT>(act_fn<ACT>(gr) * ur);
      }
    }
    if (!has_next) break;
    cur = nxt;
    item = next;
    mb = mb_next;
    t = t_next;
  }
}

// Shared by the prefill kernel below: buffer descriptors, the per-XCD work list, the stage wait.
constexpr int TG_XCDS = 8;
// Buffer resources: word 3 of a raw (stride 0) buffer descriptor on gfx9 parts; a load whose
// offset is at or past the descriptor's byte count returns zeros (a direct load writes zeros
// to LDS), which masks plan padding, the K tail and the column tail without branches. TG_OOB
// is such an offset for every buffer here (the host keeps A and each expert's W below 2 GiB).
constexpr int TG_RSRC_WORD3 = 0x00020000;
constexpr uint32_t TG_OOB = 0x80000000u;
// Cache-policy operand of a buffer load: the nt (non-temporal) bit. The W rows of the wide
// kernel are streamed once per launch; with the hint they displace less of what the next
// launches read (its A rows, the GEMM outputs): 263-267 -> 253-256 us for the first prefill
// GEMM and 179-181 -> 171 us for the second, back to back on one box. The decode kernels load W
// into registers, where the same hint measured slower (147 -> 161 us, 82 -> 97 us).
constexpr int TG_POLICY_NT = 2;
#ifndef PIA_EG_WIDE_MIN_ROUTES
#define PIA_EG_WIDE_MIN_ROUTES 2048  // routes per call from which moe_gemm_wide is used
#endif

// Work list of moe_gemm_wide from a plan (expert_ids of the used blocks ascend):
//   seg_block[s]   first plan block of the s-th expert present, seg_block[n_seg] = used blocks
//   seg_count[0]   n_seg
//   seg_xstart[s]  items of the segments before s on s's XCD lane (segments s' = s mod 8)
//   xcd_items[x]   items on XCD lane x
// where a segment has ceil(rows / bm) row tiles times n_tiles column tiles of items.
// One 1024-thread block: a compaction over the plan blocks, then waves 0..7 scan lanes 0..7.
__global__ __launch_bounds__(1024) void moe_plan_segments(
    int32_t* __restrict__ seg_block, int32_t* __restrict__ seg_count,
    int32_t* __restrict__ seg_xstart, int32_t* __restrict__ xcd_items,
    const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ npp, int block_m,
    int64_t max_rows, int n_tiles, int bm) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t base_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nblk = int(min(max_rows, int64_t(npp[0])) / block_m);
  if (tid == 0) base_lds = 0;
  __syncthreads();
  for (int c0 = 0; c0 < nblk; c0 += 1024) {
    const int b = c0 + tid;
    const int first = (b < nblk && (b == 0 || expert_ids[b] != expert_ids[b - 1])) ? 1 : 0;
    int incl = first;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int excl = base_lds + incl - first;
    for (int w = 0; w < wave; ++w) excl += wsum[w];
    if (first) seg_block[excl] = b;
    __syncthreads();
    if (tid == 1023) base_lds = excl + first;
    __syncthreads();
  }
  const int n_seg = base_lds;
  if (tid == 0) {
    seg_block[n_seg] = nblk;
    seg_count[0] = n_seg;
  }
  __syncthreads();  // seg_block (global, this block's writes) is complete and visible
  if (wave < TG_XCDS) {
    int carry = 0;
    for (int i0 = 0; wave + TG_XCDS * i0 < n_seg; i0 += 64) {
      const int sg = wave + TG_XCDS * (i0 + lane);
      int items = 0;
      if (sg < n_seg) {
        const int64_t rows = int64_t(seg_block[sg + 1] - seg_block[sg]) * block_m;
        items = int((rows + bm - 1) / bm) * n_tiles;
      }
      int incl = items;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
      }
      if (sg < n_seg) seg_xstart[sg] = carry + incl - items;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) xcd_items[wave] = carry;
  }
}

typedef __attribute__((address_space(3))) void tg_lds_t;

// Wait until at most N of this wave's vector-memory operations are outstanding and all of its
// LDS operations are done, then meet the workgroup at a barrier. No memory fence: a fence would
// also wait for the direct loads of the steps still in flight. The waits make this wave's
// direct loads of the step complete (their LDS writes done) and its reads of the buffer about
// to be refilled returned; the barrier makes both hold for every wave. The empty asm
// statements keep the compiler from moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void tg_sync() {
  asm volatile("" ::: "memory");
  // s_waitcnt fields: vmcnt [3:0] and [15:14], expcnt [6:4] (7: no wait), lgkmcnt [11:8]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------------------------
// moe_gemm_stream: the column kernel's products for 16-bit storage without a fused activation
// and K in {512, 768, 1024} (the MoE down projection at decode sizes), with the weight rows read
// in the shape HBM delivers fastest. Loaded straight into the MFMA operand layout, each load
// instruction takes a 16-byte vector from each of 16 W rows: 64 bytes of a row, half of a
// 128-byte line. A once-read stream in that shape runs at 5.7-6.0 TB/s on this GPU, while the
// same bytes with 8, 4, 2 or 1 rows per instruction (128 bytes of a row or more) run at
// 6.7-7.2 TB/s (pia_hbm_read_rows_probe, same grid and bytes in
// flight). So each wave here reads the 16 W rows of a column tile, which are one contiguous
// 32 K-byte block, with 1 KiB-contiguous loads, stores them in its own LDS buffer (rows 16 bytes
// apart in bank order) and reads the MFMA operands from there. One wave per workgroup, as many
// as are resident at once; the (plan block, column tile) pairs, in order, are split evenly over
// them, so a wave streams one contiguous run of an expert's weights and loads the plan rows'
// A operands (whose loads have the 16-row shape) into registers once per plan block it enters.
// The next tile's W is in flight while the current tile is multiplied; K is summed in order.
// ---------------------------------------------------------------------------------------------
typedef uint32_t cs_u32x4 __attribute__((ext_vector_type(4)));
constexpr int CS_MAX_WAVES_PER_CU = 8;

template <int DT, int NI>  // NI = K / 32: 1 KiB load instructions per W tile, MFMA chunks per tile
__global__ __launch_bounds__(64) void moe_gemm_stream(
    eg_elem<DT>* __restrict__ out, const eg_elem<DT>* __restrict__ a,
    const eg_elem<DT>* __restrict__ w, const float* __restrict__ topk_w,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ expert_ids,
    const int32_t* __restrict__ npp, int64_t max_rows, int64_t numel, int block_m, int a_div,
    int64_t lda, int num_experts, int n_rows, int64_t ldo, int n_tiles, int mulw) {
  static_assert(DT != PIA_DTYPE_F32, "16-bit storage only");
  using E = eg_elem<DT>;
  constexpr int K = 32 * NI, KV = K / 8;  // K and the 16-byte vectors of one W row
  constexpr int PITCH = KV + 1;           // LDS row pitch in vectors
  extern __shared__ cs_u32x4 cs_w[];      // [16][PITCH]: the current tile's W rows
  const int lane = threadIdx.x;
  const int li = lane & 15, kg = lane >> 4;
  const int64_t rows = min(max_rows, int64_t(npp[0]));
  // the tiles of every plan block in order, (mb, t) = (g / n_tiles, g % n_tiles), split evenly
  // over the persistent waves: wave b takes [g0, g1)
  const int64_t n_g = ((rows + EG_ROWS - 1) / EG_ROWS) * n_tiles;
  const int64_t g0 = n_g * blockIdx.x / gridDim.x, g1 = n_g * (blockIdx.x + 1) / gridDim.x;

  // W tile t of expert e: rows t * 16 .. + 16, one contiguous block; lane l of load i takes
  // vector i * 64 + l of it. Buffer loads with the expert's descriptor in scalar registers and
  // the whole offset in the per-lane operand, which the range check covers: rows past n_rows
  // lie past the descriptor's byte count and read as zeros (their columns are not stored), and
  // a tile loaded only to keep every path's loads alike starts at TG_OOB (zeros, no access).
  cs_u32x4 wr[NI];  // a native vector type: an array of it stays in registers
  auto load_tile = [&](int e, int t, bool real) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<E*>(w + int64_t(e) * n_rows * K), 0, n_rows * K * 2, TG_RSRC_WORD3);
    const uint32_t off = real ? uint32_t(t * EG_ROWS * K * 2 + lane * 16) : TG_OOB;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      wr[i] = __builtin_amdgcn_raw_buffer_load_b128(wres, int(off + uint32_t(i) * 1024u), 0,
                                                    TG_POLICY_NT);
  };
  // LDS accesses of one wave complete in order; the fences keep the compiler from moving this
  // wave's stores across its reads of the previous tile, or its later reads across the stores
  auto stage_tile = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int v = i * 64 + lane, row = v / KV;
      cs_w[v + row] = wr[i];  // row * PITCH + (v - row * KV)
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  };
  // the first tile from g on whose plan block names an expert (padding blocks name none)
  auto next_valid = [&](int64_t g, int64_t& mb, int& t, int& e) __attribute__((always_inline)) {
    while (g < g1) {
      mb = g / n_tiles;
      t = int(g - mb * n_tiles);
      e = __builtin_amdgcn_readfirstlane(expert_ids[(mb * EG_ROWS) / block_m]);
      if (e >= 0 && e < num_experts) return g;
      g = (mb + 1) * n_tiles;  // the next plan block
    }
    return g1;
  };

  int64_t mb;
  int t, e;
  int64_t g = next_valid(g0, mb, t, e);
  if (g >= g1) return;
  load_tile(e, t, true);
  stage_tile();
  int64_t a_mb = -1;  // plan block whose A operands are in av
  uint4 av[NI];
  int64_t rq[4];  // route of output row 4 kg + q (the MFMA output layout), numel if none
  float wq[4];    // its top-k weight (1 without the multiply)
  while (true) {
    if (mb != a_mb) {  // route r of plan row li, its weight and A operands for every K chunk
      a_mb = mb;
      const int64_t p = mb * EG_ROWS + li;
      const int r = p < rows ? sorted[p] : int(numel);
      const bool a_ok = r >= 0 && r < numel;
      const E* arow = a + int64_t(a_ok ? (a_div == 1 ? r : r / a_div) : 0) * lda;
      const float wt = (mulw && a_ok) ? topk_w[r] : 1.0f;
#pragma unroll
      for (int c = 0; c < NI; ++c)
        av[c] = *reinterpret_cast<const uint4*>(arow + c * 32 + kg * 8);
      // the output rows' routes and weights now, while the wait for them is this branch's: a
      // load pending at the branch's end would make the products wait for every load
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = __shfl(r, kg * 4 + q, 64);
        rq[q] = rr >= 0 && rr < numel ? rr : numel;
        wq[q] = __shfl(wt, kg * 4 + q, 64);
      }
    }
    int64_t mb_n;
    int t_n, e_n;
    const int64_t g_n = next_valid(g + 1, mb_n, t_n, e_n);
    // in flight while this tile is multiplied. Issued on every path (after the range's last
    // tile as out-of-range loads): with the loads on one path only, the compiler would have to
    // wait for every outstanding load, these included, before the products.
    const bool last = g_n >= g1;
    load_tile(last ? e : e_n, last ? t : t_n, !last);
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NI; ++c) {
      const cs_u32x4 x = cs_w[li * PITCH + c * 4 + kg];
      acc = mfma_16x16x32<DT>(av[c], uint4{x.x, x.y, x.z, x.w}, acc);
    }
    // output layout: lane l holds column l % 16 for plan rows 4 (l / 16) + q
    const int col = t * EG_ROWS + li;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (rq[q] < numel && col < n_rows) out[rq[q] * ldo + col] = to_dt<DT>(acc[q] * wq[q]);
    if (g_n >= g1) break;
    stage_tile();
    g = g_n;
    mb = mb_n;
    t = t_n;
    e = e_n;
  }
}

inline size_t stream_lds_bytes(int k) { return size_t(EG_ROWS) * (k / 8 + 1) * 16; }

// ---------------------------------------------------------------------------------------------
// moe_gemm_stream_fused: the expert GEMMs of 16-bit storage at K in {1024, 2048, 3072, 4096}
// with an activation (gate rows and the matching up rows), and at K in {2048, 3072, 4096}
// without one, with the weight rows read in whole lines as in moe_gemm_stream. A work item is
// (16 plan rows, 32 W rows): 16 output columns from 16 gate rows and 16 up rows, or 32 output
// columns without an activation. The four waves of a workgroup split K in quarters, as in moe_gemm_splitk;
// a wave holds its quarter of the plan rows' A operands in registers (loaded once per plan
// block) and streams its quarter of the item's 32 W rows in sub-stages of 256 K (512 bytes of
// each row): 16 loads of 2 rows x 512 bytes, written into the wave's own LDS buffer (row pitch
// 33 vectors) and read from there as MFMA operands; the next sub-stage (the next item's first
// at an item's end) is in flight during the products. The four partial tiles are summed in
// wave order through LDS and the activation applied as in moe_gemm_splitk: each output sums
// its K in the same order as there, so the two kernels give the same bits. Workgroups are as
// many as are resident and take equal runs of the (plan block, column tile) pairs.
// ---------------------------------------------------------------------------------------------
constexpr int SF_SUB = 256;                  // K per sub-stage
constexpr int SF_PITCH = SF_SUB / 8 + 1;     // LDS row pitch in 16-byte vectors
constexpr int SF_ROWS = 2 * EG_ROWS;         // W rows per item: gate, then up
constexpr int SF_LOADS = SF_ROWS * SF_SUB * 2 / 1024;  // 1 KiB loads per sub-stage (16)

template <int DT, int ACT, int KQ>  // KQ = K / 4: the K of one wave
__global__ __launch_bounds__(EG_WAVES * 64) void moe_gemm_stream_fused(
    eg_elem<DT>* __restrict__ out, const eg_elem<DT>* __restrict__ a,
    const eg_elem<DT>* __restrict__ w, const float* __restrict__ topk_w,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ expert_ids,
    const int32_t* __restrict__ npp, int64_t max_rows, int64_t numel, int block_m, int a_div,
    int64_t lda, int num_experts, int n_rows, int64_t ldo, int n_tiles, int mulw) {
  static_assert(DT != PIA_DTYPE_F32, "16-bit storage");
  constexpr bool FUSED = ACT != PIA_ACT_NONE;
  using E = eg_elem<DT>;
  constexpr int K = 4 * KQ, NS = KQ / SF_SUB, AC = KQ / 32;  // sub-stages, A chunks per wave
  __shared__ cs_u32x4 sf_w[EG_WAVES][SF_ROWS * SF_PITCH];    // each wave's sub-stage
  __shared__ float red[EG_WAVES][2][4][64];                  // [wave][gate / up][q][lane]
  __shared__ int32_t blk_route[EG_ROWS];
  __shared__ float blk_w[EG_ROWS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kg = lane >> 4;
  const int half = n_rows >> 1;
  const int64_t rows = min(max_rows, int64_t(npp[0]));
  const int64_t n_g = ((rows + EG_ROWS - 1) / EG_ROWS) * n_tiles;
  const int64_t g0 = n_g * blockIdx.x / gridDim.x, g1 = n_g * (blockIdx.x + 1) / gridDim.x;
  cs_u32x4* buf = sf_w[wv];

  // Sub-stage j of item (e, t) for this wave: K [wv KQ + 256 j, + 256) of the item's W rows
  // (with an activation row r < 16 is gate row 16 t + r, else up row half + 16 t + r - 16;
  // without, row 32 t + r). Load i takes rows 2 i and 2 i + 1, lane l row 2 i + l / 32 at
  // vector l % 32. Rows past the last column are not loaded (offset past the descriptor:
  // zeros); real == false loads nothing at all.
  cs_u32x4 wr[SF_LOADS];
  auto load_sub = [&](int e, int t, int j, bool real) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<E*>(w + int64_t(e) * n_rows * K), 0, n_rows * K * 2, TG_RSRC_WORD3);
    const uint32_t kb = uint32_t(wv * KQ + j * SF_SUB) * 2u + uint32_t(lane & 31) * 16u;
#pragma unroll
    for (int i = 0; i < SF_LOADS; ++i) {
      const int r = 2 * i + (lane >> 5);
      int n;
      bool ok;
      if constexpr (FUSED) {
        const int col = t * EG_ROWS + (r & 15);
        n = (r < EG_ROWS ? 0 : half) + col;
        ok = col < half;
      } else {
        n = t * SF_ROWS + r;
        ok = n < n_rows;
      }
      const uint32_t off = real && ok ? uint32_t(n) * uint32_t(K) * 2u + kb : TG_OOB;
      wr[i] = __builtin_amdgcn_raw_buffer_load_b128(wres, int(off), 0, TG_POLICY_NT);
    }
  };
  // into this wave's LDS buffer, after its reads of the previous sub-stage (LDS is in order)
  auto stage_sub = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < SF_LOADS; ++i) buf[(2 * i + (lane >> 5)) * SF_PITCH + (lane & 31)] = wr[i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  };
  auto next_valid = [&](int64_t g, int64_t& mb, int& t, int& e) __attribute__((always_inline)) {
    while (g < g1) {
      mb = g / n_tiles;
      t = int(g - mb * n_tiles);
      e = __builtin_amdgcn_readfirstlane(expert_ids[(mb * EG_ROWS) / block_m]);
      if (e >= 0 && e < num_experts) return g;
      g = (mb + 1) * n_tiles;
    }
    return g1;
  };

  int64_t mb;
  int t, e;
  int64_t g = next_valid(g0, mb, t, e);
  if (g >= g1) return;
  load_sub(e, t, 0, true);
  stage_sub();
  int64_t a_mb = -1;
  uint4 av[AC];
  while (true) {
    const bool new_block = mb != a_mb;
    if (new_block) {  // this wave's K quarter of the plan rows' A operands
      a_mb = mb;
      const int64_t p = mb * EG_ROWS + li;
      const int r = p < rows ? sorted[p] : int(numel);
      const bool a_ok = r >= 0 && r < numel;
      const E* arow = a + int64_t(a_ok ? (a_div == 1 ? r : r / a_div) : 0) * lda + wv * KQ;
#pragma unroll
      for (int c = 0; c < AC; ++c)
        av[c] = *reinterpret_cast<const uint4*>(arow + c * 32 + kg * 8);
    }
    int64_t mb_n;
    int t_n, e_n;
    const int64_t g_n = next_valid(g + 1, mb_n, t_n, e_n);
    f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      // the next sub-stage's loads on every path (after the run's last item: none in memory)
      if (j + 1 < NS) load_sub(e, t, j + 1, true);
      else load_sub(g_n < g1 ? e_n : e, g_n < g1 ? t_n : t, 0, g_n < g1);
#pragma unroll
      for (int c = 0; c < SF_SUB / 32; ++c)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const cs_u32x4 x = buf[(b * EG_ROWS + li) * SF_PITCH + c * 4 + kg];
          acc[b] = mfma_16x16x32<DT>(av[j * (SF_SUB / 32) + c], uint4{x.x, x.y, x.z, x.w}, acc[b]);
        }
      stage_sub();
    }

    __syncthreads();  // the previous item's epilogue is done with red / blk_*
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wv][b][q][lane] = acc[b][q];
    if (new_block && wv == 0 && lane < EG_ROWS) {  // lane l < 16: plan row l
      const int64_t p = mb * EG_ROWS + lane;
      const int r = p < rows ? sorted[p] : int(numel);
      const bool ok = r >= 0 && r < numel;
      blk_route[lane] = ok ? r : -1;
      blk_w[lane] = (mulw && ok) ? topk_w[r] : 1.0f;
    }
    __syncthreads();
    {  // wave wv: output rows 4 kg + wv of the tile
      const int q = wv, row = kg * 4 + q;
      float gs = red[0][0][q][lane], us = red[0][1][q][lane];
#pragma unroll
      for (int x = 1; x < EG_WAVES; ++x) {
        gs += red[x][0][q][lane];
        us += red[x][1][q][lane];
      }
      const int32_t rr = blk_route[row];
      const float wr_ = blk_w[row];
      if constexpr (FUSED) {  // column 16 t + li: gate block 0, up block 1
        const int col = t * EG_ROWS + li;
        if (rr >= 0 && col < half) {
          const float gr = from_dt<DT>(to_dt<DT>(gs * wr_));
          const float ur = from_dt<DT>(to_dt<DT>(us * wr_));
          out[int64_t(rr) * ldo + col] = to_dt<DT>(act_fn<ACT>(gr) * ur);
        }
      } else {  // columns 32 t + li (block 0) and 32 t + 16 + li (block 1)
        const int col = t * SF_ROWS + li;
        if (rr >= 0 && col < n_rows) out[int64_t(rr) * ldo + col] = to_dt<DT>(gs * wr_);
        if (rr >= 0 && col + EG_ROWS < n_rows)
          out[int64_t(rr) * ldo + col + EG_ROWS] = to_dt<DT>(us * wr_);
      }
    }
    if (g_n >= g1) break;
    g = g_n;
    mb = mb_n;
    t = t_n;
    e = e_n;
  }
}

// ---------------------------------------------------------------------------------------------
// moe_gemm_wide: the many-routes-per-expert case (prefill), one work item per (expert, column
// tile of 256 W rows) that holds all of the expert's plan rows up to TW_BM (an expert with more
// gets further row tiles). Every W byte is then streamed from HBM by exactly one workgroup,
// whatever the timing of the others; the expert's A rows are shared by its column tiles, which
// are adjacent in their XCD's work list and, having identical work, run side by side through
// that XCD's L2. One 8-wave workgroup per compute unit, waves 4 (rows) x 2 (columns), each
// multiplying 16 TW_RF plan rows by 128 W rows (TW_RF x 8 fragments of v_mfma_f32_16x16x32,
// 16 TW_RF accumulators per fragment column) - two waves per SIMD, so one wave's LDS reads and
// barrier overlap the other's products.
// K advances in stages of 64: each operand row contributes one whole 128-byte line per stage,
// fetched by a 16-byte direct load (global -> LDS through a buffer descriptor, no staging
// registers) whose eight lanes 8 r .. 8 r + 7 cover row r's line. Two stage buffers: the loads
// of stage s + 1 are in flight while stage s is multiplied. An item walks its K stages from its
// own first stage (stage_rot), so the workgroups do not all read one offset of their W rows. LDS holds each operand as 16-row x
// 64 K fragments of 2 KiB: row r's 128 bytes at 128 r, its 16-byte K chunk c in slot c ^ (r % 8).
// A direct load of 8 rows lands lane l at byte 16 l, so lane l fetches chunk (l % 8) ^ (l / 8)
// of row l / 8. An MFMA operand read (ds_read_b128; lane: row l % 16, chunk 4 h + l / 16 of
// sub-step h) then touches eight different 16-byte bank groups in every eight lanes.
// ---------------------------------------------------------------------------------------------
constexpr int TW_RF = 5;                               // 16-row A fragments per wave
constexpr int TW_BM = 4 * 16 * TW_RF, TW_BN = 256, TW_BK = 64;
constexpr int TW_THREADS = 512;                        // 8 waves: 4 (rows) x 2 (columns)
constexpr int TW_AH = TW_BM / 8, TW_WH = TW_BN / 8;    // 8-row half fragments per stage: A, W
constexpr int TW_AL = TW_AH / 8, TW_WL = TW_WH / 8;    // direct loads per wave per stage: A, W
constexpr int TW_STAGE = (TW_AH + TW_WH) * 64;         // uint4 per stage buffer

template <int DT, int ACT>
__global__ __launch_bounds__(TW_THREADS, 1) void moe_gemm_wide(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ a, const uint16_t* __restrict__ w,
    const float* __restrict__ topk_w, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ seg_block,
    const int32_t* __restrict__ seg_count, const int32_t* __restrict__ seg_xstart,
    const int32_t* __restrict__ xcd_items, int64_t numel, int block_m, int a_div, int64_t lda,
    int num_experts, int n_rows, int K, int64_t ldo, int n_tiles, int mulw, uint32_t a_bytes) {
  constexpr bool FUSED = ACT != PIA_ACT_NONE;
  // two stage buffers as separate arrays (the compiler tracks the direct loads into each apart)
  __shared__ __attribute__((aligned(16))) uint4 sb0[TW_STAGE];
  __shared__ __attribute__((aligned(16))) uint4 sb1[TW_STAGE];
  __shared__ int32_t tile_route[TW_BM];
  __shared__ float tile_w[TW_BM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: wave-uniform LDS bases
  const int wm = wv >> 1, wn = wv & 1;
  const int li = lane & 15, kg = lane >> 4;
  const int lr = lane >> 3, lc = (lane & 7) ^ (lane >> 3);  // direct loads: row, K chunk
  const int n_seg = seg_count[0];
  const int half = n_rows >> 1;
  const int nks = (K + TW_BK - 1) / TW_BK;
  const __amdgpu_buffer_rsrc_t ares =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a), 0, int(a_bytes), TG_RSRC_WORD3);
  const int x = blockIdx.x % TG_XCDS;
  const int nx = (n_seg - x + TG_XCDS - 1) / TG_XCDS;
  const int total = xcd_items[x];

  for (int p = blockIdx.x / TG_XCDS; p < total; p += gridDim.x / TG_XCDS) {
    int lo = 0, hi = nx - 1;  // segment of item p: the last of this lane's starting at or before p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seg_xstart[x + TG_XCDS * mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    const int sg = x + TG_XCDS * lo;
    const int b0 = seg_block[sg], b1 = seg_block[sg + 1];
    const int64_t seg0 = int64_t(b0) * block_m, seg1 = int64_t(b1) * block_m;
    const int mts = int((seg1 - seg0 + TW_BM - 1) / TW_BM);
    const int local = p - seg_xstart[sg];
    const int t = local / mts, mt = local - t * mts;
    const int e = expert_ids[b0];
    const bool e_ok = e >= 0 && e < num_experts;  // else zero rows, as in moe_gemm_splitk
    const int64_t m0 = seg0 + int64_t(mt) * TW_BM;

    // this wave's W half fragments TW_WL wv + q: tile W rows 8 (TW_WL wv + q) + lr
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(w + (e_ok ? int64_t(e) * n_rows * K : 0)), 0,
        e_ok ? n_rows * K * 2 : 0, TG_RSRC_WORD3);
    uint32_t woff[TW_WL];
#pragma unroll
    for (int q = 0; q < TW_WL; ++q) {
      const int j = 8 * (TW_WL * wv + q) + lr;  // W row of the tile; wave column j / 128 owns it
      int n;
      bool ok;
      if constexpr (FUSED) {
        // fragments 0..3 of a wave column are gate rows, 4..7 the matching up rows
        const int jj = (j & 127) >> 4;
        const int col = t * (TW_BN / 2) + (j >> 7) * 64 + (jj & 3) * 16 + (j & 15);
        ok = col < half;
        n = (jj < 4 ? 0 : half) + col;
      } else {
        n = t * TW_BN + j;
        ok = n < n_rows;
      }
      woff[q] = ok ? uint32_t(n) * uint32_t(K) * 2u + uint32_t(lc) * 16u : TG_OOB;
    }

    __syncthreads();  // the previous item's products and epilogue are done
    bool live = false;
    if (tid < TW_BM) {
      const int64_t pr = m0 + tid;
      const int64_t rr = pr < seg1 ? int64_t(sorted[pr]) : numel;
      live = rr >= 0 && rr < numel;
      tile_route[tid] = live ? int32_t(rr) : -1;
      tile_w[tid] = (mulw && live) ? topk_w[rr] : 1.0f;
    }
    // real routes come first in an expert's plan rows, so the live rows are a prefix
    const int nlive = __builtin_amdgcn_readfirstlane(__syncthreads_count(live));
    uint32_t aoff[TW_AL];
#pragma unroll
    for (int q = 0; q < TW_AL; ++q) {
      const int32_t rr = tile_route[8 * (TW_AL * wv + q) + lr];
      aoff[q] = rr >= 0 ? uint32_t(rr / a_div) * uint32_t(lda) * 2u + uint32_t(lc) * 16u : TG_OOB;
    }
    // direct loads of stage s into buf (stages past the last read out of range: zeros, no
    // memory access), K offset in the scalar offset; the item's K stages start at rot (the
    // column tiles of an expert, which share its A rows through L2, one stage apart)
    const int rot = stage_rot(tile_route[0], t, nks);
    auto issue = [&](uint4* buf, int s) __attribute__((always_inline)) {
      const int sr = s + rot >= nks ? s + rot - nks : s + rot;
      const int k0 = (s < nks ? sr : nks) * TW_BK;
      const bool kin = k0 + 8 * lc < K;
#pragma unroll
      for (int q = 0; q < TW_AL; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (tg_lds_t*)(buf + (TW_AL * wv + q) * 64),
                                                 16, kin ? aoff[q] : TG_OOB, k0 * 2, 0, 0);
#pragma unroll
      for (int q = 0; q < TW_WL; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wres, (tg_lds_t*)(buf + (TW_AH + TW_WL * wv + q) * 64), 16,
            kin ? woff[q] : TG_OOB, k0 * 2, 0, TG_POLICY_NT);
    };
    f32x4_t acc[TW_RF][8];
#pragma unroll
    for (int i = 0; i < TW_RF; ++i)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) acc[i][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const bool wave_live = wm * 16 * TW_RF < nlive;
    // operand slots: row li of a fragment, chunk 4 h + kg of sub-step h
    const int rs0 = 8 * li + ((0 + kg) ^ (li & 7)), rs1 = 8 * li + ((4 + kg) ^ (li & 7));
    auto comp = [&](const uint4* buf) __attribute__((always_inline)) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int rs = h ? rs1 : rs0;
        uint4 fa[TW_RF], fb[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) fb[jj] = buf[(TW_AH + 2 * (wn * 8 + jj)) * 64 + rs];
#pragma unroll
        for (int i = 0; i < TW_RF; ++i) fa[i] = buf[2 * (wm * TW_RF + i) * 64 + rs];
#pragma unroll
        for (int i = 0; i < TW_RF; ++i)
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            acc[i][jj] = mfma_16x16x32<DT>(fa[i], fb[jj], acc[i][jj]);
      }
    };

    // stage s in buffer s % 2: before it is multiplied, this wave's loads of it have completed
    // (the only ones outstanding) and every wave has finished reading the other buffer, which
    // the loads of stage s + 1 then refill
    issue(sb0, 0);
    for (int s = 0; s < nks; s += 2) {
      tg_sync<0>();
      issue(sb1, s + 1);
      if (wave_live) comp(sb0);
      if (s + 1 >= nks) break;
      tg_sync<0>();
      issue(sb0, s + 2);
      if (wave_live) comp(sb1);
    }

    // epilogue: lane holds column li of each 16-column fragment, rows 4 kg + q
#pragma unroll
    for (int i = 0; i < TW_RF; ++i) {
      if (wm * 16 * TW_RF + i * 16 >= nlive) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = wm * 16 * TW_RF + i * 16 + kg * 4 + q;
        const int32_t rr = tile_route[row];
        if (rr < 0) continue;
        const float wr = tile_w[row];
        uint16_t* orow = out + int64_t(rr) * ldo;
        if constexpr (FUSED) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int col = t * (TW_BN / 2) + wn * 64 + jj * 16 + li;
            if (col < half) {
              const float gr = from_dt<DT>(to_dt<DT>(acc[i][jj][q] * wr));
              const float ur = from_dt<DT>(to_dt<DT>(acc[i][jj + 4][q] * wr));
              orow[col] = to_dt<DT>(act_fn<ACT>(gr) * ur);
            }
          }
        } else {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const int col = t * TW_BN + wn * 128 + jj * 16 + li;
            if (col < n_rows) orow[col] = to_dt<DT>(acc[i][jj][q] * wr);
          }
        }
      }
    }
  }
}

// y[r, j] = round(act(x[r, j]) * x[r, d + j]) over [rows, 2d] -> [rows, d]; one 16-byte vector
// per thread (eight bf16 / f16 or four fp32 elements) on 16-byte aligned rows, one element
// otherwise.
template <int DT, int ACT, bool VEC>
__global__ __launch_bounds__(256) void act_and_mul_kernel(eg_elem<DT>* __restrict__ y,
                                                          const eg_elem<DT>* __restrict__ x,
                                                          int64_t rows, int64_t d) {
  using E = eg_elem<DT>;
  constexpr int W = VEC ? eg_vec<DT> : 1;
  const int64_t per_row = d / W;
  const int64_t total = rows * per_row;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / per_row, j = (i - r * per_row) * W;
    const E* xr = x + r * 2 * d;
    E* yr = y + r * d;
    if constexpr (VEC) {
      const uint4 gv = *reinterpret_cast<const uint4*>(xr + j);
      const uint4 uv = *reinterpret_cast<const uint4*>(xr + d + j);
      const E* g = reinterpret_cast<const E*>(&gv);
      const E* u = reinterpret_cast<const E*>(&uv);
      uint4 ov;
      E* o = reinterpret_cast<E*>(&ov);
#pragma unroll
      for (int q = 0; q < W; ++q) o[q] = to_dt<DT>(act_fn<ACT>(from_dt<DT>(g[q])) * from_dt<DT>(u[q]));
      *reinterpret_cast<uint4*>(yr + j) = ov;
    } else {
      yr[j] = to_dt<DT>(act_fn<ACT>(from_dt<DT>(xr[j])) * from_dt<DT>(xr[d + j]));
    }
  }
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int64_t pia_moe_expert_gemm_workspace_bytes(int64_t max_num_tokens_padded,
                                                       int block_m) {
  if (max_num_tokens_padded < 0 || block_m <= 0) return 0;
  return (2 * ceil_div(max_num_tokens_padded, block_m) + 2 + TG_XCDS) * int64_t(sizeof(int32_t));
}

extern "C" int pia_moe_expert_gemm(void* out, const void* a, const void* w,
                                   const float* topk_weights, const int32_t* sorted_token_ids,
                                   const int32_t* expert_ids, const int32_t* num_tokens_post_pad,
                                   int64_t max_num_tokens_padded, int block_m, int64_t numel,
                                   int a_div, int64_t lda, int num_experts, int n_rows, int k_dim,
                                   int64_t ldo, int activation, int mul_routed_weight, int dtype,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != PIA_DTYPE_BF16 && dtype != PIA_DTYPE_F16 && dtype != PIA_DTYPE_F32)
    return fail(PIA_EUNSUPPORTED, "moe_expert_gemm: dtype must be bf16, fp16 or fp32");
  if (activation < PIA_ACT_NONE || activation > PIA_ACT_GELU_TANH)
    return fail(PIA_EINVAL, "moe_expert_gemm: unknown activation");
  const bool f32 = dtype == PIA_DTYPE_F32;
  const int vec = f32 ? 4 : 8;  // elements per 16-byte vector
  if (max_num_tokens_padded < 0 || numel < 0 || a_div <= 0 || num_experts <= 0 || n_rows <= 0 ||
      k_dim <= 0 || lda < k_dim || block_m <= 0)
    return fail(PIA_EINVAL, "moe_expert_gemm: invalid size");
  if (block_m % EG_ROWS)
    return fail(PIA_EUNSUPPORTED, "moe_expert_gemm: block_m must be a multiple of 16");
  if (k_dim % vec || lda % vec)
    return fail(PIA_EUNSUPPORTED, f32 ? "moe_expert_gemm: K and the A row stride must be "
                                        "multiples of 4 (fp32)"
                                      : "moe_expert_gemm: K and the A row stride must be "
                                        "multiples of 8");
  const bool fused = activation != PIA_ACT_NONE;
  if (fused && n_rows % 2) return fail(PIA_EINVAL, "moe_expert_gemm: gate/up rows must be even");
  const int out_cols = fused ? n_rows / 2 : n_rows;
  if (ldo < out_cols) return fail(PIA_EINVAL, "moe_expert_gemm: output row stride too small");
  if (max_num_tokens_padded == 0 || numel == 0) return 0;
  if (max_num_tokens_padded >= 0x7fffffff || numel >= 0x7fffffff)
    return fail(PIA_EINVAL, "moe_expert_gemm: sizes must fit int32");
  if (!out || !a || !w || !sorted_token_ids || !expert_ids || !num_tokens_post_pad ||
      (mul_routed_weight && !topk_weights) || !workspace)
    return fail(PIA_EINVAL, "moe_expert_gemm: null pointer");
  if (workspace_bytes < pia_moe_expert_gemm_workspace_bytes(max_num_tokens_padded, block_m))
    return fail(PIA_EINVAL, "moe_expert_gemm: workspace too small");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(workspace, 4))
    return fail(PIA_EINVAL, "moe_expert_gemm: A and W must be 16-byte aligned, workspace 4");
  hipStream_t s = as_stream(stream);
  uint16_t* o = reinterpret_cast<uint16_t*>(out);
  const uint16_t* aa = reinterpret_cast<const uint16_t*>(a);
  const uint16_t* ww = reinterpret_cast<const uint16_t*>(w);
  const int mulw = mul_routed_weight ? 1 : 0;
  const int64_t elt = f32 ? 4 : 2;
  const int cus = device_cus();
  // bytes of A the plan can reach: rows ceil(numel / a_div), the last one k_dim long
  const int64_t a_bytes = ((ceil_div(numel, a_div) - 1) * lda + k_dim) * elt;
  const int64_t w_bytes = int64_t(n_rows) * k_dim * elt;
  // the wide kernel is built for 16-bit storage; fp32 runs the decode kernels at every size
  if (!f32 && numel >= PIA_EG_WIDE_MIN_ROUTES && a_bytes < (int64_t(1) << 31) &&
      w_bytes < (int64_t(1) << 31)) {
    const int64_t max_blocks = ceil_div(max_num_tokens_padded, block_m);
    int32_t* seg_block = reinterpret_cast<int32_t*>(workspace);  // [max_blocks + 1]
    int32_t* seg_count = seg_block + max_blocks + 1;                // [1]
    int32_t* seg_xstart = seg_count + 1;                             // [max_blocks]
    int32_t* xcd_items = seg_xstart + max_blocks;                   // [8]
    const int n_tiles = int(ceil_div(out_cols, fused ? TW_BN / 2 : TW_BN));
    hipLaunchKernelGGL(moe_plan_segments, dim3(1), dim3(1024), 0, s, seg_block, seg_count,
                       seg_xstart, xcd_items, expert_ids, num_tokens_post_pad, block_m,
                       max_num_tokens_padded, n_tiles, TW_BM);
    if (int rc = check_launch("moe_plan_segments")) return rc;
    const int64_t max_seg = std::min<int64_t>(max_blocks, int64_t(num_experts) + 1);
    const int64_t ub = (ceil_div(max_num_tokens_padded, TW_BM) + max_seg) * n_tiles;
    const int64_t g = std::min<int64_t>(ub, int64_t(cus));  // one workgroup per CU
    const unsigned grid = unsigned(std::max<int64_t>(TG_XCDS, g / TG_XCDS * TG_XCDS));
#define PIA_TW(DT, ACT)                                                                        \
  hipLaunchKernelGGL((moe_gemm_wide<DT, ACT>), dim3(grid), dim3(TW_THREADS), 0, s, o, aa, ww,  \
                     topk_weights, sorted_token_ids, expert_ids, seg_block, seg_count,         \
                     seg_xstart, xcd_items, numel, block_m, a_div, lda, num_experts, n_rows,   \
                     k_dim, ldo, n_tiles, mulw, uint32_t(a_bytes))
#define PIA_TW_ACT(DT)                                                                         \
  switch (activation) {                                                                        \
    case PIA_ACT_NONE: PIA_TW(DT, PIA_ACT_NONE); break;                                        \
    case PIA_ACT_SILU: PIA_TW(DT, PIA_ACT_SILU); break;                                        \
    case PIA_ACT_GELU: PIA_TW(DT, PIA_ACT_GELU); break;                                        \
    default: PIA_TW(DT, PIA_ACT_GELU_TANH); break;                                             \
  }
    if (dtype == PIA_DTYPE_BF16) {
      PIA_TW_ACT(PIA_DTYPE_BF16)
    } else {
      PIA_TW_ACT(PIA_DTYPE_F16)
    }
#undef PIA_TW_ACT
#undef PIA_TW
    return check_launch("moe_gemm_wide");
  }
  const bool cols = k_dim <= EG_COLS_MAX_K;
  if (!f32 && k_dim % 1024 == 0 && k_dim <= 4096 && (fused || k_dim > EG_COLS_MAX_K) &&
      w_bytes < (int64_t(1) << 31)) {
    const int n_tiles = int(ceil_div(out_cols, fused ? EG_ROWS : SF_ROWS));
    const int64_t n_items = ceil_div(max_num_tokens_padded, EG_ROWS) * n_tiles;
#define PIA_SF(DT, ACT, KQ)                                                                       \
  {                                                                                               \
    auto* kern = &moe_gemm_stream_fused<DT, ACT, KQ>;                                             \
    static std::atomic<int> cached{0}; /* resident workgroups per CU, queried once */             \
    int per_cu = cached.load(std::memory_order_relaxed);                                          \
    if (per_cu == 0) {                                                                            \
      if (int rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(                        \
                                 &per_cu, reinterpret_cast<const void*>(kern), EG_WAVES * 64, 0), \
                             "moe_gemm_stream_fused: occupancy"))                                  \
        return rc;                                                                                \
      per_cu = std::max(1, per_cu);                                                               \
      cached.store(per_cu, std::memory_order_relaxed);                                            \
    }                                                                                             \
    const unsigned grid = unsigned(std::min<int64_t>(n_items, int64_t(cus) * per_cu));           \
    hipLaunchKernelGGL(kern, dim3(grid), dim3(EG_WAVES * 64), 0, s,                               \
                       reinterpret_cast<eg_elem<DT>*>(out),                                       \
                       reinterpret_cast<const eg_elem<DT>*>(a),                                   \
                       reinterpret_cast<const eg_elem<DT>*>(w), topk_weights, sorted_token_ids,    \
                       expert_ids, num_tokens_post_pad, max_num_tokens_padded, numel, block_m,     \
                       a_div, lda, num_experts, n_rows, ldo, n_tiles, mulw);                      \
  }
#define PIA_SF_K(DT, ACT)                                                                         \
  if (k_dim == 1024) PIA_SF(DT, ACT, 256)                                                         \
  else if (k_dim == 2048) PIA_SF(DT, ACT, 512)                                                    \
  else if (k_dim == 3072) PIA_SF(DT, ACT, 768)                                                    \
  else PIA_SF(DT, ACT, 1024)
#define PIA_SF_ACT(DT)                                                                            \
  switch (activation) {                                                                           \
    case PIA_ACT_NONE: PIA_SF_K(DT, PIA_ACT_NONE); break;                                         \
    case PIA_ACT_SILU: PIA_SF_K(DT, PIA_ACT_SILU); break;                                         \
    case PIA_ACT_GELU: PIA_SF_K(DT, PIA_ACT_GELU); break;                                         \
    default: PIA_SF_K(DT, PIA_ACT_GELU_TANH); break;                                              \
  }
    if (dtype == PIA_DTYPE_BF16) {
      PIA_SF_ACT(PIA_DTYPE_BF16)
    } else {
      PIA_SF_ACT(PIA_DTYPE_F16)
    }
#undef PIA_SF_ACT
#undef PIA_SF_K
#undef PIA_SF
    return check_launch("moe_gemm_stream_fused");
  }
  // (32-bit buffer offsets: the last tile of an expert starts below n_rows but reaches up to 15
  // rows past it, and offsets from TG_OOB up read zeros)
  if (!f32 && !fused && (k_dim == 512 || k_dim == 768 || k_dim == 1024) &&
      w_bytes + 16 * int64_t(k_dim) * 2 < (int64_t(1) << 31)) {
    const int n_tiles = int(ceil_div(n_rows, EG_ROWS));
    const int64_t n_items = ceil_div(max_num_tokens_padded, EG_ROWS) * n_tiles;  // tiles
    const size_t lds = stream_lds_bytes(k_dim);
    // persistent waves: as many as are resident at once (registers and LDS decide), so no wave
    // starts its items only after others have finished theirs
#define PIA_CS(DT, NI)                                                                            \
  {                                                                                               \
    auto* kern = &moe_gemm_stream<DT, NI>;                                                        \
    static std::atomic<int> cached{0}; /* resident workgroups per CU, queried once */             \
    int per_cu = cached.load(std::memory_order_relaxed);                                          \
    if (per_cu == 0) {                                                                            \
      if (int rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(                        \
                                 &per_cu, reinterpret_cast<const void*>(kern), 64, lds),          \
                             "moe_gemm_stream: occupancy"))                                        \
        return rc;                                                                                \
      per_cu = std::max(1, std::min(per_cu, CS_MAX_WAVES_PER_CU));                                \
      cached.store(per_cu, std::memory_order_relaxed);                                            \
    }                                                                                             \
    const unsigned grid = unsigned(std::min<int64_t>(n_items, int64_t(cus) * per_cu));           \
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64), lds, s,                                        \
                       reinterpret_cast<eg_elem<DT>*>(out),                                       \
                       reinterpret_cast<const eg_elem<DT>*>(a),                                   \
                       reinterpret_cast<const eg_elem<DT>*>(w), topk_weights, sorted_token_ids,    \
                       expert_ids, num_tokens_post_pad, max_num_tokens_padded, numel, block_m,     \
                       a_div, lda, num_experts, n_rows, ldo, n_tiles, mulw);                      \
  }
#define PIA_CS_K(DT)                                                                              \
  if (k_dim == 512) PIA_CS(DT, 16)                                                                \
  else if (k_dim == 768) PIA_CS(DT, 24)                                                           \
  else PIA_CS(DT, 32)
    if (dtype == PIA_DTYPE_BF16) {
      PIA_CS_K(PIA_DTYPE_BF16)
    } else {
      PIA_CS_K(PIA_DTYPE_F16)
    }
#undef PIA_CS_K
#undef PIA_CS
    return check_launch("moe_gemm_stream");
  }
  const int n_tiles = int(ceil_div(out_cols, cols ? EG_ROWS : (fused ? 32 : 64)));
  const int64_t n_items = ceil_div(max_num_tokens_padded, EG_ROWS) * n_tiles;
  const int64_t ub = cols ? ceil_div(n_items, EG_WAVES) : n_items;
  const unsigned grid = unsigned(std::min<int64_t>(ub, int64_t(cus) * EG_WGS_PER_CU));
#define PIA_EG_K(KERN, DT, ACT)                                                                   \
  hipLaunchKernelGGL((KERN<DT, ACT>), dim3(grid), dim3(EG_WAVES * 64), 0, s,                       \
                     reinterpret_cast<eg_elem<DT>*>(out), reinterpret_cast<const eg_elem<DT>*>(a), \
                     reinterpret_cast<const eg_elem<DT>*>(w),                                     \
                     topk_weights, sorted_token_ids, expert_ids, num_tokens_post_pad,             \
                     max_num_tokens_padded, numel, block_m, a_div, lda, num_experts, n_rows,       \
                     k_dim, ldo, n_tiles, mulw)
#define PIA_EG(DT, ACT)                                                                           \
  if (cols) PIA_EG_K(moe_gemm_cols, DT, ACT); else PIA_EG_K(moe_gemm_splitk, DT, ACT)
#define PIA_EG_ACT(DT)                                                                            \
  switch (activation) {                                                                           \
    case PIA_ACT_NONE: PIA_EG(DT, PIA_ACT_NONE); break;                                           \
    case PIA_ACT_SILU: PIA_EG(DT, PIA_ACT_SILU); break;                                           \
    case PIA_ACT_GELU: PIA_EG(DT, PIA_ACT_GELU); break;                                           \
    default: PIA_EG(DT, PIA_ACT_GELU_TANH); break;                                                \
  }
  if (dtype == PIA_DTYPE_BF16) {
    PIA_EG_ACT(PIA_DTYPE_BF16)
  } else if (dtype == PIA_DTYPE_F16) {
    PIA_EG_ACT(PIA_DTYPE_F16)
  } else {
    PIA_EG_ACT(PIA_DTYPE_F32)
  }
#undef PIA_EG_ACT
#undef PIA_EG
#undef PIA_EG_K
  return check_launch(cols ? "moe_gemm_cols" : "moe_gemm_splitk");
}

extern "C" int pia_act_and_mul(void* out, const void* x, int64_t rows, int64_t d, int activation,
                               int dtype, void* stream) {
  if (dtype != PIA_DTYPE_BF16 && dtype != PIA_DTYPE_F16 && dtype != PIA_DTYPE_F32)
    return fail(PIA_EUNSUPPORTED, "act_and_mul: dtype must be bf16, fp16 or fp32");
  if (activation < PIA_ACT_SILU || activation > PIA_ACT_GELU_TANH)
    return fail(PIA_EINVAL, "act_and_mul: unknown activation");
  if (rows < 0 || d < 0) return fail(PIA_EINVAL, "act_and_mul: invalid size");
  if (rows == 0 || d == 0) return 0;
  if (!out || !x) return fail(PIA_EINVAL, "act_and_mul: null pointer");
  const int per_vec = dtype == PIA_DTYPE_F32 ? 4 : 8;
  const bool vec = d % per_vec == 0 && aligned(out, 16) && aligned(x, 16);
  const int64_t work = rows * (vec ? d / per_vec : d);
  const unsigned grid =
      unsigned(std::min<int64_t>(ceil_div(work, 256), int64_t(device_cus()) * 16));
  hipStream_t s = as_stream(stream);
#define PIA_AM(DT, ACT)                                                                      \
  if (vec)                                                                                   \
    hipLaunchKernelGGL((act_and_mul_kernel<DT, ACT, true>), dim3(grid), dim3(256), 0, s,     \
                       reinterpret_cast<eg_elem<DT>*>(out),                                  \
                       reinterpret_cast<const eg_elem<DT>*>(x), rows, d);                    \
  else                                                                                       \
    hipLaunchKernelGGL((act_and_mul_kernel<DT, ACT, false>), dim3(grid), dim3(256), 0, s,    \
                       reinterpret_cast<eg_elem<DT>*>(out),                                  \
                       reinterpret_cast<const eg_elem<DT>*>(x), rows, d)
#define PIA_AM_ACT(DT)                                   \
  switch (activation) {                                  \
    case PIA_ACT_SILU: PIA_AM(DT, PIA_ACT_SILU); break;  \
    case PIA_ACT_GELU: PIA_AM(DT, PIA_ACT_GELU); break;  \
    default: PIA_AM(DT, PIA_ACT_GELU_TANH); break;       \
  }
  if (dtype == PIA_DTYPE_BF16) {
    PIA_AM_ACT(PIA_DTYPE_BF16)
  } else if (dtype == PIA_DTYPE_F16) {
    PIA_AM_ACT(PIA_DTYPE_F16)
  } else {
    PIA_AM_ACT(PIA_DTYPE_F32)
  }
#undef PIA_AM_ACT
#undef PIA_AM
  return check_launch("act_and_mul");
}
