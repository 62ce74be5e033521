// Paged attention of many query rows per sequence (prefill, chunked prefill) on the matrix
// cores, gfx950: bf16, head_dim 128, page size 16, Hq / Hkv = G in {1, 2, 4, 8}.
//
// Work item (one 256-thread workgroup): one kv head and 64 / G consecutive query positions of
// one sequence, i.e. 64 (position, q head) rows that share the kv head's keys: row r is
// position s0 + r / G, head h * G + r % G. Wave w owns rows 16 w .. 16 w + 15. The keys are
// walked in 64-token tiles (four pages): K and V come from the pool into registers one tile
// ahead, then into LDS (double buffered, one barrier per tile):
//   K as [token][d] (the pool stores [d][token]; the transpose happens in the LDS writes),
//   V as [d][token] (its pool layout).
// Per tile each wave runs
//   S^T = K . Q^T   16 v_mfma_f32_16x16x32_bf16: A = K rows from LDS, B = the wave's q rows
//                   (registers, loaded once). Lane l then holds the scores of row l % 16 for
//                   tokens 16 m + 4 (l / 16) + j (m < 4, j < 4) of the tile.
//   online softmax  per row in fp32, base 2 with the scale folded in; a row's 64 scores sit
//                   in four lanes (l, l ^ 16, l ^ 32, l ^ 48), reduced by two shuffles.
//   O += P . V      16 MFMAs: the probabilities are the A operand straight from the score
//                   registers (bf16): k slot 8 (l / 16) + j of 32-token chunk c is token
//                   32 c + 4 (l / 16) + j for j < 4 and 32 c + 16 + 4 (l / 16) + j - 4 after,
//                   and the B operand reads V at the same tokens (two 8-byte LDS reads), so
//                   both sides of every MFMA sum the same 32 tokens. O (16 rows x 128) stays in
//                   8 accumulator blocks; lane l holds rows 4 (l / 16) + j, column l % 16.
// Keys a row may not see (past its causal limit or the sequence's length, on a page whose
// block-table id is outside the pool) score -inf; their V words are zeros from the loads.
//
// Work list: sequence-major, then kv head, then position tile (the last tiles of a sequence,
// which see the most keys when causal, first). A 1-D grid is dispatched round-robin over the 8
// XCDs (workgroup i runs on XCD i % 8); the list is cut into 8 contiguous runs and XCD x takes
// run x in order, so the ~64 workgroups resident on one XCD are the position tiles of one
// (sequence, kv head) and read its K / V through that XCD's L2 once between them.
#include <algorithm>

#include "pia_internal.h"

namespace pia {
namespace {

typedef __bf16 pf_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float pf_f32x4_t __attribute__((ext_vector_type(4)));

constexpr int PF_D = 128, PF_P = 16;
constexpr int PF_ROWS = 64;           // (position, head) rows per work item: 4 waves x 16
constexpr int PF_KT = 64;             // keys per tile: four pages
constexpr int PF_KS = PF_D + 8;       // K tile row stride in LDS (elements), [token][d]
constexpr int PF_VS = PF_KT + 8;      // V tile row stride in LDS (elements), [d][token]
constexpr int PF_MAX_SEQS = 1024;     // sequences per launch (tile prefix in LDS)
constexpr float kNegBigPf = -1.0e30f;

__device__ __forceinline__ pf_f32x4_t pf_mfma(const uint4& a, const uint4& b, pf_f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8_t, a),
                                                 __builtin_bit_cast(pf_bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pf_pack(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t p = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, p);
}

template <int G>
__global__ __launch_bounds__(256, 2) void paged_prefill_mfma(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ kpool, const uint16_t* __restrict__ vpool,
    const int32_t* __restrict__ bt, int64_t bt_stride, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ offsets, int B, int Hkv,
    int64_t num_pages, float scale_log2) {
  constexpr int D = PF_D, P = PF_P, TILE = D * P;
  constexpr int PPT = PF_ROWS / G;  // query positions per work item
  constexpr int XCDS = 8;
  __shared__ __align__(16) uint16_t ks[2][PF_KT * PF_KS];
  __shared__ __align__(16) uint16_t vs[2][PF_D * PF_VS];
  __shared__ int tile_pref[PF_MAX_SEQS + 1];
  __shared__ int wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Hq = Hkv * G;
  const int64_t q_row = int64_t(Hq) * D;  // elements between query positions

  // work items per sequence (ceil(rows / PPT)) and their prefix, scanned 256 sequences at a time
  if (tid == 0) tile_pref[0] = 0;
  int carry = 0;
  for (int c0 = 0; c0 < B; c0 += 256) {
    const int i = c0 + tid;
    const int n = i < B ? (cu_q ? cu_q[i + 1] - cu_q[i] : 1) : 0;
    const int t = n > 0 ? (n + PPT - 1) / PPT : 0;
    int incl = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = carry;
    for (int x = 0; x < wave; ++x) base += wsum[x];
    if (i < B) tile_pref[i + 1] = base + incl;
    carry += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
  }
  // this workgroup's item: XCD x = blockIdx % 8 runs items [x * run, (x + 1) * run) in order
  const int64_t items = int64_t(carry) * Hkv;
  const int64_t run = (items + XCDS - 1) / XCDS;
  const int64_t k = blockIdx.x / XCDS;
  const int64_t item = (blockIdx.x % XCDS) * run + k;
  if (k >= run || item >= items) return;
  int lo = 0, hi = B - 1;  // the sequence holding the item: Hkv * tile_pref[b] <= item
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(tile_pref[mid]) * Hkv <= item) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int nt_b = tile_pref[b + 1] - tile_pref[b];
  const int rem = int(item - int64_t(tile_pref[b]) * Hkv);
  const int h = rem / nt_b;
  const int s0 = (nt_b - 1 - rem % nt_b) * PPT;
  const int64_t row0 = cu_q ? int64_t(cu_q[b]) : int64_t(b);
  const int n_b = cu_q ? cu_q[b + 1] - cu_q[b] : 1;
  int kv_len = kv_lens[b];
  kv_len = kv_len < 0 ? 0 : (int64_t(kv_len) > bt_stride * P ? int(bt_stride * P) : kv_len);
  const int off = offsets ? offsets[b] : 0;
  const int s_last = min(s0 + PPT, n_b) - 1;
  int kmax = kv_len;
  if (offsets) kmax = max(0, min(kmax, off + s_last + 1));
  const int npages = (kv_len + P - 1) / P;
  const int nkt = (kmax + PF_KT - 1) / PF_KT;
  const int32_t* btb = bt + int64_t(b) * bt_stride;

  // this lane's score row (16 wave + l % 16) and its q operand: d = 32 kc + 8 (l / 16) .. + 7
  const int g4 = lane >> 4, n16 = lane & 15;
  const int r_s = 16 * wave + n16;
  const int s_r = s0 + r_s / G;
  const bool row_ok = s_r < n_b;
  const int lim_r = !row_ok ? 0 : (offsets ? min(kv_len, off + s_r + 1) : kv_len);
  uint4 qreg[4];
  {
    const uint16_t* qp = q + (row0 + (row_ok ? s_r : 0)) * q_row + int64_t(h * G + r_s % G) * D;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
      qreg[kc] = row_ok ? *reinterpret_cast<const uint4*>(qp + 32 * kc + 8 * g4)
                        : make_uint4(0u, 0u, 0u, 0u);
  }

  // tile loads: thread t moves piece t of each of the tile's four (page, head) K and V tiles:
  // row d = t / 2, tokens 8 (t % 2) .. + 7 of page i
  const int ld_d = tid >> 1, ld_half = tid & 1;
  uint4 kr[4], vr[4];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pi = 4 * kt + i;
      const int id = pi < npages ? btb[pi] : -1;
      const bool ok = id >= 0 && int64_t(id) < num_pages;
      const int64_t base = (int64_t(ok ? id : 0) * Hkv + h) * TILE + ld_d * P + ld_half * 8;
      kr[i] = ok ? *reinterpret_cast<const uint4*>(kpool + base) : make_uint4(0u, 0u, 0u, 0u);
      vr[i] = ok ? *reinterpret_cast<const uint4*>(vpool + base) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t0 = i * P + ld_half * 8;
      const uint16_t* ke = reinterpret_cast<const uint16_t*>(&kr[i]);
#pragma unroll
      for (int x = 0; x < 8; ++x) ks[buf][(t0 + x) * PF_KS + ld_d] = ke[x];
      *reinterpret_cast<uint4*>(&vs[buf][ld_d * PF_VS + t0]) = vr[i];
    }
  };

  float m = kNegBigPf, l = 0.f;
  pf_f32x4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = pf_f32x4_t{0.f, 0.f, 0.f, 0.f};
  // page ids of the tile, for the score mask: bit i set when page i holds keys
  auto page_mask = [&](int kt) {
    int mk = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pi = 4 * kt + i;
      const int id = pi < npages ? btb[pi] : -1;
      mk |= (id >= 0 && int64_t(id) < num_pages) ? (1 << i) : 0;
    }
    return mk;
  };

  if (nkt > 0) fetch(0);
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    stage(buf);
    __syncthreads();
    const int pmask = page_mask(kt);
    if (kt + 1 < nkt) fetch(kt + 1);

    // S^T for the wave's 16 rows: 4 token blocks (one per page) x 4 d chunks
    pf_f32x4_t sc[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      sc[mb] = pf_f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const uint4 a =
            *reinterpret_cast<const uint4*>(&ks[buf][(16 * mb + n16) * PF_KS + 32 * kc + 8 * g4]);
        sc[mb] = pf_mfma(a, qreg[kc], sc[mb]);
      }
    }
    // mask, scale, online softmax of row r_s (tokens 64 kt + 16 mb + 4 g4 + j)
    float x[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = kt * PF_KT + 16 * mb + 4 * g4 + j;
        const bool ok = t < lim_r && ((pmask >> mb) & 1);
        x[mb][j] = ok ? sc[mb][j] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[mb][j]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    float ps = 0.f;
    uint4 pk[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float p[2][4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[hh][j] = __builtin_amdgcn_exp2f(x[2 * c + hh][j] - mnew);
          ps += p[hh][j];
        }
      pk[c] = make_uint4(pf_pack(p[0][0], p[0][1]), pf_pack(p[0][2], p[0][3]),
                         pf_pack(p[1][0], p[1][1]), pf_pack(p[1][2], p[1][3]));
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mnew;
    // rescale O: lane l's accumulator rows are 4 g4 + j; their alpha sits in lane 4 g4 + j
    float aj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) aj[j] = __shfl(alpha, 4 * g4 + j, 64);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[nb][j] *= aj[j];
    // O += P . V over the tile's two 32-token chunks
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint16_t* vrow = &vs[buf][(16 * nb + n16) * PF_VS + 4 * g4];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint2 v0 = *reinterpret_cast<const uint2*>(vrow + 32 * c);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 32 * c + 16);
        acc[nb] = pf_mfma(pk[c], make_uint4(v0.x, v0.y, v1.x, v1.y), acc[nb]);
      }
    }
  }

  // out = O / l for rows 4 g4 + j of the wave (their l sits in lane 4 g4 + j)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lj = __shfl(l, 4 * g4 + j, 64);
    const int r = 16 * wave + 4 * g4 + j;
    const int s = s0 + r / G;
    if (s >= n_b) continue;
    uint16_t* o = out + (row0 + s) * q_row + int64_t(h * G + r % G) * D + n16;
    const float inv = lj > 0.f ? 1.f / lj : 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[16 * nb] = f32_to_bf16(acc[nb][j] * inv);
  }
}

}  // namespace

bool prefill_mfma_path(int dtype, int Hq, int Hkv, int D, int P, int num_seqs,
                       int64_t total_q_rows, const int32_t* cu_q) {
  const int G = Hq / Hkv;
  return dtype == PIA_DTYPE_BF16 && D == PF_D && P == PF_P &&
         (G == 1 || G == 2 || G == 4 || G == 8) && cu_q != nullptr && num_seqs <= PF_MAX_SEQS &&
         total_q_rows >= 4 * int64_t(num_seqs);
}

int launch_prefill_mfma(void* out, const void* q, const void* k_pages, const void* v_pages,
                        const int32_t* bt, int64_t bt_stride, const int32_t* kv_lens,
                        const int32_t* cu_q, const int32_t* offsets, int num_seqs,
                        int64_t total_q_rows, int Hq, int Hkv, int64_t num_pages,
                        float scale_log2, hipStream_t s) {
  const int G = Hq / Hkv;
  const int ppt = PF_ROWS / G;
  // work items: at most ceil(total rows / ppt) + one partial item per sequence
  const int64_t items = (ceil_div(total_q_rows, ppt) + num_seqs) * Hkv;
  const int64_t blocks = ceil_div(items, 8) * 8;
  if (blocks > 0x7fffffff)
    return fail(PIA_EINVAL, "paged_attention: too many query rows for the prefill kernel");
  const dim3 grid{unsigned(blocks), 1u, 1u};
#define PIA_PF(GG)                                                                             \
  hipLaunchKernelGGL((paged_prefill_mfma<GG>), grid, dim3(256), 0, s,                          \
                     reinterpret_cast<uint16_t*>(out), reinterpret_cast<const uint16_t*>(q),   \
                     reinterpret_cast<const uint16_t*>(k_pages),                               \
                     reinterpret_cast<const uint16_t*>(v_pages), bt, bt_stride, kv_lens, cu_q, \
                     offsets, num_seqs, Hkv, num_pages, scale_log2)
  switch (G) {
    case 1: PIA_PF(1); break;
    case 2: PIA_PF(2); break;
    case 4: PIA_PF(4); break;
    default: PIA_PF(8); break;
  }
#undef PIA_PF
  return check_launch("paged_prefill_mfma");
}

}  // namespace pia
